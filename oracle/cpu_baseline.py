"""CPU baselines: the reference's own PyTorch attention paths, restated (test /
benchmark infrastructure only; imported by bench.py's cpu_baseline legs).

* ``reference_fwd_bwd``: the training-step attention of
  ``kempnerforge/model/attention.py:160-175,228-234`` as the reference runs it:
  ``apply_rope`` in the input dtype (``kempnerforge/model/position.py:43-71``),
  ``repeat_interleave`` GQA expansion, ``F.scaled_dot_product_attention(...,
  is_causal=True)`` and autograd for the backward.
* ``reference_decode``: one KV-cache decode step per sequence as
  ``scripts/generate.py`` drives it through ``kempnerforge/model/generate.py:
  114-124``: RoPE at the cached length, ``KVCache.update``'s slice assignment
  (``kempnerforge/model/attention.py:54-70``), the whole-cache GQA expansion
  (``:173-175``) and SDPA with ``is_causal=False`` (``:229-231``).
* ``reference_capture``: ``_attention_with_weights``
  (``kempnerforge/model/attention.py:238-280``): ``matmul -> scale ->
  masked_fill(triu) -> softmax -> matmul`` in the input dtype, after RoPE and
  the GQA expansion.

All are evaluated by PyTorch's CPU kernels in the dtype of the GPU run.
"""

from __future__ import annotations

import os
import time

import torch
import torch.nn.functional as F

from oracle.attention_ref import apply_rope, rope_tables


def cpu_threads() -> int:
    """Use the host's cores, capped by OMP_NUM_THREADS when the environment
    sets it (a GPU box's CPU share); returns the thread count in use."""
    n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    torch.set_num_threads(n)
    return torch.get_num_threads()


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def reference_fwd_bwd(q, k, v, cos, sin, dout):
    """Forward + backward of the reference path on BSHD inputs; returns
    ``(out BSHD, dq, dk, dv)``."""
    q = q.detach().requires_grad_(True)
    k = k.detach().requires_grad_(True)
    v = v.detach().requires_grad_(True)
    n_rep = q.shape[2] // k.shape[2]
    qr = apply_rope(q.transpose(1, 2), cos, sin)
    kr = apply_rope(k.transpose(1, 2), cos, sin)
    vt = v.transpose(1, 2)
    if n_rep > 1:
        kr = kr.repeat_interleave(n_rep, dim=1)
        vt = vt.repeat_interleave(n_rep, dim=1)
    out = F.scaled_dot_product_attention(qr, kr, vt, is_causal=True)
    out = out.transpose(1, 2).contiguous()
    dq, dk, dv = torch.autograd.grad(out, (q, k, v), dout)
    return out.detach(), dq, dk, dv


def reference_decode(q_new, k_new, v_new, k_cache, v_cache, pos: int, cos, sin):
    """One decode step of one sequence (B = 1) at position ``pos``: updates the
    caches ``[1, Hkv, Smax, D]`` in place and returns out ``[1, 1, Hq, D]``."""
    n_rep = q_new.shape[2] // k_new.shape[2]
    c, s = cos[pos:pos + 1], sin[pos:pos + 1]
    q = apply_rope(q_new.transpose(1, 2), c, s)
    k = apply_rope(k_new.transpose(1, 2), c, s)
    k_cache[:, :, pos:pos + 1] = k
    v_cache[:, :, pos:pos + 1] = v_new.transpose(1, 2)
    kk, vv = k_cache[:, :, :pos + 1], v_cache[:, :, :pos + 1]
    if n_rep > 1:
        kk = kk.repeat_interleave(n_rep, dim=1)
        vv = vv.repeat_interleave(n_rep, dim=1)
    return F.scaled_dot_product_attention(q, kk, vv, is_causal=False).transpose(1, 2)


def reference_capture(q, k, v, cos, sin):
    """Causal manual attention with materialised probabilities on BSHD inputs;
    returns ``(out BSHD, P [B, Hq, S, S])``."""
    n_rep = q.shape[2] // k.shape[2]
    qr = apply_rope(q.transpose(1, 2), cos, sin)
    kr = apply_rope(k.transpose(1, 2), cos, sin)
    vt = v.transpose(1, 2)
    if n_rep > 1:
        kr = kr.repeat_interleave(n_rep, dim=1)
        vt = vt.repeat_interleave(n_rep, dim=1)
    S = qr.shape[2]
    attn = torch.matmul(qr, kr.transpose(-2, -1)) * q.shape[-1] ** -0.5
    mask = torch.ones(S, S, dtype=torch.bool).triu(diagonal=1)
    attn = F.softmax(attn.masked_fill(mask, float("-inf")), dim=-1)
    return torch.matmul(attn, vt).transpose(1, 2), attn


def _median_time(fn, min_seconds: float, max_reps: int):
    """One warm-up, then repetitions until ``min_seconds`` have elapsed (at
    least 3, at most ``max_reps``); returns ``(median seconds, reps)``."""
    fn()
    times = []
    start = time.perf_counter()
    while len(times) < max_reps and (len(times) < 3 or time.perf_counter() - start < min_seconds):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def _with_dtype_fallback(make, run, dtype):
    """Run ``run(*make(dtype))`` once; on a CPU kernel that rejects ``dtype``
    fall back to float32.  Returns ``(args, dtype used)``."""
    try:
        args = make(dtype)
        run(*args)
        return args, dtype
    except RuntimeError:
        args = make(torch.float32)
        run(*args)
        return args, torch.float32


def time_fwd_bwd(B, S, Hq, Hkv, D, theta, dtype, *, min_seconds=10.0, max_reps=20):
    """Time :func:`reference_fwd_bwd` on seeded inputs.  Returns
    ``(median_seconds, reps, dtype_used)``."""
    cos, sin = rope_tables(D, S, theta)

    def make(dt):
        g = torch.Generator().manual_seed(0)
        return tuple(torch.randn(*shape, generator=g).to(dt)
                     for shape in ((B, S, Hq, D), (B, S, Hkv, D), (B, S, Hkv, D), (B, S, Hq, D)))

    def run(q, k, v, do):
        return reference_fwd_bwd(q, k, v, cos, sin, do)

    args, used = _with_dtype_fallback(make, run, dtype)
    secs, reps = _median_time(lambda: run(*args), min_seconds, max_reps)
    return secs, reps, used


def time_decode(lens, Hq, Hkv, D, theta, dtype, *, min_seconds=10.0, max_reps=20):
    """Time one decode step of the sequences with cache lengths ``lens``, each
    run alone through :func:`reference_decode` (the reference's generate loop
    decodes the batch with one SDPA call over the expanded cache; per-sequence
    calls are what a ragged batch needs and move the same bytes).  Returns
    ``(median seconds for all of lens, reps, dtype_used)``."""
    Smax = max(lens) + 1
    cos, sin = rope_tables(D, Smax, theta)

    def make(dt):
        g = torch.Generator().manual_seed(4)
        caches = [(torch.randn(1, Hkv, L + 1, D, generator=g).to(dt),
                   torch.randn(1, Hkv, L + 1, D, generator=g).to(dt)) for L in lens]
        new = [tuple(torch.randn(1, 1, h, D, generator=g).to(dt) for h in (Hq, Hkv, Hkv))
               for _ in lens]
        return caches, new

    def run(caches, new):
        for L, (kc, vc), (q, k, v) in zip(lens, caches, new):
            reference_decode(q, k, v, kc, vc, L, cos, sin)

    args, used = _with_dtype_fallback(make, run, dtype)
    secs, reps = _median_time(lambda: run(*args), min_seconds, max_reps)
    return secs, reps, used


def time_capture(S, Hq, Hkv, D, theta, dtype, *, min_seconds=10.0, max_reps=20):
    """Time :func:`reference_capture` (B = 1).  Returns ``(median seconds,
    reps, dtype_used)``."""
    cos, sin = rope_tables(D, S, theta)

    def make(dt):
        g = torch.Generator().manual_seed(0)
        return tuple(torch.randn(1, S, h, D, generator=g).to(dt) for h in (Hq, Hkv, Hkv))

    def run(q, k, v):
        return reference_capture(q, k, v, cos, sin)

    args, used = _with_dtype_fallback(make, run, dtype)
    secs, reps = _median_time(lambda: run(*args), min_seconds, max_reps)
    return secs, reps, used
