"""CPU baseline: the reference's own PyTorch attention path, restated (test /
benchmark infrastructure only; imported by bench.py's cpu_baseline leg).

``reference_fwd_bwd`` is the training-step attention of
``kempnerforge/model/attention.py:160-175,228-234`` as the reference runs it:
``apply_rope`` in the input dtype (``kempnerforge/model/position.py:43-71``),
``repeat_interleave`` GQA expansion, ``F.scaled_dot_product_attention(...,
is_causal=True)`` and autograd for the backward — evaluated by PyTorch's CPU
kernels in the same dtype as the GPU run.
"""

from __future__ import annotations

import time

import torch
import torch.nn.functional as F

from oracle.attention_ref import apply_rope


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


def time_fwd_bwd(B, S, Hq, Hkv, D, theta, dtype, *, min_seconds=10.0, max_reps=20):
    """Time :func:`reference_fwd_bwd` on seeded inputs: one warm-up, then
    repetitions until ``min_seconds`` have elapsed (at least 3, at most
    ``max_reps``).  Returns ``(median_seconds, reps, dtype_used)``; falls back
    to float32 if the CPU build rejects ``dtype``."""
    from oracle.attention_ref import rope_tables

    def make(dt):
        g = torch.Generator().manual_seed(0)
        q = torch.randn(B, S, Hq, D, generator=g).to(dt)
        k = torch.randn(B, S, Hkv, D, generator=g).to(dt)
        v = torch.randn(B, S, Hkv, D, generator=g).to(dt)
        do = torch.randn(B, S, Hq, D, generator=g).to(dt)
        return q, k, v, do

    cos, sin = rope_tables(D, S, theta)
    used = dtype
    try:
        args = make(dtype)
        reference_fwd_bwd(*args[:3], cos, sin, args[3])
    except RuntimeError:
        used = torch.float32
        args = make(used)
        reference_fwd_bwd(*args[:3], cos, sin, args[3])
    times = []
    start = time.perf_counter()
    while len(times) < max_reps and (len(times) < 3 or time.perf_counter() - start < min_seconds):
        t0 = time.perf_counter()
        reference_fwd_bwd(*args[:3], cos, sin, args[3])
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times), used
