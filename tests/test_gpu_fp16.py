"""float16 on the MFMA kernels.

The reference trains in float16 when ``mixed_precision = "fp16"``
(kempnerforge/config/training.py:31,61): q, k and v then reach SDPA
(kempnerforge/model/attention.py:231) and the decode and capture paths in
float16.  The same kernels as for bfloat16 run, with fp16 MFMAs and the
roundings (RoPE's eager per-op rounding, P, dS, outputs) to fp16.  Checked
here against the float64 oracle on the same inputs: outputs and gradients
within 5e-3 (gpu_util.TOL, plus half an fp16 ulp on gradients), LSE within
1e-3, the rotated keys the forward keeps and the decode writes into the cache
bit for bit, capture probabilities within 1e-5; the rotated-operand pair equal
to the plain entry points bit for bit; and the launches named by the library's
kernel timer are the MFMA ones, not the generic kernels.
"""

from __future__ import annotations

import pytest
import torch

from gpu_util import DEV, TOL, announce, check_grad, check_out, max_abs, seeded
from kempnerforge_amd import _lib, ops
from kempnerforge_amd.norm import RMSNorm
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu

F16 = torch.float16
GENERIC = {"fwd_generic", "bwd_dkdv_generic", "bwd_dq_generic", "bwd_delta_generic",
           "capture_probs_generic", "decode_generic"}


def _inputs(B, S, Hq, Hkv, D, seed=0, theta=5e5):
    q = seeded((B, S, Hq, D), seed, F16)
    k = seeded((B, S, Hkv, D), seed + 1, F16)
    v = seeded((B, S, Hkv, D), seed + 2, F16)
    do = seeded((B, S, Hq, D), seed + 3, F16)
    cos, sin = ref.rope_tables(D, S, theta)
    return q, k, v, do, cos, sin


def _doc_ids(B, S, seed=5):
    g = torch.Generator().manual_seed(seed)
    cuts = torch.sort(torch.randint(1, S, (B, 4), generator=g), dim=1).values
    pos = torch.arange(S).expand(B, S)
    return (pos[:, :, None] >= cuts[:, None, :]).sum(-1).to(torch.int32)


def _key_padding(B, S):
    valid = torch.ones(B, S, dtype=torch.bool)
    valid[0, :17] = False           # leading padding: guarded rows
    if B > 1:
        valid[1, S - 40:] = False   # trailing padding
    return valid


CASES = [
    # B, S, Hq, Hkv, D, causal, mask
    (2, 200, 8, 2, 128, True, None),
    (1, 300, 8, 1, 128, True, None),
    (2, 130, 4, 4, 64, True, None),
    (1, 257, 8, 2, 128, False, None),
    (2, 320, 8, 2, 128, True, "doc"),
    (2, 192, 4, 2, 64, True, "kpm"),
]


def _masks(mask, B, S):
    if mask == "doc":
        return {"doc_ids": _doc_ids(B, S)}
    if mask == "kpm":
        return {"key_padding_mask": _key_padding(B, S)}
    return {}


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(map(str, c)))
def test_forward_backward(case):
    B, S, Hq, Hkv, D, causal, mask = case
    announce(f"fp16 fwd+bwd {case}")
    q, k, v, do, cos, sin = _inputs(B, S, Hq, Hkv, D)
    m = _masks(mask, B, S)
    md = {n: t.to(DEV) for n, t in m.items()}
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    with _lib.KernelTimer() as timer:
        out = ops.attention(qd, kd, vd, cos.to(DEV), sin.to(DEV), causal=causal, **md)
        out.backward(do.to(DEV))
        torch.cuda.synchronize()
    ran = set(timer.stats)
    assert {"fwd_mfma", "bwd_dkdv"} <= ran and not ran & GENERIC, ran
    o_ref, _ = ref.attention_fwd(q, k, v, cos, sin, causal=causal, **m)
    check_out(out, o_ref, TOL[F16], "out")
    grads = ref.attention_bwd(q, k, v, cos, sin, do, causal=causal, **m)
    for got, want, name in zip((qd.grad, kd.grad, vd.grad), grads, ("dq", "dk", "dv")):
        check_grad(got, want, F16, name, group=Hq // Hkv if name != "dq" else 1)


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(map(str, c)))
def test_lse_rot_and_ds_paths(case):
    """LSE against the closed form; the rotated-operand pair equals the plain
    entry points bit for bit and its rot holds the oracle's fp16 rotation; dK
    and dV are the same bits with the dS records kept or recomputed."""
    B, S, Hq, Hkv, D, causal, mask = case
    announce(f"fp16 lse/rot/dS {case}")
    q, k, v, do, cos, sin = _inputs(B, S, Hq, Hkv, D, seed=10)
    m = _masks(mask, B, S)
    md = {n: t.to(DEV) for n, t in m.items()}
    q, k, v, do, cos, sin = (t.to(DEV) for t in (q, k, v, do, cos, sin))
    res = ops.fwd_rot_raw(q, k, v, cos, sin, causal=causal, **md)
    assert res is not None, "the rotated-operand path should take fp16"
    out_r, lse_r, rot = res
    out, lse = ops.fwd_raw(q, k, v, cos, sin, causal=causal, k_rotated=False, **md)
    torch.cuda.synchronize()
    assert torch.equal(out_r, out) and torch.equal(lse_r, lse)
    _, l_ref = ref.attention_fwd(q.cpu(), k.cpu(), v.cpu(), cos.cpu(), sin.cpu(),
                                 causal=causal, **m)
    check_out(lse, l_ref, 1e-3, "lse")
    P = (S + 127) // 128 * 128
    kr = rot[:B * Hkv * P * D].view(B, Hkv, P, D).cpu()
    qr = rot[B * Hkv * P * D:].view(B, Hq, P, D).cpu()
    cs, sn = cos.cpu(), sin.cpu()
    assert torch.equal(kr[:, :, :S], ref.apply_rope(k.cpu().transpose(1, 2), cs, sn))
    assert torch.equal(qr[:, :, :S], ref.apply_rope(q.cpu().transpose(1, 2), cs, sn))
    assert not kr[:, :, S:].any() and not qr[:, :, S:].any()
    kept = ops.bwd_rot_raw(rot, v, cos, sin, out, lse, do, causal=causal, **md)
    plain = ops.bwd_raw(q, k, v, cos, sin, out, lse, do, causal=causal, **md)
    recomputed = ops.bwd_raw(q, k, v, cos, sin, out, lse, do, causal=causal, low_memory=True,
                             **md)
    torch.cuda.synchronize()
    for a, b, name in zip(kept, plain, ("dq", "dk", "dv")):
        assert torch.equal(a, b), f"rot pair {name} differs"
    assert torch.equal(plain[1], recomputed[1]) and torch.equal(plain[2], recomputed[2])
    grads = ref.attention_bwd(q.cpu(), k.cpu(), v.cpu(), cs, sn, do.cpu(), causal=causal, **m)
    check_grad(recomputed[0], grads[0], F16, "dq (recomputed)")


@pytest.mark.parametrize("cfg", [
    # B, Hq, Hkv, D, lens lo, hi, Smax
    (4, 32, 8, 128, 900, 2100, 2200),
    (3, 8, 8, 64, 1, 300, 400),
    (2, 16, 1, 128, 500, 700, 800),   # n_rep 16, the widest the stream kernel takes
], ids=lambda c: "-".join(map(str, c)))
def test_decode(cfg):
    B, Hq, Hkv, D, lo, hi, Smax = cfg
    announce(f"fp16 decode {cfg}")
    g = torch.Generator().manual_seed(4)
    lens = torch.randint(lo, hi + 1, (B,), generator=g, dtype=torch.int32)
    q = seeded((B, 1, Hq, D), 0, F16)
    kn = seeded((B, 1, Hkv, D), 1, F16)
    vn = seeded((B, 1, Hkv, D), 2, F16)
    kc = seeded((B, Hkv, Smax, D), 5, F16)
    vc = seeded((B, Hkv, Smax, D), 6, F16)
    cos, sin = ref.rope_tables(D, Smax, 5e5)
    kcd, vcd = kc.to(DEV), vc.to(DEV)
    with _lib.KernelTimer() as timer:
        out = ops.decode_raw(q.to(DEV), kn.to(DEV), vn.to(DEV), kcd, vcd, lens.to(DEV),
                             cos.to(DEV), sin.to(DEV), rope_row_offset=0,
                             max_len=int(lens.max()) + 1)
        torch.cuda.synchronize()
    assert "decode_stream" in timer.stats and "decode_generic" not in timer.stats, timer.stats
    o_ref, kc_ref, vc_ref = ref.decode_step(q, kn, vn, kc, vc, lens, cos, sin)
    check_out(out, o_ref, TOL[F16], "decode out")
    assert torch.equal(kcd.cpu(), kc_ref) and torch.equal(vcd.cpu(), vc_ref)


def test_decode_qk_norm():
    """The fused QK-norm decode in fp16 equals RMSNorm (reference module, fp16
    weights) followed by the plain decode, and the oracle on the normalised rows."""
    announce("fp16 qk-norm decode")
    B, Hq, Hkv, D, Smax = 3, 8, 2, 128, 700
    lens = torch.tensor([5, 333, 698], dtype=torch.int32)
    qn = seeded((B, 1, Hq, D), 0, F16) * 3
    kn = seeded((B, 1, Hkv, D), 1, F16) * 3
    vn = seeded((B, 1, Hkv, D), 2, F16)
    kc = seeded((B, Hkv, Smax, D), 3, F16)
    vc = seeded((B, Hkv, Smax, D), 4, F16)
    cos, sin = ref.rope_tables(D, Smax, 5e5)
    g = torch.Generator().manual_seed(9)
    qnorm, knorm = RMSNorm(D), RMSNorm(D)
    with torch.no_grad():
        qnorm.weight.copy_(1 + 0.1 * torch.randn(D, generator=g))
        knorm.weight.copy_(1 + 0.1 * torch.randn(D, generator=g))
    qnorm, knorm = qnorm.to(DEV, F16), knorm.to(DEV, F16)
    args = dict(rope_row_offset=0, max_len=Smax)
    kc1, vc1, kc2, vc2 = (t.to(DEV) for t in (kc, vc, kc, vc))
    fused = ops.decode_raw(qn.to(DEV), kn.to(DEV), vn.to(DEV), kc1, vc1, lens.to(DEV),
                           cos.to(DEV), sin.to(DEV), q_norm_weight=qnorm.weight,
                           k_norm_weight=knorm.weight, norm_eps=qnorm.eps, **args)
    with torch.no_grad():
        qq, kk = qnorm(qn.to(DEV)), knorm(kn.to(DEV))
    plain = ops.decode_raw(qq, kk, vn.to(DEV), kc2, vc2, lens.to(DEV), cos.to(DEV), sin.to(DEV),
                           **args)
    want, kc_ref, _ = ref.decode_step(qq.cpu(), kk.cpu(), vn, kc, vc, lens, cos, sin)
    torch.cuda.synchronize()
    check_out(fused, plain.cpu(), TOL[F16], "fused vs RMSNorm + decode")
    check_out(fused, want, TOL[F16], "fused vs oracle")
    # the new key row: the plain path writes the oracle's rotation of the
    # normalised key bit for bit; the fused one normalises in the kernel (its
    # float32 reduction order differs from torch's: within the tolerance)
    assert torch.equal(vc1, vc2)
    for b in range(B):
        L = int(lens[b])
        assert torch.equal(kc2[b, :, L].cpu(), kc_ref[b, :, L])
        check_out(kc1[b, :, L], kc_ref[b, :, L], TOL[F16], f"new key row {b}")


@pytest.mark.parametrize("cfg", [
    (1, 200, 8, 2, 128, True, None),
    (2, 130, 4, 4, 64, False, None),
    (2, 256, 8, 2, 128, True, "doc"),
    (2, 192, 4, 2, 64, True, "kpm"),
], ids=lambda c: "-".join(map(str, c)))
def test_capture(cfg):
    B, S, Hq, Hkv, D, causal, mask = cfg
    announce(f"fp16 capture {cfg}")
    q, k, v, _, cos, sin = _inputs(B, S, Hq, Hkv, D)
    m = _masks(mask, B, S)
    md = {n: t.to(DEV) for n, t in m.items()}
    with _lib.KernelTimer() as timer:
        out, p, _ = ops.capture_raw(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV),
                                    causal=causal, k_rotated=False, **md)
        torch.cuda.synchronize()
    assert "capture_probs_mfma" in timer.stats and not set(timer.stats) & GENERIC, timer.stats
    o_ref, p_ref = ref.capture(q, k, v, cos, sin, causal=causal, **m)
    check_out(p, p_ref, 1e-5, "probs")
    check_out(out, o_ref, TOL[F16], "capture out")


def test_llama8b_shape_fp16():
    """C3 in float16: spot rows of the forward against the oracle, one KV group's
    gradients in full, determinism of a recompute."""
    B, S, Hq, Hkv, D = 4, 4096, 32, 8, 128
    announce("fp16 8B shape")
    q, k, v, do, cos, sin = _inputs(B, S, Hq, Hkv, D)
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    out = ops.attention(qd, kd, vd, cos.to(DEV), sin.to(DEV))
    out.backward(do.to(DEV))
    out2, _ = ops.fwd_raw(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV), causal=True,
                          k_rotated=False)
    torch.cuda.synchronize()
    assert torch.equal(out.detach(), out2)
    rows = torch.tensor([0, 1, 63, 64, 1000, 2048, 4095])
    heads = torch.tensor([0, 5, 31])
    o_ref, _ = ref.attention_fwd_rows(q, k, v, cos, sin, rows, heads=heads)
    check_out(out.detach().cpu()[:, rows][:, :, heads], o_ref, TOL[F16], "out rows")
    # KV group 3 of batch row 1 alone: its four query heads and one KV head
    b, g = 1, 3
    hs = slice(4 * g, 4 * g + 4)
    grads = ref.attention_bwd(q[b:b + 1, :, hs], k[b:b + 1, :, g:g + 1], v[b:b + 1, :, g:g + 1],
                              cos, sin, do[b:b + 1, :, hs])
    check_grad(qd.grad[b:b + 1, :, hs], grads[0], F16, "dq group")
    check_grad(kd.grad[b:b + 1, :, g:g + 1], grads[1], F16, "dk group", group=4)
    check_grad(vd.grad[b:b + 1, :, g:g + 1], grads[2], F16, "dv group", group=4)
