"""float32 on the fp32 matrix-core kernels (kf_f32.hip).

The reference trains in float32 when ``mixed_precision = "fp32"``
(kempnerforge/config/training.py:31); q, k and v then reach SDPA
(kempnerforge/model/attention.py:231) in float32 and nothing in the path
rounds below it.  Checked here against the float64 oracle on the same inputs
with the north star's float32 bound, max-abs 1e-5 on the output, the LSE and
every gradient element; the launches named by the library's kernel timer are
the fp32 MFMA ones, not the generic kernels (which keep float32 for other
head sizes and both explicit masks at once, tested in the other files).
"""

from __future__ import annotations

import pytest
import torch

from gpu_util import DEV, announce, check_grad, check_out, seeded
from kempnerforge_amd import _lib, ops
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu

F32 = torch.float32
TOL = 1e-5
GENERIC = {"fwd_generic", "bwd_dkdv_generic", "bwd_dq_generic", "bwd_delta_generic"}
FWD = {"fwd_f32"}
BWD = {"stats_f32", "bwd_dkdv_f32"}  # and bwd_dq_f32 or, from the dS records, bwd_dq_rec_f32


def _inputs(B, S, Hq, Hkv, D, seed=0, theta=5e5):
    q = seeded((B, S, Hq, D), seed, F32)
    k = seeded((B, S, Hkv, D), seed + 1, F32)
    v = seeded((B, S, Hkv, D), seed + 2, F32)
    do = seeded((B, S, Hq, D), seed + 3, F32)
    cos, sin = ref.rope_tables(D, S, theta)
    return q, k, v, do, cos, sin


CASES = [
    # B, S, Hq, Hkv, D, causal        (what it exercises)
    (2, 256, 4, 2, 64, True),      # the debug configuration's shape (C1)
    (1, 300, 8, 1, 128, True),     # MQA, ragged last tile and key block
    (2, 130, 4, 4, 64, False),     # MHA, full attention
    (1, 257, 8, 2, 128, False),
    (1, 100, 12, 4, 128, True),    # n_rep 3: 63 of 64 workgroup rows used
    (1, 96, 64, 1, 128, True),     # n_rep 64: one position per workgroup
    (1, 1, 4, 2, 128, True),       # single token
    (2, 33, 6, 2, 64, True),
    (1, 1000, 8, 2, 128, True),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(map(str, c)))
def test_forward_backward(case):
    B, S, Hq, Hkv, D, causal = case
    announce(f"fp32 fwd+bwd {case}")
    q, k, v, do, cos, sin = _inputs(B, S, Hq, Hkv, D)
    args = [t.to(DEV) for t in (q, k, v, cos, sin)]
    with _lib.KernelTimer() as t:
        out, lse = ops.fwd_raw(*args, causal=causal, k_rotated=False)
        dq, dk, dv = ops.bwd_raw(*args, out, lse, do.to(DEV), causal=causal)
        torch.cuda.synchronize()
    ran = set(t.stats)
    assert FWD | BWD <= ran and not ran & GENERIC, ran
    o_ref, l_ref = ref.attention_fwd(q, k, v, cos, sin, causal=causal)
    check_out(out, o_ref, TOL, "out")
    check_out(lse, l_ref, TOL, "lse")
    dq_r, dk_r, dv_r = ref.attention_bwd(q, k, v, cos, sin, do, causal=causal)
    check_grad(dq, dq_r, F32, "dq")
    check_grad(dk, dk_r, F32, "dk", group=Hq // Hkv)
    check_grad(dv, dv_r, F32, "dv", group=Hq // Hkv)


def test_autograd_and_determinism():
    """ops.attention's autograd takes the same kernels; a recompute (activation
    checkpointing) gives the same bits."""
    B, S, Hq, Hkv, D = 2, 384, 8, 2, 128
    announce("fp32 autograd + determinism")
    q, k, v, do, cos, sin = _inputs(B, S, Hq, Hkv, D, seed=20)
    grads = []
    for _ in range(2):
        qd, kd, vd = (x.to(DEV).requires_grad_(True) for x in (q, k, v))
        out = ops.attention(qd, kd, vd, cos.to(DEV), sin.to(DEV), causal=True)
        out.backward(do.to(DEV))
        torch.cuda.synchronize()
        grads.append((out.detach(), qd.grad, kd.grad, vd.grad))
    for a, b in zip(*grads):
        assert torch.equal(a, b)
    dq_r, dk_r, dv_r = ref.attention_bwd(q, k, v, cos, sin, do, causal=True)
    check_grad(grads[0][1], dq_r, F32, "dq")
    check_grad(grads[0][2], dk_r, F32, "dk", group=Hq // Hkv)
    check_grad(grads[0][3], dv_r, F32, "dv", group=Hq // Hkv)


@pytest.mark.parametrize("Sq,Sk", [(1, 300), (64, 333), (200, 200)])
def test_rotated_cache_forward(Sq, Sk):
    """Multi-token forward over a rotated KV cache ([B, Hkv, Smax, D] views,
    Sq <= Sk, top-left causal): the fp32 forward reads the cache rows
    directly (no rotation prepass)."""
    B, Hq, Hkv, D, Smax = 2, 8, 2, 128, 400
    announce(f"fp32 cache forward Sq={Sq} Sk={Sk}")
    q = seeded((B, Sq, Hq, D), 30, F32)
    kc = seeded((B, Hkv, Smax, D), 31, F32)
    vc = seeded((B, Hkv, Smax, D), 32, F32)
    cos, sin = ref.rope_tables(D, Sq, 1e4)
    kd, vd = kc.to(DEV), vc.to(DEV)
    with _lib.KernelTimer() as t:
        out, lse = ops.fwd_raw(q.to(DEV), kd[:, :, :Sk], vd[:, :, :Sk], cos.to(DEV), sin.to(DEV),
                               causal=True, k_rotated=True, k_layout="bhsd")
        torch.cuda.synchronize()
    assert FWD <= set(t.stats) and not set(t.stats) & GENERIC, t.stats
    o_ref, l_ref = ref.attention_fwd_rotated(q, kc[:, :, :Sk], vc[:, :, :Sk], cos, sin)
    check_out(out, o_ref, TOL, "out")
    check_out(lse, l_ref, TOL, "lse")


def test_longer_rows():
    """2048 positions, groups of 4: gradients summed over thousands of float32
    terms still within 1e-5 of the float64 oracle."""
    B, S, Hq, Hkv, D = 1, 2048, 8, 2, 128
    announce("fp32 S=2048")
    q, k, v, do, cos, sin = _inputs(B, S, Hq, Hkv, D, seed=40)
    args = [t.to(DEV) for t in (q, k, v, cos, sin)]
    out, lse = ops.fwd_raw(*args, causal=True, k_rotated=False)
    dq, dk, dv = ops.bwd_raw(*args, out, lse, do.to(DEV), causal=True)
    torch.cuda.synchronize()
    o_ref, l_ref = ref.attention_fwd(q, k, v, cos, sin)
    check_out(out, o_ref, TOL, "out")
    check_out(lse, l_ref, TOL, "lse")
    dq_r, dk_r, dv_r = ref.attention_bwd(q, k, v, cos, sin, do)
    check_grad(dq, dq_r, F32, "dq")
    check_grad(dk, dk_r, F32, "dk", group=Hq // Hkv)
    check_grad(dv, dv_r, F32, "dv", group=Hq // Hkv)


def _doc_ids(B, S, seed):
    g = torch.Generator().manual_seed(seed)
    cuts = torch.sort(torch.randint(1, S, (B, 5), generator=g), dim=1).values
    pos = torch.arange(S).expand(B, S)
    return (pos[:, :, None] >= cuts[:, None, :]).sum(-1).to(torch.int32)


def _key_padding(B, S, layout, seed=0):
    m = torch.ones(B, S, dtype=torch.bool)
    g = torch.Generator().manual_seed(seed)
    for b in range(B):
        if layout == "leading":       # rows before the first valid key are guarded
            m[b, : 45 + 29 * b] = False
        elif layout == "random":
            m[b] = torch.rand(S, generator=g) > 0.3
        elif layout == "none_valid":  # an all-padded row: every row guarded
            m[b] = b % 2 == 1
        elif layout == "trailing":
            m[b, S - 50 - 7 * b:] = False
        elif layout == "row1_only":   # batch row 0 all valid (plain causal), row 1 padded
            m[b, 100:] = b == 0
    return m


# B, S, Hq, Hkv, D, mask
MASKED = [
    (2, 300, 8, 2, 128, "doc"),
    (1, 333, 4, 4, 64, "doc"),
    (1, 200, 32, 1, 128, "doc"),
    (2, 300, 8, 2, 128, "leading"),
    (2, 257, 6, 2, 64, "random"),
    (2, 160, 4, 2, 128, "none_valid"),
    (2, 190, 8, 1, 128, "trailing"),
    (2, 230, 8, 2, 128, "row1_only"),
    (1, 333, 8, 2, 64, "doc_repeating"),
    (1, 1, 4, 2, 128, "leading"),        # a single guarded position
]


@pytest.mark.parametrize("case", MASKED, ids=lambda c: "-".join(map(str, c)))
def test_explicit_masks(case):
    """Packed documents and key padding (guarded rows included) on the fp32
    kernels: out, LSE and gradients against the oracle with the explicit mask."""
    B, S, Hq, Hkv, D, kind = case
    announce(f"fp32 masked {case}")
    q, k, v, do, cos, sin = _inputs(B, S, Hq, Hkv, D, seed=50)
    if kind == "doc":
        masks = {"doc_ids": _doc_ids(B, S, 51)}
    elif kind == "doc_repeating":  # ids recur (0, 1, 2, 0, 1, ...): same-id runs apart see each other
        masks = {"doc_ids": ((torch.arange(S) // 37) % 3).to(torch.int32).expand(B, S).contiguous()}
    else:
        masks = {"key_padding_mask": _key_padding(B, S, kind, 52)}
    dev_masks = {n: t.to(DEV) for n, t in masks.items()}
    args = [t.to(DEV) for t in (q, k, v, cos, sin)]
    with _lib.KernelTimer() as t:
        out, lse = ops.fwd_raw(*args, causal=True, k_rotated=False, **dev_masks)
        dq, dk, dv = ops.bwd_raw(*args, out, lse, do.to(DEV), causal=True, **dev_masks)
        torch.cuda.synchronize()
    ran = set(t.stats)
    assert FWD | BWD <= ran and not ran & GENERIC, ran
    o_ref, l_ref = ref.attention_fwd(q, k, v, cos, sin, causal=True, **masks)
    check_out(out, o_ref, TOL, "out")
    check_out(lse, l_ref, TOL, "lse")
    dq_r, dk_r, dv_r = ref.attention_bwd(q, k, v, cos, sin, do, causal=True, **masks)
    check_grad(dq, dq_r, F32, "dq")
    check_grad(dk, dk_r, F32, "dk", group=Hq // Hkv)
    check_grad(dv, dv_r, F32, "dv", group=Hq // Hkv)


# decode: B, Hq, Hkv, D, lo, hi, Smax
DECODE = [
    (3, 8, 8, 64, 1, 300, 400),        # MHA, D=64
    (6, 16, 2, 128, 1022, 1025, 1100),
    (40, 8, 2, 64, 900, 3100, 3200),   # many sequences: few splits each
    (2, 8, 1, 128, 0, 3, 8),           # empty cache (len 0) and tiny
    (2, 6, 2, 128, 10, 90, 100),       # n_rep 3: padded MFMA columns
    (2, 16, 1, 128, 500, 700, 800),    # n_rep 16, the widest
    (1, 64, 8, 128, 1000, 1300, 1400),
]


@pytest.mark.parametrize("cfg", DECODE, ids=lambda c: "-".join(map(str, c)))
def test_decode(cfg):
    """One decode step in float32 on the fp32 matrix cores (split-K over the
    cache, then the merge): out within 1e-5 of the oracle, the new row written
    to the cache bit for bit."""
    B, Hq, Hkv, D, lo, hi, Smax = cfg
    announce(f"fp32 decode {cfg}")
    g = torch.Generator().manual_seed(4)
    lens = torch.randint(lo, hi + 1, (B,), generator=g, dtype=torch.int32)
    q = seeded((B, 1, Hq, D), 0, F32)
    kn = seeded((B, 1, Hkv, D), 1, F32)
    vn = seeded((B, 1, Hkv, D), 2, F32)
    kc = seeded((B, Hkv, Smax, D), 5, F32)
    vc = seeded((B, Hkv, Smax, D), 6, F32)
    cos, sin = ref.rope_tables(D, Smax, 5e5)
    kcd, vcd = kc.to(DEV), vc.to(DEV)
    with _lib.KernelTimer() as t:
        out = ops.decode_raw(q.to(DEV), kn.to(DEV), vn.to(DEV), kcd, vcd, lens.to(DEV),
                             cos.to(DEV), sin.to(DEV), rope_row_offset=0,
                             max_len=int(lens.max()) + 1)
        torch.cuda.synchronize()
    assert {"decode_f32", "decode_merge_f32"} <= set(t.stats) and "decode_generic" not in t.stats
    o_ref, kc_ref, vc_ref = ref.decode_step(q, kn, vn, kc, vc, lens, cos, sin)
    check_out(out, o_ref, TOL, "out")
    assert torch.equal(kcd.cpu(), kc_ref) and torch.equal(vcd.cpu(), vc_ref)


def test_decode_qk_norm_and_bad_length():
    """The fused QK-norm decode in float32 against RMSNorm (the reference
    module, float32) followed by the oracle's decode; then a sequence with an
    out-of-range length: NaN output, caches untouched."""
    from kempnerforge_amd.norm import RMSNorm

    B, Hq, Hkv, D, Smax = 3, 8, 2, 128, 700
    announce("fp32 decode qk-norm")
    lens = torch.tensor([5, 333, 698], dtype=torch.int32)
    qn = seeded((B, 1, Hq, D), 0, F32) * 3
    kn = seeded((B, 1, Hkv, D), 1, F32) * 3
    vn = seeded((B, 1, Hkv, D), 2, F32)
    kc = seeded((B, Hkv, Smax, D), 3, F32)
    vc = seeded((B, Hkv, Smax, D), 4, F32)
    cos, sin = ref.rope_tables(D, Smax, 5e5)
    qnorm, knorm = RMSNorm(D), RMSNorm(D)
    with torch.no_grad():
        g = torch.Generator().manual_seed(9)
        qnorm.weight.copy_(1 + 0.1 * torch.randn(D, generator=g))
        knorm.weight.copy_(1 + 0.1 * torch.randn(D, generator=g))
    kcd, vcd = kc.to(DEV), vc.to(DEV)
    out = ops.decode_raw(qn.to(DEV), kn.to(DEV), vn.to(DEV), kcd, vcd, lens.to(DEV),
                         cos.to(DEV), sin.to(DEV), rope_row_offset=0, max_len=Smax,
                         q_norm_weight=qnorm.weight.to(DEV), k_norm_weight=knorm.weight.to(DEV),
                         norm_eps=qnorm.eps)
    torch.cuda.synchronize()
    with torch.no_grad():
        qq, kk = qnorm(qn), knorm(kn)
    o_ref, kc_ref, _ = ref.decode_step(qq, kk, vn, kc, vc, lens, cos, sin)
    check_out(out, o_ref, TOL, "out")
    for b in range(B):
        L = int(lens[b])
        check_out(kcd[b, :, L], kc_ref[b, :, L], TOL, "k written")
    # lens[1] + 1 > max_len: NaN for that sequence and no cache write
    lens = torch.tensor([10, 700, 20], dtype=torch.int32)
    before = kcd.clone()
    out = ops.decode_raw(qn.to(DEV), kn.to(DEV), vn.to(DEV), kcd, vcd, lens.to(DEV),
                         cos.to(DEV), sin.to(DEV), rope_row_offset=0, max_len=Smax)
    torch.cuda.synchronize()
    assert torch.isnan(out[1]).all()
    assert torch.isfinite(out[0]).all() and torch.isfinite(out[2]).all()
    assert torch.equal(kcd[1], before[1])


# capture: B, S, Hq, Hkv, D, causal, mask
CAPTURE = [
    (1, 200, 8, 2, 128, True, None),
    (2, 130, 4, 4, 64, False, None),
    (1, 33, 6, 2, 128, True, None),      # Sk % 4 != 0: element stores
    (1, 300, 8, 2, 128, True, "doc"),
    (2, 160, 4, 2, 64, True, "leading"),
]


@pytest.mark.parametrize("case", CAPTURE, ids=lambda c: "-".join(map(str, c)))
def test_capture(case):
    """The probability capture in float32 (forward, then the probabilities
    recomputed per tile): P within 1e-5 of the oracle, zeros where masked,
    out within 1e-5."""
    B, S, Hq, Hkv, D, causal, kind = case
    announce(f"fp32 capture {case}")
    q, k, v, _, cos, sin = _inputs(B, S, Hq, Hkv, D, seed=60)
    masks = {}
    if kind == "doc":
        masks = {"doc_ids": _doc_ids(B, S, 61)}
    elif kind is not None:
        masks = {"key_padding_mask": _key_padding(B, S, kind, 62)}
    dev_masks = {n: t.to(DEV) for n, t in masks.items()}
    with _lib.KernelTimer() as t:
        out, p, lse = ops.capture_raw(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV),
                                      causal=causal, k_rotated=False, **dev_masks)
        torch.cuda.synchronize()
    assert {"fwd_f32", "capture_f32"} <= set(t.stats) and not set(t.stats) & GENERIC, t.stats
    o_ref, p_ref = ref.capture(q, k, v, cos, sin, causal=causal, **masks)
    check_out(p, p_ref, TOL, "probs")
    check_out(out, o_ref, TOL, "out")
    assert (p.cpu()[p_ref == 0] == 0).all()  # masked entries exactly zero


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", [(2, 300, 8, 2, 128), (1, 257, 6, 3, 64), (1, 64, 4, 4, 128)],
                         ids=lambda c: "-".join(map(str, c)))
def test_ds_records_and_recompute(shape, causal):
    """The two float32 dQ paths: from the dS records the dK/dV pass keeps
    (default workspace) and recomputing S and dP (low_memory).  dK and dV are
    the same bits either way; both dQ within 1e-5 of the oracle."""
    B, S, Hq, Hkv, D = shape
    announce(f"fp32 dS records {shape} causal={causal}")
    q, k, v, do, cos, sin = _inputs(B, S, Hq, Hkv, D, seed=70)
    args = [t.to(DEV) for t in (q, k, v, cos, sin)]
    out, lse = ops.fwd_raw(*args, causal=causal, k_rotated=False)
    with _lib.KernelTimer() as t1:
        kept = ops.bwd_raw(*args, out, lse, do.to(DEV), causal=causal)
        torch.cuda.synchronize()
    with _lib.KernelTimer() as t2:
        rec = ops.bwd_raw(*args, out, lse, do.to(DEV), causal=causal, low_memory=True)
        torch.cuda.synchronize()
    assert "bwd_dq_rec_f32" in t1.stats and "bwd_dq_f32" not in t1.stats, t1.stats
    assert "bwd_dq_f32" in t2.stats and "bwd_dq_rec_f32" not in t2.stats, t2.stats
    assert torch.equal(kept[1], rec[1]) and torch.equal(kept[2], rec[2])
    dq_r, dk_r, dv_r = ref.attention_bwd(q, k, v, cos, sin, do, causal=causal)
    check_grad(kept[0], dq_r, F32, "dq (records)")
    check_grad(rec[0], dq_r, F32, "dq (recomputed)")
    check_grad(kept[1], dk_r, F32, "dk", group=Hq // Hkv)
    check_grad(kept[2], dv_r, F32, "dv", group=Hq // Hkv)
