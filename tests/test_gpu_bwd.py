"""GPU parity of the backward (kf_attn_bwd via autograd of kf::attn_fwd).

Every gradient element is checked against the float64 oracle from the same
inputs with a per-element bound (gpu_util.grad_bound): absolute 1e-5 for
float32; for bf16, 2e-2 plus half a bf16 ulp of the reference value (the
rounding of the bf16 output itself).  Each check prints its observed error.
"""

from __future__ import annotations

import pytest
import torch

import make_fixtures as mf
from gpu_util import DEV, TOL, announce, check_grad, check_out, half_ulp, load_fixture, seeded
from kempnerforge_amd import _lib, ops
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu

def _grads(q, k, v, do, cos, sin, causal=True):
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    out = ops.attention(qd, kd, vd, cos.to(DEV), sin.to(DEV), causal=causal)
    out.backward(do.to(DEV))
    torch.cuda.synchronize()
    return out, qd.grad, kd.grad, vd.grad


@pytest.mark.parametrize("name", list(mf.ATTN_CASES))
def test_fixture(name):
    announce(f"bwd fixture {name}")
    fx = load_fixture(name)
    dtype = mf.ATTN_CASES[name][0]
    q, k, v, do, cos, sin = mf.attn_inputs(*mf.ATTN_CASES[name])
    _, dq, dk, dv = _grads(q, k, v, do, cos, sin)
    for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        check_grad(got, torch.from_numpy(fx[key]), dtype, f"{name} {key}")


SHAPES = [
    (torch.bfloat16, 2, 200, 4, 4, 64),
    (torch.bfloat16, 1, 300, 8, 1, 128),
    (torch.bfloat16, 1, 130, 6, 2, 128),
    (torch.bfloat16, 1, 64, 4, 2, 32),
    (torch.float32, 1, 100, 8, 2, 128),      # fp32 matrix-core kernels
    (torch.float32, 1, 64, 4, 2, 32),        # generic kernels (fp32, D=32)
]


@pytest.mark.parametrize("cfg", SHAPES, ids=lambda c: "-".join(map(str, c)))
@pytest.mark.parametrize("causal", [True, False])
def test_shapes(cfg, causal):
    dtype, B, S, Hq, Hkv, D = cfg
    announce(f"bwd {cfg} causal={causal}")
    q = seeded((B, S, Hq, D), 0, dtype)
    k = seeded((B, S, Hkv, D), 1, dtype)
    v = seeded((B, S, Hkv, D), 2, dtype)
    do = seeded((B, S, Hq, D), 3, dtype)
    cos, sin = ref.rope_tables(D, S, 5e5)
    _, dq, dk, dv = _grads(q, k, v, do, cos, sin, causal)
    dq_r, dk_r, dv_r = ref.attention_bwd(q, k, v, cos, sin, do, causal=causal)
    check_grad(dq, dq_r, dtype, "dq")
    check_grad(dk, dk_r, dtype, "dk", group=Hq // Hkv)
    check_grad(dv, dv_r, dtype, "dv", group=Hq // Hkv)


# n_rep 1, 2, 3, 4 and 8 (the dQ kernel groups 4, 2 or 1 query heads per
# workgroup); lengths off the 64-position tiles and 128-key blocks
DS_SHAPES = [
    (1, 333, 2, 2, 128),
    (2, 200, 4, 2, 64),
    (1, 130, 6, 2, 128),
    (1, 257, 8, 2, 128),
    (1, 190, 16, 2, 64),
]


@pytest.mark.parametrize("cfg", DS_SHAPES, ids=lambda c: "-".join(map(str, c)))
@pytest.mark.parametrize("causal", [True, False])
def test_kept_and_recomputed_ds(cfg, causal):
    """Both backward paths against the oracle: the default workspace, with which
    the dK/dV pass keeps its dS tiles for dQ, and the minimal one (low_memory),
    with which dQ recomputes S and dP.  dK and dV come from the same arithmetic
    either way (bitwise equal)."""
    B, S, Hq, Hkv, D = cfg
    announce(f"bwd kept/recomputed dS {cfg} causal={causal}")
    q = seeded((B, S, Hq, D), 10, torch.bfloat16)
    k = seeded((B, S, Hkv, D), 11, torch.bfloat16)
    v = seeded((B, S, Hkv, D), 12, torch.bfloat16)
    do = seeded((B, S, Hq, D), 13, torch.bfloat16)
    cos, sin = ref.rope_tables(D, S, 5e5)
    args = [t.to(DEV) for t in (q, k, v, cos, sin)]
    out, lse = ops.fwd_raw(*args, causal=causal, k_rotated=False)
    kept = ops.bwd_raw(*args, out, lse, do.to(DEV), causal=causal)
    recomputed = ops.bwd_raw(*args, out, lse, do.to(DEV), causal=causal, low_memory=True)
    torch.cuda.synchronize()
    assert torch.equal(kept[1], recomputed[1]) and torch.equal(kept[2], recomputed[2])
    refs = ref.attention_bwd(q, k, v, cos, sin, do, causal=causal)
    for path, grads in (("kept", kept), ("recomputed", recomputed)):
        for got, want, name in zip(grads, refs, ("dq", "dk", "dv")):
            check_grad(got, want, torch.bfloat16, f"{path} {name}",
                       group=Hq // Hkv if name != "dq" else 1)


def test_ds_budget_switches_paths():
    """The memory-aware default: with a budget too small for the dS tiles the
    default backward takes the recomputing path (dQ equals low_memory=True bit
    for bit), with a large one the kept-tile path; dK and dV are the same bits
    on both paths."""
    B, S, Hq, Hkv, D = 1, 1024, 8, 2, 128
    announce("bwd dS budget switch")
    q, k, v, do = (seeded((B, S, h, D), 20 + i, torch.bfloat16).to(DEV)
                   for i, h in enumerate((Hq, Hkv, Hkv, Hq)))
    cos, sin = (t.to(DEV) for t in ref.rope_tables(D, S, 5e5))
    out, lse = ops.fwd_raw(q, k, v, cos, sin, causal=True, k_rotated=False)
    rec = ops.bwd_raw(q, k, v, cos, sin, out, lse, do, causal=True, low_memory=True)
    try:
        ops.set_backward_ds_budget(1e-9)
        small = ops.bwd_raw(q, k, v, cos, sin, out, lse, do, causal=True)
        ops.set_backward_ds_budget(1.0)
        large = ops.bwd_raw(q, k, v, cos, sin, out, lse, do, causal=True)
    finally:
        ops.set_backward_ds_budget(0.5)
    torch.cuda.synchronize()
    assert torch.equal(small[0], rec[0])
    assert not torch.equal(large[0], rec[0])  # the kept tiles' dQ is other arithmetic
    for a, b in ((small, rec), (large, rec)):
        assert torch.equal(a[1], b[1]) and torch.equal(a[2], b[2])


def test_llama8b_shape_one_group():
    """C3 at full size (B=4, S=4096, Hq=32, Hkv=8, D=128): the backward of KV
    group (b=1, g=6) against the oracle (groups are independent), plus
    determinism of a second backward."""
    B, S, Hq, Hkv, D = 4, 4096, 32, 8, 128
    announce("bwd 8B shape")
    q = seeded((B, S, Hq, D), 0, torch.bfloat16)
    k = seeded((B, S, Hkv, D), 1, torch.bfloat16)
    v = seeded((B, S, Hkv, D), 2, torch.bfloat16)
    do = seeded((B, S, Hq, D), 3, torch.bfloat16)
    cos, sin = ref.rope_tables(D, S, 5e5)
    with _lib.KernelTimer() as kt:
        _, dq, dk, dv = _grads(q, k, v, do, cos, sin)
    # 1024 dK/dV items: the persistent grid needs no split of them
    assert "dkdv_reduce" not in kt.stats, kt.stats
    _, dq2, dk2, dv2 = _grads(q, k, v, do, cos, sin)
    assert torch.equal(dq, dq2) and torch.equal(dk, dk2) and torch.equal(dv, dv2)
    b, g = 1, 6
    hs = slice(4 * g, 4 * g + 4)
    dq_r, dk_r, dv_r = ref.attention_bwd(q[b:b + 1, :, hs], k[b:b + 1, :, g:g + 1],
                                         v[b:b + 1, :, g:g + 1], cos, sin, do[b:b + 1, :, hs])
    check_grad(dq[b:b + 1, :, hs], dq_r, torch.bfloat16, "C3 dq")
    check_grad(dk[b:b + 1, :, g:g + 1], dk_r, torch.bfloat16, "C3 dk")
    check_grad(dv[b:b + 1, :, g:g + 1], dv_r, torch.bfloat16, "C3 dv")


# The reference's tensor-parallel rank shares (TP = 4, configs/train/*_tp4*.toml:
# 70B B=2 Hq=16 Hkv=2, 29B B=1 Hq=12 Hkv=2, 13B B=4 Hq=10 Hkv=2) at shorter
# lengths, and a one-KV-head case: too few dK/dV items for the persistent grid,
# so each is split over the KV group's query heads (8, 6, 5 and 4 parts) and
# dkdv_reduce adds the parts
SPLIT_SHAPES = [
    (2, 1024, 16, 2, 128),
    (1, 1024, 12, 2, 128),
    (4, 512, 10, 2, 128),
    (1, 700, 4, 1, 64),
]


@pytest.mark.parametrize("cfg", SPLIT_SHAPES, ids=lambda c: "-".join(map(str, c)))
def test_split_dkdv_items(cfg):
    B, S, Hq, Hkv, D = cfg
    announce(f"bwd split dK/dV items {cfg}")
    q = seeded((B, S, Hq, D), 50, torch.bfloat16)
    k = seeded((B, S, Hkv, D), 51, torch.bfloat16)
    v = seeded((B, S, Hkv, D), 52, torch.bfloat16)
    do = seeded((B, S, Hq, D), 53, torch.bfloat16)
    cos, sin = ref.rope_tables(D, S, 5e5)
    with _lib.KernelTimer() as kt:
        _, dq, dk, dv = _grads(q, k, v, do, cos, sin)
    assert "dkdv_reduce" in kt.stats, kt.stats
    dq_r, dk_r, dv_r = ref.attention_bwd(q, k, v, cos, sin, do)
    check_grad(dq, dq_r, torch.bfloat16, "dq")
    check_grad(dk, dk_r, torch.bfloat16, "dk", group=Hq // Hkv)
    check_grad(dv, dv_r, torch.bfloat16, "dv", group=Hq // Hkv)
    # a second backward is bit-identical (the parts are added in a fixed order)
    _, dq2, dk2, dv2 = _grads(q, k, v, do, cos, sin)
    assert torch.equal(dq, dq2) and torch.equal(dk, dk2) and torch.equal(dv, dv2)


def test_llama70b_shape_prefix_and_identities():
    """C5 at full size (B=1, S=16384, Hq=64, Hkv=8, D=128), fwd+bwd.

    The oracle cannot hold this size, so it is tied to one it can:
    * causal prefix: rows < 2048 of out, LSE and dQ depend only on the first
      2048 positions, so they equal (bitwise) a run on that prefix, which is
      checked against the oracle for one KV group;
    * dV: rows of P sum to one, so sum_j dV_j = sum over the group's query
      heads and positions of dO;
    * dK: rows of dS sum to zero, so the RoPE-rotated dK sums to zero over keys.
    """
    B, S, Hq, Hkv, D, Sp = 1, 16384, 64, 8, 128, 2048
    n_rep = Hq // Hkv
    announce("bwd 70B shape")
    q = seeded((B, S, Hq, D), 0, torch.bfloat16)
    k = seeded((B, S, Hkv, D), 1, torch.bfloat16)
    v = seeded((B, S, Hkv, D), 2, torch.bfloat16)
    do = seeded((B, S, Hq, D), 3, torch.bfloat16)
    cos, sin = ref.rope_tables(D, S, 5e5)
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    out, lse = ops.fwd_raw(qd.detach(), kd.detach(), vd.detach(), cos.to(DEV), sin.to(DEV),
                           causal=True, k_rotated=False)
    out_a = ops.attention(qd, kd, vd, cos.to(DEV), sin.to(DEV), causal=True)
    out_a.backward(do.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(out, out_a.detach())
    dq, dk, dv = qd.grad, kd.grad, vd.grad
    assert all(torch.isfinite(t.float()).all() for t in (out, dq, dk, dv))

    # causal prefix
    out_p, lse_p = ops.fwd_raw(q[:, :Sp].to(DEV), k[:, :Sp].to(DEV), v[:, :Sp].to(DEV),
                               cos[:Sp].to(DEV), sin[:Sp].to(DEV), causal=True, k_rotated=False)
    _, dq_p, dk_p, dv_p = _grads(q[:, :Sp], k[:, :Sp], v[:, :Sp], do[:, :Sp], cos[:Sp], sin[:Sp])
    assert torch.equal(out[:, :Sp], out_p)
    assert torch.equal(lse[:, :, :Sp], lse_p)
    assert torch.equal(dq[:, :Sp], dq_p)
    g = 5
    hs = slice(n_rep * g, n_rep * g + n_rep)
    args = (q[:, :Sp, hs], k[:, :Sp, g:g + 1], v[:, :Sp, g:g + 1], cos[:Sp], sin[:Sp])
    o_r, _ = ref.attention_fwd(*args)
    dq_r, dk_r, dv_r = ref.attention_bwd(*args, do[:, :Sp, hs])
    check_out(out_p[:, :, hs], o_r, 2e-2, "C5 prefix out")
    check_grad(dq_p[:, :, hs], dq_r, torch.bfloat16, "C5 prefix dq")
    check_grad(dk_p[:, :, g:g + 1], dk_r, torch.bfloat16, "C5 prefix dk")
    check_grad(dv_p[:, :, g:g + 1], dv_r, torch.bfloat16, "C5 prefix dv")

    # sum identities at full length, per KV head
    dv_sum = dv.float().sum(dim=1)                                   # [B, Hkv, D]
    do_sum = do.to(DEV).float().view(B, S, Hkv, n_rep, D).sum(dim=(1, 3))
    assert (dv_sum - do_sum).abs().max() <= 2e-2 * max(1.0, do_sum.abs().max().item())
    dk_rot = ref.apply_rope(dk.float().transpose(1, 2).cpu(), cos, sin)   # [B, Hkv, S, D]
    resid = dk_rot.sum(dim=2).abs().max().item()
    scale = dk_rot.pow(2).sum(dim=2).sqrt().max().item()
    assert resid <= 2e-2 * scale


def test_two_tile_dq_long_odd_sequence():
    """S > 8192 takes the two-query-tile dQ-from-records kernel; with an odd
    number of 64-row tiles its last workgroup holds one tile.  Its dQ rows
    below 2048 equal a 2048-token run's (the one-tile kernel) bit for bit (a
    causal row's dQ depends on rows and keys up to it only), the whole dQ
    agrees with the recomputing path (low_memory) to twice the per-element bf16
    gradient bound (each path is within it of the exact value), and
    dK / dV are the same bits on both paths."""
    B, S, Hq, Hkv, D = 1, 8256, 8, 2, 128  # 129 query tiles
    announce("bwd two-tile dQ, S=8256")
    q, k, v, do = (seeded((B, S, h, D), 40 + i, torch.bfloat16).to(DEV)
                   for i, h in enumerate((Hq, Hkv, Hkv, Hq)))
    cos, sin = (t.to(DEV) for t in ref.rope_tables(D, S, 5e5))
    out, lse = ops.fwd_raw(q, k, v, cos, sin, causal=True, k_rotated=False)
    kept = ops.bwd_raw(q, k, v, cos, sin, out, lse, do, causal=True)
    rec = ops.bwd_raw(q, k, v, cos, sin, out, lse, do, causal=True, low_memory=True)
    n = 2048
    sl = lambda t: t[:, :n].contiguous()  # noqa: E731
    o2, l2 = ops.fwd_raw(sl(q), sl(k), sl(v), cos[:n], sin[:n], causal=True, k_rotated=False)
    short = ops.bwd_raw(sl(q), sl(k), sl(v), cos[:n], sin[:n], o2, l2, sl(do), causal=True)
    torch.cuda.synchronize()
    assert torch.equal(kept[1], rec[1]) and torch.equal(kept[2], rec[2])
    assert torch.equal(kept[0][:, :n], short[0])
    # each path within the per-element gradient bound (2e-2 + half an ulp) of
    # the exact value, so the two within twice that of each other
    err = (kept[0].double() - rec[0].double()).abs()
    bound = 2 * (2e-2 + half_ulp(rec[0].double(), torch.bfloat16))
    print(f"dq kept vs recomputed max-abs {err.max().item():.3e}, "
          f"worst/bound {(err / bound).max().item():.3f}")
    assert bool((err <= bound).all())
