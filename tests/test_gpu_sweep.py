"""Seeded randomized sweep of the MFMA paths against the float64 oracle.

The fixed-shape tests pin the cases each kernel was written around; this
sweep draws shapes the kernels' tiling does not favour: lengths 1..700 (off the
32-, 64- and 128-position tiles), n_rep 1..16 (odd groups included), head_dim
64 and 128, several batch rows, causal and full attention, packed documents
and key padding with random boundaries, bf16, fp16 and fp32.  Each case checks the
output and LSE, every gradient element (gpu_util.grad_bound, with the error
that rounding P and dS to the operand type forces added to the bound: on these
short rows it can exceed 2e-2 with otherwise exact arithmetic) and that dK / dV
are the same bits with the dS records kept or recomputed; decode cases check
the output and the cache rows written.  The draws come from a fixed seed, so
the cases are the same on every run and each one is named by its parameters.
"""

from __future__ import annotations

import random

import pytest
import torch

from gpu_util import DEV, TOL, announce, check_grad, check_out, seeded
from kempnerforge_amd import ops
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu


def _draw_attention_cases(n, seed=2024):
    rng = random.Random(seed)
    cases = []
    for i in range(n):
        dtype = rng.choice(["bf16", "fp16"])
        D = rng.choice([64, 128])
        Hkv = rng.choice([1, 2, 4])
        n_rep = rng.choice([1, 2, 3, 4, 5, 8, 16])
        B = rng.choice([1, 2, 3])
        S = rng.choice([1, 2, 31, 33, 63, 65, 127, 129, 191, 255, 257, 300, 383, 448, 511,
                        513, 640, 700])
        mask = rng.choice([None, None, "doc", "kpm"])
        causal = True if mask else rng.random() < 0.75
        cases.append((i, dtype, B, S, Hkv * n_rep, Hkv, D, causal, mask))
    return cases


ATTN = _draw_attention_cases(40)
DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16}


def _mask_tensors(case, rng_seed):
    i, _, B, S, *_rest, mask = case
    g = torch.Generator().manual_seed(rng_seed)
    if mask == "doc":
        ids = []
        for _ in range(B):
            ncut = int(torch.randint(0, 6, (1,), generator=g))
            cuts = torch.sort(torch.randint(1, max(S, 2), (ncut,), generator=g)).values
            pos = torch.arange(S)
            ids.append((pos[:, None] >= cuts[None, :]).sum(-1))
        return {"doc_ids": torch.stack(ids).to(torch.int32)}
    if mask == "kpm":
        valid = torch.rand(B, S, generator=g) > 0.25
        lead = int(torch.randint(0, max(S // 3, 1), (1,), generator=g))
        valid[0, :lead] = False  # a padded prefix in the first row: guarded rows
        if B > 1:
            valid[1] = True      # an unpadded row: the unmasked kernels' share
        return {"key_padding_mask": valid}
    return {}


@pytest.mark.parametrize("case", ATTN, ids=lambda c: "-".join(map(str, c)))
def test_attention_sweep(case):
    i, dname, B, S, Hq, Hkv, D, causal, mask = case
    dtype = DTYPES[dname]
    announce(f"sweep {case}")
    q = seeded((B, S, Hq, D), 100 + i, dtype)
    k = seeded((B, S, Hkv, D), 200 + i, dtype)
    v = seeded((B, S, Hkv, D), 300 + i, dtype)
    do = seeded((B, S, Hq, D), 400 + i, dtype)
    cos, sin = ref.rope_tables(D, S, 5e5)
    m = _mask_tensors(case, 500 + i)
    md = {n: t.to(DEV) for n, t in m.items()}
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    out = ops.attention(qd, kd, vd, cos.to(DEV), sin.to(DEV), causal=causal, **md)
    out.backward(do.to(DEV))
    _, lse = ops.fwd_raw(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV),
                         causal=causal, k_rotated=False, **md)
    rec = ops.bwd_raw(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV), out.detach(),
                      lse, do.to(DEV), causal=causal, low_memory=True, **md)
    torch.cuda.synchronize()
    o_ref, l_ref = ref.attention_fwd(q, k, v, cos, sin, causal=causal, **m)
    check_out(out, o_ref, TOL[dtype], "out")
    check_out(lse, l_ref, 1e-3, "lse")
    grads = ref.attention_bwd(q, k, v, cos, sin, do, causal=causal, **m)
    # the same gradients with P and dS rounded to the operand type: their
    # distance to the exact ones is what the format alone forces (grad_bound)
    rounded = ref.attention_bwd_rounded_operands(q, k, v, cos, sin, do, operand_dtype=dtype,
                                                 causal=causal, **m)
    for got, want, r, name in zip((qd.grad, kd.grad, vd.grad), grads, rounded,
                                  ("dq", "dk", "dv")):
        check_grad(got, want, dtype, name, group=Hq // Hkv if name != "dq" else 1,
                   operand_ref=r)
    check_grad(rec[0], grads[0], dtype, "dq (recomputed)", operand_ref=rounded[0])
    assert torch.equal(rec[1], kd.grad) and torch.equal(rec[2], vd.grad)


def _draw_decode_cases(n, seed=77):
    rng = random.Random(seed)
    cases = []
    for i in range(n):
        dtype = rng.choice(["bf16", "fp16"])
        D = rng.choice([64, 128])
        Hkv = rng.choice([1, 2, 8])
        n_rep = rng.choice([1, 3, 4, 8, 16])
        B = rng.choice([1, 5, 17, 33, 70])
        hi = rng.choice([1, 40, 300, 1100, 2500])
        cases.append((i, dtype, B, Hkv * n_rep, Hkv, D, hi))
    return cases


@pytest.mark.parametrize("case", _draw_decode_cases(12), ids=lambda c: "-".join(map(str, c)))
def test_decode_sweep(case):
    i, dname, B, Hq, Hkv, D, hi = case
    dtype = DTYPES[dname]
    announce(f"decode sweep {case}")
    g = torch.Generator().manual_seed(600 + i)
    lens = torch.randint(0, hi + 1, (B,), generator=g, dtype=torch.int32)
    Smax = hi + 3
    q = seeded((B, 1, Hq, D), 700 + i, dtype)
    kn = seeded((B, 1, Hkv, D), 800 + i, dtype)
    vn = seeded((B, 1, Hkv, D), 900 + i, dtype)
    kc = seeded((B, Hkv, Smax, D), 1000 + i, dtype)
    vc = seeded((B, Hkv, Smax, D), 1100 + i, dtype)
    cos, sin = ref.rope_tables(D, Smax, 5e5)
    kcd, vcd = kc.to(DEV), vc.to(DEV)
    out = ops.decode_raw(q.to(DEV), kn.to(DEV), vn.to(DEV), kcd, vcd, lens.to(DEV), cos.to(DEV),
                         sin.to(DEV), rope_row_offset=0, max_len=Smax)
    torch.cuda.synchronize()
    o_ref, kc_ref, vc_ref = ref.decode_step(q, kn, vn, kc, vc, lens, cos, sin)
    check_out(out, o_ref, TOL[dtype], "decode out")
    assert torch.equal(kcd.cpu(), kc_ref) and torch.equal(vcd.cpu(), vc_ref)


def _draw_f32_cases(n, seed=4242):
    rng = random.Random(seed)
    cases = []
    for i in range(n):
        D = rng.choice([64, 128])
        Hkv = rng.choice([1, 2, 4])
        n_rep = rng.choice([1, 2, 3, 4, 5, 8, 16, 32])
        B = rng.choice([1, 2, 3])
        S = rng.choice([1, 2, 31, 33, 63, 65, 127, 129, 191, 255, 257, 300, 383, 448, 511,
                        513, 640, 700])
        mask = rng.choice([None, None, "doc", "kpm"])
        causal = True if mask else rng.random() < 0.75
        cases.append((i, "fp32", B, S, Hkv * n_rep, Hkv, D, causal, mask))
    return cases


@pytest.mark.parametrize("case", _draw_f32_cases(24), ids=lambda c: "-".join(map(str, c)))
def test_fp32_sweep(case):
    """float32 on the fp32 matrix-core kernels: out, LSE and every gradient
    element within 1e-5 of the float64 oracle (nothing below float32 is
    rounded, so no operand allowance), the autograd and the raw backward the
    same bits."""
    i, _, B, S, Hq, Hkv, D, causal, mask = case
    dtype = torch.float32
    announce(f"fp32 sweep {case}")
    q = seeded((B, S, Hq, D), 1300 + i, dtype)
    k = seeded((B, S, Hkv, D), 1400 + i, dtype)
    v = seeded((B, S, Hkv, D), 1500 + i, dtype)
    do = seeded((B, S, Hq, D), 1600 + i, dtype)
    cos, sin = ref.rope_tables(D, S, 5e5)
    m = _mask_tensors(case, 1700 + i)
    md = {n: t.to(DEV) for n, t in m.items()}
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    out = ops.attention(qd, kd, vd, cos.to(DEV), sin.to(DEV), causal=causal, **md)
    out.backward(do.to(DEV))
    _, lse = ops.fwd_raw(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV),
                         causal=causal, k_rotated=False, **md)
    raw = ops.bwd_raw(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV), out.detach(),
                      lse, do.to(DEV), causal=causal, **md)
    torch.cuda.synchronize()
    o_ref, l_ref = ref.attention_fwd(q, k, v, cos, sin, causal=causal, **m)
    check_out(out, o_ref, TOL[dtype], "out")
    check_out(lse, l_ref, TOL[dtype], "lse")
    grads = ref.attention_bwd(q, k, v, cos, sin, do, causal=causal, **m)
    for got, want, name in zip((qd.grad, kd.grad, vd.grad), grads, ("dq", "dk", "dv")):
        check_grad(got, want, dtype, name, group=Hq // Hkv if name != "dq" else 1)
    for a, b in zip(raw, (qd.grad, kd.grad, vd.grad)):
        assert torch.equal(a, b)


@pytest.mark.parametrize("case", [(i, "fp32", *c[2:]) for i, c in
                                  enumerate(_draw_decode_cases(8, seed=91))],
                         ids=lambda c: "-".join(map(str, c)))
def test_fp32_decode_sweep(case):
    i, _, B, Hq, Hkv, D, hi = case
    dtype = torch.float32
    announce(f"fp32 decode sweep {case}")
    g = torch.Generator().manual_seed(1800 + i)
    lens = torch.randint(0, hi + 1, (B,), generator=g, dtype=torch.int32)
    Smax = hi + 3
    q = seeded((B, 1, Hq, D), 1900 + i, dtype)
    kn = seeded((B, 1, Hkv, D), 2000 + i, dtype)
    vn = seeded((B, 1, Hkv, D), 2100 + i, dtype)
    kc = seeded((B, Hkv, Smax, D), 2200 + i, dtype)
    vc = seeded((B, Hkv, Smax, D), 2300 + i, dtype)
    cos, sin = ref.rope_tables(D, Smax, 5e5)
    kcd, vcd = kc.to(DEV), vc.to(DEV)
    out = ops.decode_raw(q.to(DEV), kn.to(DEV), vn.to(DEV), kcd, vcd, lens.to(DEV), cos.to(DEV),
                         sin.to(DEV), rope_row_offset=0, max_len=Smax)
    torch.cuda.synchronize()
    o_ref, kc_ref, vc_ref = ref.decode_step(q, kn, vn, kc, vc, lens, cos, sin)
    check_out(out, o_ref, TOL[dtype], "decode out")
    assert torch.equal(kcd.cpu(), kc_ref) and torch.equal(vcd.cpu(), vc_ref)
