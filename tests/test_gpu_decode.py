"""GPU parity of the KV-cache decode (kf_attn_decode) and cache append."""

from __future__ import annotations

import pytest
import torch

import make_fixtures as mf
from gpu_util import DEV, announce, load_fixture, max_abs, seeded
from kempnerforge_amd import ops
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu


def _decode(q, kn, vn, kc, vc, lens, cos, sin, max_len):
    kcd, vcd = kc.to(DEV), vc.to(DEV)
    out = ops.decode_raw(q.to(DEV), kn.to(DEV), vn.to(DEV), kcd, vcd, lens.to(DEV),
                         cos.to(DEV), sin.to(DEV), rope_row_offset=0, max_len=max_len)
    torch.cuda.synchronize()
    return out, kcd, vcd


def test_fixture():
    announce("decode fixture")
    fx = load_fixture("decode_bf16")
    q, kn, vn, kc, vc, lens, cos, sin = mf.decode_inputs(**mf.DECODE_CASE)
    out, kcd, vcd = _decode(q, kn, vn, kc, vc, lens, cos, sin, mf.DECODE_CASE["Smax"])
    assert max_abs(out, torch.from_numpy(fx["out"])) <= 2e-2
    b = torch.arange(lens.numel())
    # the rotated key written into the cache is bit-exact (eager bf16 rounding)
    written = kcd.cpu()[b, :, lens.long()].float()
    assert torch.equal(written, torch.from_numpy(fx["k_written"]))
    assert torch.equal(vcd.cpu()[b, :, lens.long()], vn[:, 0])


@pytest.mark.parametrize("cfg", [
    # dtype, B, Hq, Hkv, D, lo, hi, Smax
    (torch.bfloat16, 3, 8, 8, 64, 1, 300, 400),      # MHA fast path, D=64
    (torch.bfloat16, 2, 16, 2, 128, 255, 257, 300),  # sub-split lengths
    (torch.bfloat16, 6, 16, 2, 128, 1022, 1025, 1100),  # split boundaries (1024 keys)
    (torch.bfloat16, 40, 8, 2, 64, 900, 3100, 3200),  # longest-first split order (B <= 64)
    (torch.bfloat16, 70, 8, 2, 64, 900, 2200, 2300),  # plain split order (B > 64)
    (torch.bfloat16, 2, 8, 1, 128, 0, 3, 8),         # empty cache (len 0) and tiny
    (torch.bfloat16, 2, 6, 2, 128, 10, 90, 100),     # n_rep 3 (padded MFMA columns)
    (torch.bfloat16, 2, 16, 1, 128, 500, 700, 800),  # n_rep 16, the widest fast case
    (torch.bfloat16, 2, 32, 1, 128, 500, 700, 800),  # n_rep 32 -> generic kernel
    (torch.bfloat16, 1, 64, 8, 128, 1000, 1300, 1400),  # 70B heads, n_rep 8
    (torch.bfloat16, 2, 64, 1, 64, 10, 90, 100),     # n_rep 64 -> generic kernel
    (torch.float32, 2, 4, 2, 64, 10, 90, 100),       # fp32 matrix-core decode
    (torch.float32, 2, 4, 2, 32, 10, 90, 100),       # fp32, D=32 -> generic kernel
    (torch.bfloat16, 2, 4, 2, 32, 10, 90, 100),      # D=32 -> generic kernel
], ids=lambda c: "-".join(map(str, c)))
def test_shapes(cfg):
    dtype, B, Hq, Hkv, D, lo, hi, Smax = cfg
    announce(f"decode {cfg}")
    g = torch.Generator().manual_seed(4)
    lens = torch.randint(lo, hi + 1, (B,), generator=g, dtype=torch.int32)
    q = seeded((B, 1, Hq, D), 0, dtype)
    kn = seeded((B, 1, Hkv, D), 1, dtype)
    vn = seeded((B, 1, Hkv, D), 2, dtype)
    kc = seeded((B, Hkv, Smax, D), 5, dtype)
    vc = seeded((B, Hkv, Smax, D), 6, dtype)
    cos, sin = ref.rope_tables(D, Smax, 5e5)
    out, kcd, vcd = _decode(q, kn, vn, kc, vc, lens, cos, sin, int(lens.max()) + 1)
    o_ref, kc_ref, vc_ref = ref.decode_step(q, kn, vn, kc, vc, lens, cos, sin)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert max_abs(out, o_ref) <= tol
    assert torch.equal(kcd.cpu(), kc_ref) and torch.equal(vcd.cpu(), vc_ref)


def test_llama8b_decode_config():
    """C4: B=32, Hq=32, Hkv=8, D=128, L_b ~ U[1024, 8192] from seed 4."""
    B, Hq, Hkv, D = 32, 32, 8, 128
    announce("decode C4")
    g = torch.Generator().manual_seed(4)
    lens = torch.randint(1024, 8192 + 1, (B,), generator=g, dtype=torch.int32)
    Smax = 8193
    q = seeded((B, 1, Hq, D), 0, torch.bfloat16)
    kn = seeded((B, 1, Hkv, D), 1, torch.bfloat16)
    vn = seeded((B, 1, Hkv, D), 2, torch.bfloat16)
    kc = seeded((B, Hkv, Smax, D), 5, torch.bfloat16)
    vc = seeded((B, Hkv, Smax, D), 6, torch.bfloat16)
    cos, sin = ref.rope_tables(D, Smax, 5e5)
    out, kcd, _ = _decode(q, kn, vn, kc, vc, lens, cos, sin, Smax)
    sel = [0, 5, 17, 31]
    o_ref, kc_ref, _ = ref.decode_step(q[sel], kn[sel], vn[sel], kc[sel], vc[sel], lens[sel],
                                       cos, sin)
    assert max_abs(out.cpu()[sel], o_ref) <= 2e-2
    for i, b in enumerate(sel):
        L = int(lens[b])
        assert torch.equal(kcd[b, :, L].cpu(), kc_ref[i, :, L])


def test_cache_append_bit_exact():
    announce("cache append")
    B, S, Hkv, D, Smax, start = 2, 37, 4, 128, 64, 9
    kn = seeded((B, S, Hkv, D), 1, torch.bfloat16)
    vn = seeded((B, S, Hkv, D), 2, torch.bfloat16)
    cos, sin = ref.rope_tables(D, Smax, 5e5)
    kc = torch.zeros(B, Hkv, Smax, D, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    c, s = cos[start:start + S], sin[start:start + S]
    ops.cache_append_raw(kn.to(DEV), vn.to(DEV), c.to(DEV), s.to(DEV), kc, vc, start)
    torch.cuda.synchronize()
    want = ref.apply_rope(kn.transpose(1, 2), c, s)
    assert torch.equal(kc.cpu()[:, :, start:start + S], want)
    assert torch.equal(vc.cpu()[:, :, start:start + S], vn.transpose(1, 2))
    assert (kc.cpu()[:, :, :start] == 0).all() and (kc.cpu()[:, :, start + S:] == 0).all()


def test_stale_rows_are_not_read():
    """Cache rows past each sequence's length hold NaN; the output and the
    written rows must not see them (the reference reads rows <= len only)."""
    B, Hq, Hkv, D, Smax = 3, 8, 2, 128, 700
    announce("decode stale NaN rows")
    lens = torch.tensor([0, 255, 600], dtype=torch.int32)
    q = seeded((B, 1, Hq, D), 0, torch.bfloat16)
    kn = seeded((B, 1, Hkv, D), 1, torch.bfloat16)
    vn = seeded((B, 1, Hkv, D), 2, torch.bfloat16)
    kc = seeded((B, Hkv, Smax, D), 5, torch.bfloat16)
    vc = seeded((B, Hkv, Smax, D), 6, torch.bfloat16)
    for b in range(B):
        kc[b, :, int(lens[b]):] = float("nan")
        vc[b, :, int(lens[b]):] = float("nan")
    cos, sin = ref.rope_tables(D, Smax, 5e5)
    out, kcd, vcd = _decode(q, kn, vn, kc, vc, lens, cos, sin, Smax)
    o_ref, kc_ref, vc_ref = ref.decode_step(q, kn, vn, kc, vc, lens, cos, sin)
    assert torch.isfinite(out.cpu().float()).all()
    assert max_abs(out, o_ref) <= 2e-2
    for b in range(B):
        L = int(lens[b]) + 1
        assert torch.equal(kcd.cpu()[b, :, :L], kc_ref[b, :, :L])
        assert torch.equal(vcd.cpu()[b, :, :L], vc_ref[b, :, :L])


def test_consecutive_steps_and_bad_length():
    """Three decode steps in a row on the same caches and a fresh workspace
    each (nothing one call leaves behind may change the next one's result),
    then one sequence with an out-of-range length (NaN output, caches
    untouched)."""
    B, Hq, Hkv, D, Smax = 3, 8, 2, 128, 1200
    announce("decode consecutive steps")
    cos, sin = ref.rope_tables(D, Smax, 5e5)
    kc = seeded((B, Hkv, Smax, D), 5, torch.bfloat16)
    vc = seeded((B, Hkv, Smax, D), 6, torch.bfloat16)
    kcd, vcd = kc.to(DEV), vc.to(DEV)
    lens = torch.tensor([700, 1023, 5], dtype=torch.int32)
    for step in range(3):
        q = seeded((B, 1, Hq, D), 10 + step, torch.bfloat16)
        kn = seeded((B, 1, Hkv, D), 20 + step, torch.bfloat16)
        vn = seeded((B, 1, Hkv, D), 30 + step, torch.bfloat16)
        o_ref, kc, vc = ref.decode_step(q, kn, vn, kc, vc, lens, cos, sin)
        out = ops.decode_raw(q.to(DEV), kn.to(DEV), vn.to(DEV), kcd, vcd, lens.to(DEV),
                             cos.to(DEV), sin.to(DEV), rope_row_offset=0, max_len=1100)
        torch.cuda.synchronize()
        assert max_abs(out, o_ref) <= 2e-2
        assert torch.equal(kcd.cpu(), kc) and torch.equal(vcd.cpu(), vc)
        lens = lens + 1
    # lens[1] + 1 > max_len: that sequence gets NaN and no cache write
    lens = torch.tensor([10, 1100, 20], dtype=torch.int32)
    q = seeded((B, 1, Hq, D), 40, torch.bfloat16)
    kn = seeded((B, 1, Hkv, D), 41, torch.bfloat16)
    vn = seeded((B, 1, Hkv, D), 42, torch.bfloat16)
    before = kcd.clone()
    out = ops.decode_raw(q.to(DEV), kn.to(DEV), vn.to(DEV), kcd, vcd, lens.to(DEV),
                         cos.to(DEV), sin.to(DEV), rope_row_offset=0, max_len=1100)
    torch.cuda.synchronize()
    assert torch.isnan(out[1].float()).all()
    assert torch.isfinite(out[0].float()).all() and torch.isfinite(out[2].float()).all()
    assert torch.equal(kcd[1], before[1])
