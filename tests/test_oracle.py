"""Pin the CPU oracle (oracle/attention_ref.py) before trusting it.

Every check compares the oracle with something other than a retyping of its own
formula: scalar Python loops with explicit rounding, PyTorch's library SDPA,
finite differences, closed forms and invariants.  Invariant checks taken from
the reference's own tests cite them.  Each block names the mistakes it would
catch.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention_ref as ref

torch.set_num_threads(min(8, torch.get_num_threads()))


def _bf16(x: float) -> float:
    return float(torch.tensor(x, dtype=torch.float32).to(torch.bfloat16).float())


def _f32(x: float) -> float:
    return float(np.float32(x))


def _f16(x: float) -> float:
    return float(np.float16(np.float32(x)))


# --------------------------------------------------------------------------- RoPE tables
class TestRopeTables:
    # reference tests/unit/test_model.py:67-106
    def test_shape_and_dtype(self):
        cos, sin = ref.rope_tables(128, 256, 10000.0)
        assert cos.shape == (256, 64) and sin.shape == (256, 64)
        assert cos.dtype == torch.float32

    def test_unit_magnitude_and_identity_at_zero(self):
        cos, sin = ref.rope_tables(64, 128)
        assert torch.allclose(cos.pow(2) + sin.pow(2), torch.ones_like(cos), atol=1e-5)
        assert torch.allclose(cos[0], torch.ones(32)) and torch.allclose(sin[0], torch.zeros(32))

    @pytest.mark.parametrize("D,theta", [(64, 1e4), (128, 5e5)])
    def test_closed_form(self, D, theta):
        # catches: wrong exponent (2i/D vs i/D), theta applied to the wrong side,
        # swapped cos/sin, a position offset.
        S = 300
        cos, sin = ref.rope_tables(D, S, theta)
        i = np.arange(D // 2, dtype=np.float64)
        inv64 = theta ** (-2.0 * i / D)
        angles = np.arange(S, dtype=np.float64)[:, None] * inv64[None, :]
        # float32 angle rounding grows with position: |err| <= S * inv * 2^-23
        tol = S * 2.0 ** -23 + 1e-6
        assert np.abs(cos.double().numpy() - np.cos(angles)).max() < tol
        assert np.abs(sin.double().numpy() - np.sin(angles)).max() < tol


# --------------------------------------------------------------------------- apply_rope
class TestApplyRope:
    def test_scalar_loop_bf16_rounding(self):
        # catches: interleaved instead of half-split pairing, sign errors, a
        # missing cast of the tables to bf16, a missing per-op rounding.
        g = torch.Generator().manual_seed(11)
        S, D = 5, 8
        cos, sin = ref.rope_tables(D, S, 10000.0)
        x = torch.randn(1, 1, S, D, generator=g).bfloat16()
        got = ref.apply_rope(x, cos, sin).float()
        d = D // 2
        for s in range(S):
            for j in range(d):
                c, sn = _bf16(float(cos[s, j])), _bf16(float(sin[s, j]))
                x1, x2 = float(x[0, 0, s, j]), float(x[0, 0, s, j + d])
                r1 = _bf16(_f32(_bf16(x1 * c) - _bf16(x2 * sn)))
                r2 = _bf16(_f32(_bf16(x2 * c) + _bf16(x1 * sn)))
                assert float(got[0, 0, s, j]) == r1
                assert float(got[0, 0, s, j + d]) == r2

    def test_scalar_loop_fp16_rounding(self):
        # the same for float16 (the reference's mixed_precision = "fp16"): the
        # tables cast to fp16 and every product and sum rounded to fp16
        g = torch.Generator().manual_seed(14)
        S, D = 5, 8
        cos, sin = ref.rope_tables(D, S, 10000.0)
        x = torch.randn(1, 1, S, D, generator=g).half()
        got = ref.apply_rope(x, cos, sin).float()
        d = D // 2
        for s in range(S):
            for j in range(d):
                c, sn = _f16(float(cos[s, j])), _f16(float(sin[s, j]))
                x1, x2 = float(x[0, 0, s, j]), float(x[0, 0, s, j + d])
                r1 = _f16(_f32(_f16(x1 * c) - _f16(x2 * sn)))
                r2 = _f16(_f32(_f16(x2 * c) + _f16(x1 * sn)))
                assert float(got[0, 0, s, j]) == r1
                assert float(got[0, 0, s, j + d]) == r2

    def test_scalar_loop_fp32(self):
        g = torch.Generator().manual_seed(12)
        S, D = 4, 6
        cos, sin = ref.rope_tables(D, S, 10000.0)
        x = torch.randn(1, 2, S, D, generator=g)
        got = ref.apply_rope(x, cos, sin)
        d = D // 2
        for h in range(2):
            for s in range(S):
                for j in range(d):
                    c, sn = float(cos[s, j]), float(sin[s, j])
                    x1, x2 = float(x[0, h, s, j]), float(x[0, h, s, j + d])
                    r1 = _f32(_f32(x1 * c) - _f32(x2 * sn))
                    r2 = _f32(_f32(x2 * c) + _f32(x1 * sn))
                    assert float(got[0, h, s, j]) == r1
                    assert float(got[0, h, s, j + d]) == r2

    def test_rotation_invariants_fp64(self):
        # pair norms are preserved; rotating by a then by b equals rotating by a+b
        g = torch.Generator().manual_seed(13)
        D, S = 16, 9
        x = torch.randn(2, 3, S, D, generator=g, dtype=torch.float64)
        a = torch.rand(S, D // 2, generator=g, dtype=torch.float64) * 6
        b = torch.rand(S, D // 2, generator=g, dtype=torch.float64) * 6
        ra = ref.apply_rope(x, a.cos(), a.sin())
        rab = ref.apply_rope(ra, b.cos(), b.sin())
        direct = ref.apply_rope(x, (a + b).cos(), (a + b).sin())
        assert torch.allclose(rab, direct, atol=1e-12)
        n0 = x[..., : D // 2] ** 2 + x[..., D // 2:] ** 2
        n1 = ra[..., : D // 2] ** 2 + ra[..., D // 2:] ** 2
        assert torch.allclose(n0, n1, atol=1e-12)

    def test_position_zero_is_identity(self):
        # reference tests/unit/test_model.py:101-106
        cos, sin = ref.rope_tables(64, 4)
        x = torch.randn(1, 1, 1, 64)
        assert torch.allclose(ref.apply_rope(x, cos[:1], sin[:1]), x, atol=1e-5)

    def test_inverse_is_adjoint(self):
        # <rope(x), g> == <x, rope_bwd(g)> for fp64 (catches a sign/transposition
        # error in the RoPE backward)
        g = torch.Generator().manual_seed(14)
        D, S = 12, 7
        cos, sin = ref.rope_tables(D, S, 10000.0)
        x = torch.randn(1, 2, S, D, generator=g, dtype=torch.float64)
        gr = torch.randn(1, 2, S, D, generator=g, dtype=torch.float64)
        lhs = (ref.apply_rope(x, cos.double(), sin.double()) * gr).sum()
        rhs = (x * ref.rotate_half_inverse(gr, cos.double(), sin.double(), torch.float64)).sum()
        assert abs(float(lhs - rhs)) < 1e-12


# --------------------------------------------------------------------------- forward
def _inputs(B, S, Hq, Hkv, D, dtype, seed=0, theta=10000.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, S, Hq, D, generator=g).to(dtype)
    k = torch.randn(B, S, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B, S, Hkv, D, generator=g).to(dtype)
    cos, sin = ref.rope_tables(D, S, theta)
    return q, k, v, cos, sin


def _sdpa_reference(q, k, v, cos, sin, causal=True):
    """The reference's composition with PyTorch's library SDPA in float64."""
    qr = ref.apply_rope(q.transpose(1, 2), cos, sin).double()
    kr = ref.apply_rope(k.transpose(1, 2), cos, sin).double()
    vt = v.transpose(1, 2).double()
    n_rep = q.shape[2] // k.shape[2]
    kr = kr.repeat_interleave(n_rep, dim=1)
    vt = vt.repeat_interleave(n_rep, dim=1)
    return F.scaled_dot_product_attention(qr, kr, vt, is_causal=causal).transpose(1, 2)


class TestForward:
    @pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
    @pytest.mark.parametrize("Hq,Hkv", [(4, 4), (4, 2), (8, 1)])
    def test_matches_library_sdpa(self, dtype, Hq, Hkv):
        q, k, v, cos, sin = _inputs(2, 33, Hq, Hkv, 16, dtype)
        out, _ = ref.attention_fwd(q, k, v, cos, sin)
        assert torch.allclose(out, _sdpa_reference(q, k, v, cos, sin), atol=1e-12)

    def test_noncausal_matches_library_sdpa(self):
        q, k, v, cos, sin = _inputs(1, 17, 4, 2, 8, torch.float32)
        out, _ = ref.attention_fwd(q, k, v, cos, sin, causal=False)
        assert torch.allclose(out, _sdpa_reference(q, k, v, cos, sin, causal=False), atol=1e-12)

    def test_brute_force_scalar(self):
        # catches: GQA head map h % Hkv instead of h // n_rep (distinct kv heads),
        # a missing scale, a mask aligned bottom-right, a wrong LSE base.
        B, S, Hq, Hkv, D = 1, 5, 4, 2, 4
        q, k, v, cos, sin = _inputs(B, S, Hq, Hkv, D, torch.float64, seed=3)
        out, lse = ref.attention_fwd(q, k, v, cos.double(), sin.double())
        d = D // 2

        def rot(x, s):
            c = [math.cos(s * 10000.0 ** (-2 * j / D)) for j in range(d)]
            sn = [math.sin(s * 10000.0 ** (-2 * j / D)) for j in range(d)]
            return [x[j] * c[j] - x[j + d] * sn[j] for j in range(d)] + \
                   [x[j + d] * c[j] + x[j] * sn[j] for j in range(d)]

        n_rep = Hq // Hkv
        for h in range(Hq):
            g = h // n_rep
            for i in range(S):
                qi = rot(q[0, i, h].tolist(), i)
                sc = []
                for j in range(i + 1):
                    kj = rot(k[0, j, g].tolist(), j)
                    sc.append(sum(a * b for a, b in zip(qi, kj)) / math.sqrt(D))
                lse_i = ref.logsumexp_closed_form(sc)
                assert abs(float(lse[0, h, i]) - lse_i) < 1e-6
                w = [math.exp(s_ - lse_i) for s_ in sc]
                for dd in range(D):
                    o = sum(w[j] * float(v[0, j, g, dd]) for j in range(i + 1))
                    assert abs(float(out[0, i, h, dd]) - o) < 1e-6

    def test_zero_query_closed_form(self):
        # q = 0: all scores 0, so lse_i = log(i+1) and out_i = mean(v_0..v_i)
        B, S, Hq, Hkv, D = 1, 20, 2, 1, 8
        _, k, v, cos, sin = _inputs(B, S, Hq, Hkv, D, torch.float64, seed=5)
        q = torch.zeros(B, S, Hq, D, dtype=torch.float64)
        out, lse = ref.attention_fwd(q, k, v, cos.double(), sin.double())
        i = torch.arange(S, dtype=torch.float64)
        assert torch.allclose(lse[0, 0], torch.log(i + 1), atol=1e-12)
        mean = v[0, :, 0].cumsum(0) / (i + 1)[:, None]
        assert torch.allclose(out[0, :, 1], mean, atol=1e-12)

    def test_lse_normalises(self):
        q, k, v, cos, sin = _inputs(1, 24, 2, 2, 8, torch.float32)
        _, lse = ref.attention_fwd(q, k, v, cos, sin)
        _, p = ref.capture(q, k, v, cos, sin)
        s = torch.log(p.clamp_min(1e-300)) + lse.unsqueeze(-1)  # = scores where p > 0
        assert torch.allclose(p.sum(-1), torch.ones_like(lse), atol=1e-12)
        assert torch.isfinite(s[p > 0]).all()

    @pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
    def test_rows_subset_equals_full(self, dtype):
        q, k, v, cos, sin = _inputs(2, 40, 8, 2, 16, dtype, seed=23)
        out, lse = ref.attention_fwd(q, k, v, cos, sin)
        rows, heads = torch.tensor([0, 7, 39, 21]), torch.tensor([1, 6, 3])
        o2, l2 = ref.attention_fwd_rows(q, k, v, cos, sin, rows, heads=heads)
        assert torch.allclose(o2, out[:, rows][:, :, heads], atol=1e-12)
        assert torch.allclose(l2, lse[:, heads][:, :, rows], atol=1e-12)

    def test_rotated_cache_fwd_matches_sdpa_top_left(self):
        # multi-token forward over a cache with Sq < Sk: SDPA's is_causal aligns
        # top-left (the reference quirk at kempnerforge/model/attention.py:229)
        g = torch.Generator().manual_seed(21)
        B, Sq, Sk, Hq, Hkv, D = 1, 6, 10, 4, 2, 8
        q = torch.randn(B, Sq, Hq, D, generator=g)
        kc = torch.randn(B, Hkv, Sk, D, generator=g)
        vc = torch.randn(B, Hkv, Sk, D, generator=g)
        cos, sin = ref.rope_tables(D, Sq, 1e4)
        out, _ = ref.attention_fwd_rotated(q, kc, vc, cos, sin, causal=True)
        qr = ref.apply_rope(q.transpose(1, 2), cos, sin).double()
        kk = kc.repeat_interleave(2, dim=1).double()
        vv = vc.repeat_interleave(2, dim=1).double()
        want = F.scaled_dot_product_attention(qr, kk, vv, is_causal=True).transpose(1, 2)
        assert torch.allclose(out, want, atol=1e-12)


# --------------------------------------------------------------------------- backward
class TestBackward:
    def test_finite_differences(self):
        # central differences of L = <out, dO> through the oracle forward (which
        # is pinned above); catches a missing group sum, a missing RoPE backward
        # or a transposed rotation, a wrong softmax Jacobian.
        B, S, Hq, Hkv, D = 1, 6, 4, 2, 4
        q, k, v, cos, sin = _inputs(B, S, Hq, Hkv, D, torch.float64, seed=7)
        cos, sin = cos.double(), sin.double()
        do = torch.randn(B, S, Hq, D, generator=torch.Generator().manual_seed(8),
                         dtype=torch.float64)
        dq, dk, dv = ref.attention_bwd(q, k, v, cos, sin, do)

        def loss(qq, kk, vv):
            return float((ref.attention_fwd(qq, kk, vv, cos, sin)[0] * do).sum())

        h = 1e-6
        for name, t, grad in (("q", q, dq), ("k", k, dk), ("v", v, dv)):
            flat = t.view(-1)
            gflat = grad.reshape(-1)
            for idx in range(0, flat.numel(), 3):
                old = float(flat[idx])
                flat[idx] = old + h
                lp = loss(q, k, v)
                flat[idx] = old - h
                lm = loss(q, k, v)
                flat[idx] = old
                fd = (lp - lm) / (2 * h)
                assert abs(fd - float(gflat[idx])) < 1e-6, (name, idx)

    def test_matches_library_autograd(self):
        # autograd through the literal reference composition (fp64, so RoPE has
        # no rounding): apply_rope -> repeat_interleave -> SDPA
        B, S, Hq, Hkv, D = 2, 19, 8, 2, 16
        q, k, v, cos, sin = _inputs(B, S, Hq, Hkv, D, torch.float64, seed=9)
        cos, sin = cos.double(), sin.double()
        do = torch.randn(B, S, Hq, D, generator=torch.Generator().manual_seed(10),
                         dtype=torch.float64)
        qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
        out = _sdpa_reference(qq, kk, vv, cos, sin)
        out.backward(do)
        dq, dk, dv = ref.attention_bwd(q, k, v, cos, sin, do)
        assert torch.allclose(dq, qq.grad, atol=1e-10)
        assert torch.allclose(dk, kk.grad, atol=1e-10)
        assert torch.allclose(dv, vv.grad, atol=1e-10)


    @pytest.mark.parametrize("mask", [None, "noncausal", "doc", "kpm"])
    def test_rounded_operands_without_rounding_equal_autograd(self, mask):
        # the closed-form restatement (no rounding) against autograd of the
        # pinned forward, masks and NaN guard included: catches a wrong
        # Delta, a missing group sum or scale, a transposed dS
        B, S, Hq, Hkv, D = 2, 23, 6, 2, 16
        q, k, v, cos, sin = _inputs(B, S, Hq, Hkv, D, torch.bfloat16, seed=31)
        do = torch.randn(B, S, Hq, D, generator=torch.Generator().manual_seed(32)).bfloat16()
        kw = {}
        if mask == "doc":
            kw["doc_ids"] = torch.tensor([[0] * 9 + [1] * 14, [0] * 3 + [1] * 20])
        elif mask == "kpm":
            kpm = torch.ones(B, S, dtype=torch.bool)
            kpm[0, :5] = False
            kpm[1, 10:15] = False
            kw["key_padding_mask"] = kpm
        causal = mask != "noncausal"
        want = ref.attention_bwd(q, k, v, cos, sin, do, causal=causal, **kw)
        got = ref.attention_bwd_rounded_operands(q, k, v, cos, sin, do, operand_dtype=None,
                                                 causal=causal, **kw)
        for g, w in zip(got, want):
            assert torch.allclose(g, w, atol=1e-10, rtol=0)

    def test_rounded_operands_scalar_loop(self):
        # brute force on one head: P and dS rounded to bf16, O as stored in bf16,
        # everything else exact (catches rounding at the wrong point, e.g. dS
        # formed from the unrounded P or rounded before the product)
        S, D = 4, 2
        q, k, v, cos, sin = _inputs(1, S, 1, 1, D, torch.bfloat16, seed=33)
        do = torch.randn(1, S, 1, D, generator=torch.Generator().manual_seed(34)).bfloat16()
        got = ref.attention_bwd_rounded_operands(q, k, v, cos, sin, do,
                                                 operand_dtype=torch.bfloat16)
        qr = ref.apply_rope(q.transpose(1, 2), cos, sin)[0, 0].double().tolist()
        kr = ref.apply_rope(k.transpose(1, 2), cos, sin)[0, 0].double().tolist()
        vv = v[0, :, 0].double().tolist()
        dd = do[0, :, 0].double().tolist()
        sc = D ** -0.5
        dqr = [[0.0] * D for _ in range(S)]
        dkr = [[0.0] * D for _ in range(S)]
        dv = [[0.0] * D for _ in range(S)]
        for i in range(S):
            s = [sum(qr[i][d] * kr[j][d] for d in range(D)) * sc for j in range(i + 1)]
            m = max(s)
            z = sum(math.exp(x - m) for x in s)
            p = [math.exp(x - m) / z for x in s]
            o = [_bf16(sum(p[j] * vv[j][d] for j in range(i + 1))) for d in range(D)]
            delta = sum(dd[i][d] * o[d] for d in range(D))
            for j in range(i + 1):
                pr = _bf16(p[j])
                dp = sum(dd[i][d] * vv[j][d] for d in range(D))
                ds = _bf16(pr * (dp - delta))
                for d in range(D):
                    dv[j][d] += pr * dd[i][d]
                    dqr[i][d] += ds * kr[j][d] * sc
                    dkr[j][d] += ds * qr[i][d] * sc
        want_dv = torch.tensor(dv, dtype=torch.float64)
        assert torch.allclose(got[2][0, :, 0], want_dv, atol=1e-12, rtol=0)
        dq = ref.rotate_half_inverse(torch.tensor(dqr, dtype=torch.float64).view(1, 1, S, D), cos, sin,
                                     torch.bfloat16)
        dk = ref.rotate_half_inverse(torch.tensor(dkr, dtype=torch.float64).view(1, 1, S, D), cos, sin,
                                     torch.bfloat16)
        assert torch.allclose(got[0][0, :, 0], dq[0, 0], atol=1e-12, rtol=0)
        assert torch.allclose(got[1][0, :, 0], dk[0, 0], atol=1e-12, rtol=0)


# --------------------------------------------------------------------------- packed documents
def _packed_doc_ids(B, lengths_per_row):
    """[B, S] int64 document ids, contiguous increasing segments per row (what
    the packing dataset produces, kempnerforge/data/dataset.py:27-65)."""
    rows = []
    for lens in lengths_per_row:
        rows.append(torch.cat([torch.full((n,), d, dtype=torch.long) for d, n in enumerate(lens)]))
    return torch.stack(rows)


def _sdpa_doc_reference(q, k, v, cos, sin, doc_ids):
    """The reference's packed-sequence branch with PyTorch's library SDPA in
    float64: explicit bool mask causal & same-document
    (kempnerforge/model/attention.py:204-227)."""
    qr = ref.apply_rope(q.transpose(1, 2), cos, sin).double()
    kr = ref.apply_rope(k.transpose(1, 2), cos, sin).double()
    vt = v.transpose(1, 2).double()
    n_rep = q.shape[2] // k.shape[2]
    kr = kr.repeat_interleave(n_rep, dim=1)
    vt = vt.repeat_interleave(n_rep, dim=1)
    S = q.shape[1]
    causal = torch.ones(S, S, dtype=torch.bool).tril().unsqueeze(0).unsqueeze(0)
    mask = causal & (doc_ids.unsqueeze(2) == doc_ids.unsqueeze(1)).unsqueeze(1)
    mask = mask | ~mask.any(dim=-1, keepdim=True)
    return F.scaled_dot_product_attention(qr, kr, vt, attn_mask=mask).transpose(1, 2)


class TestPackedDocuments:
    def test_matches_library_sdpa_with_explicit_mask(self):
        q, k, v, cos, sin = _inputs(2, 29, 4, 2, 16, torch.bfloat16, seed=21)
        doc = _packed_doc_ids(2, [[7, 1, 13, 8], [29]])
        out, _ = ref.attention_fwd(q, k, v, cos, sin, doc_ids=doc)
        assert torch.allclose(out, _sdpa_doc_reference(q, k, v, cos, sin, doc), atol=1e-12)

    def test_equals_separate_documents(self):
        # rows of document d equal attention over that document alone (same
        # absolute RoPE positions): documents are independent
        q, k, v, cos, sin = _inputs(1, 24, 4, 1, 8, torch.float32, seed=22)
        lens = [5, 11, 8]
        doc = _packed_doc_ids(1, [lens])
        out, lse = ref.attention_fwd(q, k, v, cos, sin, doc_ids=doc)
        start = 0
        for n in lens:
            sl = slice(start, start + n)
            o_d, l_d = ref.attention_fwd(q[:, sl], k[:, sl], v[:, sl], cos[sl], sin[sl])
            assert torch.allclose(out[:, sl], o_d, atol=1e-13)
            assert torch.allclose(lse[:, :, sl], l_d, atol=1e-13)
            start += n

    def test_single_document_is_plain_causal(self):
        q, k, v, cos, sin = _inputs(2, 17, 4, 2, 8, torch.float32, seed=23)
        out_d, lse_d = ref.attention_fwd(q, k, v, cos, sin, doc_ids=torch.zeros(2, 17, dtype=torch.long))
        out, lse = ref.attention_fwd(q, k, v, cos, sin)
        assert torch.equal(out_d, out) and torch.equal(lse_d, lse)

    def test_backward_matches_library_autograd(self):
        B, S, Hq, Hkv, D = 2, 21, 4, 2, 8
        q, k, v, cos, sin = _inputs(B, S, Hq, Hkv, D, torch.float64, seed=24)
        cos, sin = cos.double(), sin.double()
        doc = _packed_doc_ids(B, [[4, 9, 8], [21]])
        do = torch.randn(B, S, Hq, D, generator=torch.Generator().manual_seed(25),
                         dtype=torch.float64)
        qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
        _sdpa_doc_reference(qq, kk, vv, cos, sin, doc).backward(do)
        dq, dk, dv = ref.attention_bwd(q, k, v, cos, sin, do, doc_ids=doc)
        assert torch.allclose(dq, qq.grad, atol=1e-10)
        assert torch.allclose(dk, kk.grad, atol=1e-10)
        assert torch.allclose(dv, vv.grad, atol=1e-10)

    def test_capture_rows_and_zeros(self):
        q, k, v, cos, sin = _inputs(1, 12, 2, 1, 8, torch.float32, seed=26)
        doc = _packed_doc_ids(1, [[5, 7]])
        _, P = ref.capture(q, k, v, cos, sin, doc_ids=doc)
        assert torch.allclose(P.sum(-1), torch.ones_like(P.sum(-1)), atol=1e-12)
        assert torch.all(P[..., 5:, :5] == 0) and torch.all(P[..., :5, 5:] == 0)


def _sdpa_masked_reference(q, k, v, cos, sin, doc_ids=None, key_padding_mask=None):
    """The reference's explicit-mask branch literally, with PyTorch's library
    SDPA in float64 (kempnerforge/model/attention.py:209-226): causal AND
    same-document AND valid key, NaN guard, attn_mask=."""
    qr = ref.apply_rope(q.transpose(1, 2), cos, sin).double()
    kr = ref.apply_rope(k.transpose(1, 2), cos, sin).double()
    vt = v.transpose(1, 2).double()
    n_rep = q.shape[2] // k.shape[2]
    kr = kr.repeat_interleave(n_rep, dim=1)
    vt = vt.repeat_interleave(n_rep, dim=1)
    B, S = q.shape[0], q.shape[1]
    mask = torch.ones(S, S, dtype=torch.bool).tril().unsqueeze(0).unsqueeze(0)
    if doc_ids is not None:
        mask = mask & (doc_ids.unsqueeze(2) == doc_ids.unsqueeze(1)).unsqueeze(1)
    if key_padding_mask is not None:
        mask = mask & key_padding_mask.view(B, 1, 1, S)
    mask = mask | ~mask.any(dim=-1, keepdim=True)
    return F.scaled_dot_product_attention(qr, kr, vt, attn_mask=mask).transpose(1, 2)


def _kpm(B, S, padded):
    """[B, S] bool key_padding_mask (True = attend) with the listed positions of
    each row padded."""
    m = torch.ones(B, S, dtype=torch.bool)
    for b, pos in enumerate(padded):
        m[b, list(pos)] = False
    return m


class TestKeyPadding:
    def test_matches_library_sdpa_with_explicit_mask(self):
        # middle frames padded, leading positions padded (guarded rows), and a
        # row with no valid key at all
        q, k, v, cos, sin = _inputs(3, 23, 4, 2, 16, torch.bfloat16, seed=31)
        kpm = _kpm(3, 23, [range(6, 11), range(0, 5), range(0, 23)])
        out, _ = ref.attention_fwd(q, k, v, cos, sin, key_padding_mask=kpm)
        want = _sdpa_masked_reference(q, k, v, cos, sin, key_padding_mask=kpm)
        assert torch.allclose(out, want, atol=1e-12)

    def test_all_valid_is_plain_causal(self):
        q, k, v, cos, sin = _inputs(2, 17, 4, 2, 8, torch.float32, seed=32)
        out_m, lse_m = ref.attention_fwd(q, k, v, cos, sin,
                                         key_padding_mask=torch.ones(2, 17, dtype=torch.bool))
        out, lse = ref.attention_fwd(q, k, v, cos, sin)
        assert torch.equal(out_m, out) and torch.equal(lse_m, lse)

    def test_guarded_rows_attend_every_key(self):
        # rows before the first valid key see no key: the guard unmasks them
        # entirely, so they equal non-causal attention over the whole sequence;
        # the other rows equal attention restricted to valid keys j <= i
        q, k, v, cos, sin = _inputs(1, 14, 2, 1, 8, torch.float32, seed=33)
        kpm = _kpm(1, 14, [[0, 1, 2, 3, 9]])
        out, _ = ref.attention_fwd(q, k, v, cos, sin, key_padding_mask=kpm)
        full, _ = ref.attention_fwd(q, k, v, cos, sin, causal=False)
        assert torch.allclose(out[:, :4], full[:, :4], atol=1e-13)
        keep = [j for j in range(14) if j not in (0, 1, 2, 3, 9)]
        qr, kr, vt = ref._rotated_bhsd(q, k, v, cos, sin)
        kr, vt = kr[:, :, keep].double(), vt[:, :, keep].double()
        for i in range(4, 14):
            cols = [c for c, j in enumerate(keep) if j <= i]
            s = (qr[:, :, i:i + 1].double() @ kr[:, :, cols].transpose(-1, -2)) * 8 ** -0.5
            o = torch.softmax(s, -1) @ vt[:, :, cols]
            assert torch.allclose(out[:, i], o[:, :, 0], atol=1e-13)

    def test_with_documents(self):
        q, k, v, cos, sin = _inputs(2, 26, 4, 2, 8, torch.float32, seed=34)
        doc = _packed_doc_ids(2, [[9, 6, 11], [26]])
        kpm = _kpm(2, 26, [[9, 10, 11, 20], [0, 1, 2]])
        out, _ = ref.attention_fwd(q, k, v, cos, sin, doc_ids=doc, key_padding_mask=kpm)
        want = _sdpa_masked_reference(q, k, v, cos, sin, doc, kpm)
        assert torch.allclose(out, want, atol=1e-12)

    def test_backward_matches_library_autograd(self):
        B, S, Hq, Hkv, D = 2, 19, 4, 2, 8
        q, k, v, cos, sin = _inputs(B, S, Hq, Hkv, D, torch.float64, seed=35)
        cos, sin = cos.double(), sin.double()
        kpm = _kpm(B, S, [range(0, 4), [5, 6, 12]])
        do = torch.randn(B, S, Hq, D, generator=torch.Generator().manual_seed(36),
                         dtype=torch.float64)
        qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
        _sdpa_masked_reference(qq, kk, vv, cos, sin, key_padding_mask=kpm).backward(do)
        dq, dk, dv = ref.attention_bwd(q, k, v, cos, sin, do, key_padding_mask=kpm)
        assert torch.allclose(dq, qq.grad, atol=1e-10)
        assert torch.allclose(dk, kk.grad, atol=1e-10)
        assert torch.allclose(dv, vv.grad, atol=1e-10)

    def test_capture_zeros_padded_keys(self):
        q, k, v, cos, sin = _inputs(1, 12, 2, 1, 8, torch.float32, seed=37)
        kpm = _kpm(1, 12, [[0, 1, 7]])
        _, P = ref.capture(q, k, v, cos, sin, key_padding_mask=kpm)
        assert torch.allclose(P.sum(-1), torch.ones_like(P.sum(-1)), atol=1e-12)
        assert torch.all(P[..., 2:, 0:2] == 0) and torch.all(P[..., 2:, 7] == 0)
        assert torch.all(P[..., :2, :] > 0)  # guarded rows: every key


# --------------------------------------------------------------------------- decode
class TestDecode:
    def _setup(self, lens, Smax=24, B=3, Hq=4, Hkv=2, D=8, dtype=torch.float32):
        g = torch.Generator().manual_seed(17)
        T = Smax
        xs_q = torch.randn(B, T, Hq, D, generator=g).to(dtype)
        xs_k = torch.randn(B, T, Hkv, D, generator=g).to(dtype)
        xs_v = torch.randn(B, T, Hkv, D, generator=g).to(dtype)
        cos, sin = ref.rope_tables(D, T, 1e4)
        return xs_q, xs_k, xs_v, cos, sin

    @pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
    def test_equals_prefix_forward_row(self, dtype):
        # decoding token t after caching tokens 0..t-1 equals row t of the causal
        # forward over tokens 0..t (per sequence, ragged lengths)
        lens = torch.tensor([3, 10, 17], dtype=torch.int32)
        Smax = 24
        xq, xk, xv, cos, sin = self._setup(lens, Smax=Smax, dtype=dtype)
        B, _, Hq, D = xq.shape
        Hkv = xk.shape[2]
        kc = torch.zeros(B, Hkv, Smax, D, dtype=dtype)
        vc = torch.zeros(B, Hkv, Smax, D, dtype=dtype)
        for b in range(B):
            L = int(lens[b])
            kc[b, :, :L] = ref.apply_rope(xk[b:b + 1, :L].transpose(1, 2), cos[:L], sin[:L])[0]
            vc[b, :, :L] = xv[b, :L].transpose(0, 1)
        qn = torch.stack([xq[b, int(lens[b])] for b in range(B)])[:, None]
        kn = torch.stack([xk[b, int(lens[b])] for b in range(B)])[:, None]
        vn = torch.stack([xv[b, int(lens[b])] for b in range(B)])[:, None]
        out, kc2, vc2 = ref.decode_step(qn, kn, vn, kc, vc, lens, cos, sin)
        for b in range(B):
            L = int(lens[b])
            full, _ = ref.attention_fwd(xq[b:b + 1, : L + 1], xk[b:b + 1, : L + 1],
                                        xv[b:b + 1, : L + 1], cos[: L + 1], sin[: L + 1])
            assert torch.allclose(out[b, 0], full[0, L], atol=1e-12)
            rot = ref.apply_rope(xk[b:b + 1, : L + 1].transpose(1, 2), cos[: L + 1],
                                 sin[: L + 1])[0, :, L]
            assert torch.equal(kc2[b, :, L], rot)
            assert torch.equal(vc2[b, :, L], xv[b, L])

    def test_equal_lengths_match_reference_kvcache(self):
        # literal reference decode (kempnerforge/model/attention.py:54-70,165-175,
        # 229-231) with its scalar seq_len and library SDPA, is_causal=False
        B, Hq, Hkv, D, Smax, L = 2, 4, 2, 8, 12, 7
        g = torch.Generator().manual_seed(19)
        q = torch.randn(B, 1, Hq, D, generator=g)
        kn = torch.randn(B, 1, Hkv, D, generator=g)
        vn = torch.randn(B, 1, Hkv, D, generator=g)
        kc = torch.randn(B, Hkv, Smax, D, generator=g)
        vc = torch.randn(B, Hkv, Smax, D, generator=g)
        cos, sin = ref.rope_tables(D, Smax, 1e4)
        out, _, _ = ref.decode_step(q, kn, vn, kc, vc, torch.full((B,), L, dtype=torch.int32),
                                    cos, sin)
        c, s = cos[L:L + 1], sin[L:L + 1]
        qr = ref.apply_rope(q.transpose(1, 2), c, s)
        kr = ref.apply_rope(kn.transpose(1, 2), c, s)
        k_all = kc.clone()
        v_all = vc.clone()
        k_all[:, :, L:L + 1] = kr
        v_all[:, :, L:L + 1] = vn.transpose(1, 2)
        kk = k_all[:, :, : L + 1].repeat_interleave(2, dim=1).double()
        vv = v_all[:, :, : L + 1].repeat_interleave(2, dim=1).double()
        want = F.scaled_dot_product_attention(qr.double(), kk, vv, is_causal=False)
        assert torch.allclose(out, want.transpose(1, 2), atol=1e-12)


# --------------------------------------------------------------------------- capture
class TestCapture:
    def test_invariants(self):
        # reference tests/unit/test_hooks.py:197-234
        q, k, v, cos, sin = _inputs(2, 16, 4, 2, 16, torch.float32)
        out, p = ref.capture(q, k, v, cos, sin)
        assert p.shape == (2, 4, 16, 16)
        assert torch.allclose(p.sum(-1), torch.ones(2, 4, 16, dtype=p.dtype), atol=1e-12)
        upper = torch.triu(torch.ones(16, 16, dtype=torch.bool), diagonal=1)
        assert (p[..., upper] == 0).all()
        fwd, lse = ref.attention_fwd(q, k, v, cos, sin)
        assert torch.allclose(out, fwd, atol=1e-12)

    def test_probs_equal_exp_scores_minus_lse(self):
        q, k, v, cos, sin = _inputs(1, 12, 2, 1, 8, torch.float32)
        _, p = ref.capture(q, k, v, cos, sin)
        _, lse = ref.attention_fwd(q, k, v, cos, sin)
        qr = ref.apply_rope(q.transpose(1, 2), cos, sin).double()
        kr = ref.apply_rope(k.transpose(1, 2), cos, sin).double().repeat_interleave(2, dim=1)
        s = qr @ kr.transpose(-1, -2) / math.sqrt(8)
        tri = torch.tril(torch.ones(12, 12, dtype=torch.bool))
        assert torch.allclose(p[..., tri], torch.exp(s - lse.unsqueeze(-1))[..., tri],
                              atol=1e-12)
