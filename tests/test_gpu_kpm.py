"""GPU parity of key-padding attention (``key_padding_mask``) against the oracle.

The reference's explicit-mask branch allows key j for query i when j <= i and
the key is valid, and unmasks entirely a row left with no key (NaN guard:
``mask | ~mask.any(-1)``; kempnerforge/model/attention.py:214-225,
kempnerforge/model/mot.py:188-198).  The oracle restates it and is pinned
against PyTorch's library SDPA with that explicit mask (tests/test_oracle.py).
Here the kernels take the mask as int32 flags.  Tolerances as for the
forward/backward: output 1e-5 (float32) / 2e-2 (bf16), LSE 1e-5 / 1e-3,
gradients per element (gpu_util.grad_bound), probabilities 1e-5 for both
dtypes.
"""

from __future__ import annotations

import pytest
import torch

from gpu_util import DEV, TOL, announce, check_grad, check_out, max_abs, seeded
from kempnerforge_amd import Attention, ops
from kempnerforge_amd.position import precompute_rope_frequencies
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu



def _inputs(dtype, B, S, Hq, Hkv, D, seed=0):
    q = seeded((B, S, Hq, D), seed, dtype)
    k = seeded((B, S, Hkv, D), seed + 1, dtype)
    v = seeded((B, S, Hkv, D), seed + 2, dtype)
    do = seeded((B, S, Hq, D), seed + 3, dtype)
    cos, sin = ref.rope_tables(D, S, 5e5)
    return q, k, v, do, cos, sin


def _mask(B, S, layout, seed=0):
    m = torch.ones(B, S, dtype=torch.bool)
    g = torch.Generator().manual_seed(seed)
    for b in range(B):
        if layout == "middle":      # padded frames in the middle
            m[b, S // 3: S // 3 + 40] = False
        elif layout == "leading":   # leading padding: rows before it are guarded
            m[b, : 70 + 13 * b] = False
        elif layout == "random":
            m[b] = torch.rand(S, generator=g) > 0.3
        elif layout == "tiles":     # whole 64-key tiles padded, and ragged edges
            m[b, 64:128] = False
            m[b, 191:257] = False
        elif layout == "none_valid":  # an all-padded clip: every row guarded
            m[b] = b % 2 == 1
    return m


# (dtype, B, S, Hq, Hkv, D, layout)
CASES = [
    (torch.bfloat16, 2, 300, 8, 2, 128, "middle"),
    (torch.bfloat16, 2, 300, 8, 2, 128, "leading"),
    (torch.bfloat16, 1, 260, 4, 4, 64, "tiles"),
    (torch.bfloat16, 2, 200, 32, 1, 128, "random"),
    (torch.bfloat16, 2, 130, 6, 2, 128, "none_valid"),
    (torch.float32, 2, 150, 8, 2, 128, "leading"),
    (torch.float32, 1, 96, 4, 1, 64, "random"),
    (torch.bfloat16, 1, 4300, 2, 1, 64, "random"),   # more than 64 key tiles
]


@pytest.mark.parametrize("cfg", CASES, ids=lambda c: "-".join(map(str, c)))
def test_forward(cfg):
    dtype, B, S, Hq, Hkv, D, layout = cfg
    announce(f"kpm fwd {cfg}")
    q, k, v, _, cos, sin = _inputs(dtype, B, S, Hq, Hkv, D)
    kpm = _mask(B, S, layout)
    out, lse = ops.fwd_raw(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV),
                           causal=True, k_rotated=False, key_padding_mask=kpm.to(DEV))
    o_ref, l_ref = ref.attention_fwd(q, k, v, cos, sin, key_padding_mask=kpm)
    torch.cuda.synchronize()
    assert max_abs(out, o_ref) <= TOL[dtype]
    assert max_abs(lse, l_ref) <= (1e-5 if dtype == torch.float32 else 1e-3)


@pytest.mark.parametrize("cfg", CASES, ids=lambda c: "-".join(map(str, c)))
def test_backward(cfg):
    dtype, B, S, Hq, Hkv, D, layout = cfg
    announce(f"kpm bwd {cfg}")
    q, k, v, do, cos, sin = _inputs(dtype, B, S, Hq, Hkv, D)
    kpm = _mask(B, S, layout)
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    out = ops.attention(qd, kd, vd, cos.to(DEV), sin.to(DEV), key_padding_mask=kpm.to(DEV))
    out.backward(do.to(DEV))
    torch.cuda.synchronize()
    dq, dk, dv = ref.attention_bwd(q, k, v, cos, sin, do, key_padding_mask=kpm)
    for got, want, name in ((qd.grad, dq, "dq"), (kd.grad, dk, "dk"), (vd.grad, dv, "dv")):
        check_grad(got, want, dtype, name, group=Hq // Hkv if name != "dq" else 1)


@pytest.mark.parametrize("cfg", [CASES[1], CASES[3], CASES[4], CASES[5]],
                         ids=lambda c: "-".join(map(str, c)))
def test_capture(cfg):
    dtype, B, S, Hq, Hkv, D, layout = cfg
    announce(f"kpm capture {cfg}")
    q, k, v, _, cos, sin = _inputs(dtype, B, S, Hq, Hkv, D)
    kpm = _mask(B, S, layout)
    out, p, _ = ops.capture_raw(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV),
                                causal=True, k_rotated=False, key_padding_mask=kpm.to(DEV))
    o_ref, p_ref = ref.capture(q, k, v, cos, sin, key_padding_mask=kpm)
    torch.cuda.synchronize()
    check_out(p, p_ref, 1e-5, "probs")
    assert max_abs(out, o_ref) <= TOL[dtype]
    assert p.cpu()[p_ref == 0].abs().max().item() == 0.0  # masked exactly zero


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_with_documents(dtype):
    """doc_ids and key_padding_mask together (the reference ANDs them)."""
    announce(f"kpm + doc {dtype}")
    B, S, Hq, Hkv, D = 2, 210, 4, 2, 128
    q, k, v, do, cos, sin = _inputs(dtype, B, S, Hq, Hkv, D, seed=3)
    doc = torch.cat([torch.zeros(70), torch.ones(90), torch.full((50,), 2)]).long().repeat(B, 1)
    kpm = _mask(B, S, "random", seed=5)
    kpm[0, 70:100] = False  # a document whose first 30 keys are padded: guarded rows
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    out = ops.attention(qd, kd, vd, cos.to(DEV), sin.to(DEV), doc_ids=doc.to(DEV),
                        key_padding_mask=kpm.to(DEV))
    out.backward(do.to(DEV))
    o_ref, _ = ref.attention_fwd(q, k, v, cos, sin, doc_ids=doc, key_padding_mask=kpm)
    dq, dk, dv = ref.attention_bwd(q, k, v, cos, sin, do, doc_ids=doc, key_padding_mask=kpm)
    torch.cuda.synchronize()
    assert max_abs(out, o_ref) <= TOL[dtype]
    for got, want, name in ((qd.grad, dq, "dq"), (kd.grad, dk, "dk"), (vd.grad, dv, "dv")):
        check_grad(got, want, dtype, name, group=Hq // Hkv if name != "dq" else 1)


def test_llama8b_shape_padded_keys_drop_out():
    """C2 shape: an all-valid mask equals plain causal attention; with padded
    keys (no guarded rows) the padded keys' dK/dV are exactly zero, and the
    first 1536 rows match the oracle (a causal row only sees its prefix)."""
    B, S, Hq, Hkv, D = 2, 4096, 32, 8, 128
    announce("kpm 8B shape")
    q, k, v, do, cos, sin = (t.to(DEV) for t in _inputs(torch.bfloat16, B, S, Hq, Hkv, D))
    ones = torch.ones(B, S, dtype=torch.bool, device=DEV)
    o1, l1 = ops.fwd_raw(q, k, v, cos, sin, causal=True, k_rotated=False, key_padding_mask=ones)
    o0, l0 = ops.fwd_raw(q, k, v, cos, sin, causal=True, k_rotated=False)
    assert (o1.float() - o0.float()).abs().max().item() <= 2e-2
    assert (l1 - l0).abs().max().item() <= 1e-3
    kpm = ones.clone()
    kpm[:, 1000:1500] = False
    kpm[1, 3000:] = False
    out, lse = ops.fwd_raw(q, k, v, cos, sin, causal=True, k_rotated=False, key_padding_mask=kpm)
    dq, dk, dv = ops.bwd_raw(q, k, v, cos, sin, out, lse, do, causal=True,
                             key_padding_mask=kpm)
    torch.cuda.synchronize()
    pad = ~kpm
    assert dk[pad].abs().max().item() == 0.0 and dv[pad].abs().max().item() == 0.0
    assert torch.isfinite(dq).all() and torch.isfinite(out).all()
    # spot rows against the oracle on a prefix (the mask of a prefix is the
    # prefix of the mask: rows < 1536 only see keys < 1536)
    P = 1536
    o_ref, l_ref = ref.attention_fwd(q[:1, :P].cpu(), k[:1, :P].cpu(), v[:1, :P].cpu(),
                                     cos[:P].cpu(), sin[:P].cpu(), key_padding_mask=kpm[:1, :P].cpu())
    assert max_abs(out[:1, :P], o_ref) <= 2e-2
    assert max_abs(lse[:1, :, :P], l_ref) <= 1e-3


def _module_reference(attn, x, cos, sin, kpm):
    B, S, _ = x.shape
    xc = x.detach().cpu()
    W = {n: p.detach().cpu() for n, p in attn.named_parameters()}
    q = (xc @ W["q_proj.weight"].T).view(B, S, -1, attn.head_dim)
    k = (xc @ W["k_proj.weight"].T).view(B, S, -1, attn.head_dim)
    v = (xc @ W["v_proj.weight"].T).view(B, S, -1, attn.head_dim)
    o, _ = ref.attention_fwd(q, k, v, cos.cpu(), sin.cpu(), key_padding_mask=kpm.cpu())
    return o.reshape(B, S, -1).to(xc.dtype) @ W["o_proj.weight"].T


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_module_key_padding_mask(dtype):
    """Attention.forward(key_padding_mask=...) on the kernels, and its capture."""
    announce(f"kpm module {dtype}")
    torch.manual_seed(0)
    attn = Attention(256, 8, 2).to(DEV, dtype)
    S = 150
    cos, sin = precompute_rope_frequencies(32, S)
    cos, sin = cos.to(DEV), sin.to(DEV)
    x = torch.randn(2, S, 256, device=DEV, dtype=dtype)
    kpm = _mask(2, S, "leading").to(DEV)
    y = attn(x, cos, sin, key_padding_mask=kpm)
    want = _module_reference(attn, x, cos, sin, kpm)
    tol = 1e-4 if dtype == torch.float32 else 5e-2
    assert max_abs(y, want) <= tol
    attn.capture_attention_weights = True
    y2 = attn(x, cos, sin, key_padding_mask=kpm)
    p = attn.last_attention_weights
    assert max_abs(y2, want) <= tol
    assert p.shape == (2, 8, S, S)
    assert p[0, :, 70:, :70].abs().max().item() == 0.0  # padded keys get nothing
    assert p[0, :, :70, :].float().sum(-1).sub(1).abs().max().item() < 2e-2  # guarded rows


@pytest.mark.parametrize("cfg", [(3, 300, 8, 2, 128), (2, 200, 4, 4, 64), (2, 260, 6, 3, 128)],
                         ids=lambda c: "-".join(map(str, c)))
def test_backward_records_path(cfg):
    """Batch rows whose key 0 is valid keep the dS records (dQ from them), rows
    with guarded rows recompute dQ, in one launch: dK/dV are the same bits as
    with low_memory=True (no records), dQ of the guarded batch row too, and
    every gradient is within tolerance of the oracle."""
    B, S, Hq, Hkv, D = cfg
    announce(f"kpm records {cfg}")
    dtype = torch.bfloat16
    q, k, v, do, cos, sin = _inputs(dtype, B, S, Hq, Hkv, D, seed=11)
    kpm = torch.ones(B, S, dtype=torch.bool)
    kpm[0, S // 3: S // 3 + 40] = False           # key 0 valid: records
    kpm[1, : 45] = False                          # leading padding: guarded rows, recompute
    if B > 2:
        kpm[2, 130:200] = False                   # whole tiles and ragged edges, records
    args = [t.to(DEV) for t in (q, k, v, cos, sin)]
    out, lse = ops.fwd_raw(*args, causal=True, k_rotated=False, key_padding_mask=kpm.to(DEV))
    kept = ops.bwd_raw(*args, out, lse, do.to(DEV), causal=True, key_padding_mask=kpm.to(DEV))
    recomputed = ops.bwd_raw(*args, out, lse, do.to(DEV), causal=True,
                             key_padding_mask=kpm.to(DEV), low_memory=True)
    torch.cuda.synchronize()
    assert torch.equal(kept[1], recomputed[1]) and torch.equal(kept[2], recomputed[2])
    assert torch.equal(kept[0][1], recomputed[0][1])  # the guarded batch row's dQ
    # the records path is the one taken for the other rows: a different
    # accumulation than the recompute kernel's, so not the same bits
    assert not torch.equal(kept[0][0], recomputed[0][0])
    dq, dk, dv = ref.attention_bwd(q, k, v, cos, sin, do, key_padding_mask=kpm)
    for got, want, name in ((kept[0], dq, "dq"), (kept[1], dk, "dk"), (kept[2], dv, "dv")):
        check_grad(got, want, dtype, name, group=Hq // Hkv if name != "dq" else 1)


def test_all_valid_mask_equals_unmasked_backward():
    """An all-True key_padding_mask (what the VLM arches pass when nothing is
    padded) takes the masked kernels with the dS records kept; every tile is
    listed without an element test, so dQ, dK and dV equal the unmasked
    backward's bit for bit (same out and LSE in)."""
    B, S, Hq, Hkv, D = 2, 1100, 32, 8, 128
    announce("kpm all-valid == unmasked backward")
    q, k, v, do, cos, sin = (t.to(DEV) for t in _inputs(torch.bfloat16, B, S, Hq, Hkv, D, seed=5))
    ones = torch.ones(B, S, dtype=torch.bool, device=DEV)
    out, lse = ops.fwd_raw(q, k, v, cos, sin, causal=True, k_rotated=False)
    g_mask = ops.bwd_raw(q, k, v, cos, sin, out, lse, do, causal=True, key_padding_mask=ones)
    g_none = ops.bwd_raw(q, k, v, cos, sin, out, lse, do, causal=True)
    torch.cuda.synchronize()
    for a, b_, name in zip(g_mask, g_none, ("dq", "dk", "dv")):
        assert torch.equal(a, b_), f"{name}: max diff {(a.float() - b_.float()).abs().max().item()}"


def test_mixed_batch_split_paths():
    """A batch mixing a row without padding (unmasked forward and dK/dV kernels,
    dS records), a row with padding in the middle (masked kernels, records) and
    a row with leading padding (masked kernels, recomputed dQ): every output
    and gradient within tolerance of the oracle, and the unpadded row equal to
    the same row run without any mask, bit for bit."""
    B, S, Hq, Hkv, D = 3, 520, 8, 2, 128
    announce("kpm mixed batch")
    dtype = torch.bfloat16
    q, k, v, do, cos, sin = _inputs(dtype, B, S, Hq, Hkv, D, seed=21)
    kpm = torch.ones(B, S, dtype=torch.bool)
    kpm[1, 200:290] = False
    kpm[2, :77] = False
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    out = ops.attention(qd, kd, vd, cos.to(DEV), sin.to(DEV), key_padding_mask=kpm.to(DEV))
    out.backward(do.to(DEV))
    # row 0 alone, no mask
    q0, k0, v0 = (t[:1].to(DEV).requires_grad_(True) for t in (q, k, v))
    out0 = ops.attention(q0, k0, v0, cos.to(DEV), sin.to(DEV))
    out0.backward(do[:1].to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(out[:1], out0)
    for a, b_ in ((qd.grad, q0.grad), (kd.grad, k0.grad), (vd.grad, v0.grad)):
        assert torch.equal(a[:1], b_)
    o_ref, _ = ref.attention_fwd(q, k, v, cos, sin, key_padding_mask=kpm)
    assert max_abs(out, o_ref) <= TOL[dtype]
    dq, dk, dv = ref.attention_bwd(q, k, v, cos, sin, do, key_padding_mask=kpm)
    for got, want, name in ((qd.grad, dq, "dq"), (kd.grad, dk, "dk"), (vd.grad, dv, "dv")):
        check_grad(got, want, dtype, name, group=Hq // Hkv if name != "dq" else 1)
