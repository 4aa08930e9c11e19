"""GPU parity of packed-document attention (``doc_ids``) against the CPU oracle.

The reference builds an explicit bool mask, causal AND same-document
(kempnerforge/model/attention.py:204-227), from the ``doc_ids`` its packing
dataset emits (kempnerforge/data/dataset.py:27-65); its tests pin that one
document equals plain causal and that documents do not see each other
(tests/unit/test_packing.py:98-310).  Here the kernels take ``doc_ids`` and
apply the same condition per tile.  Tolerances are the forward/backward ones:
output max-abs 1e-5 (float32) / 2e-2 (bf16), LSE 1e-5 / 1e-3, gradients
per element (gpu_util.grad_bound), probabilities 1e-5 for both dtypes.
"""

from __future__ import annotations

import pytest
import torch

from gpu_util import DEV, TOL, announce, check_grad, check_out, max_abs, seeded
from kempnerforge_amd import Attention, ops
from kempnerforge_amd._lib import KernelError
from kempnerforge_amd.position import precompute_rope_frequencies
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu



def packed(B, lengths_per_row):
    """[B, S] int64 ids, increasing contiguous segments per row (the packing
    dataset's layout)."""
    rows = [torch.cat([torch.full((n,), d, dtype=torch.long) for d, n in enumerate(lens)])
            for lens in lengths_per_row]
    return torch.stack(rows)


def random_lengths(S, seed, lo=1, hi=300):
    g = torch.Generator().manual_seed(seed)
    out, left = [], S
    while left:
        n = min(left, int(torch.randint(lo, hi + 1, (1,), generator=g)))
        out.append(n)
        left -= n
    return out


def _inputs(dtype, B, S, Hq, Hkv, D, seed=0):
    q = seeded((B, S, Hq, D), seed, dtype)
    k = seeded((B, S, Hkv, D), seed + 1, dtype)
    v = seeded((B, S, Hkv, D), seed + 2, dtype)
    do = seeded((B, S, Hq, D), seed + 3, dtype)
    cos, sin = ref.rope_tables(D, S, 5e5)
    return q, k, v, do, cos, sin


# (dtype, B, S, Hq, Hkv, D, layout name)
CASES = [
    (torch.bfloat16, 2, 300, 8, 2, 128, "random"),
    (torch.bfloat16, 1, 256, 4, 4, 64, "tile_edges"),
    (torch.bfloat16, 1, 200, 32, 1, 128, "random"),
    (torch.bfloat16, 1, 130, 6, 2, 128, "singletons"),
    (torch.bfloat16, 2, 190, 4, 2, 128, "reused_ids"),
    (torch.float32, 1, 150, 8, 2, 128, "random"),
    (torch.float32, 2, 96, 4, 1, 64, "tile_edges"),
    # more than 64 tiles: the tile lists span several 64-tile words
    (torch.bfloat16, 1, 4500, 2, 1, 64, "random"),
    (torch.bfloat16, 1, 4200, 2, 2, 128, "reused_ids"),
]


def _doc_ids(B, S, layout, seed=0):
    if layout == "random":
        return packed(B, [random_lengths(S, seed + b) for b in range(B)])
    if layout == "tile_edges":  # boundaries on and next to 64-key tile edges
        base = [64, 1, 63, 64, 65]
        lens, left = [], S
        for n in base * (S // sum(base) + 1):
            if not left:
                break
            lens.append(min(n, left))
            left -= lens[-1]
        return packed(B, [lens] * B)
    if layout == "singletons":  # every token its own document: out = v of itself
        return torch.arange(S).repeat(B, 1)
    if layout == "reused_ids":  # an id reused after another one: still one mask
        ids = (torch.arange(S) // 23) % 3
        return torch.stack([ids, ids.roll(7)])[:B]
    raise ValueError(layout)


@pytest.mark.parametrize("cfg", CASES, ids=lambda c: "-".join(map(str, c)))
def test_forward(cfg):
    dtype, B, S, Hq, Hkv, D, layout = cfg
    announce(f"doc fwd {cfg}")
    q, k, v, _, cos, sin = _inputs(dtype, B, S, Hq, Hkv, D)
    doc = _doc_ids(B, S, layout)
    out, lse = ops.fwd_raw(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV),
                           causal=True, k_rotated=False, doc_ids=doc.to(DEV))
    o_ref, l_ref = ref.attention_fwd(q, k, v, cos, sin, doc_ids=doc)
    torch.cuda.synchronize()
    assert max_abs(out, o_ref) <= TOL[dtype]
    assert max_abs(lse, l_ref) <= (1e-5 if dtype == torch.float32 else 1e-3)


@pytest.mark.parametrize("cfg", CASES, ids=lambda c: "-".join(map(str, c)))
def test_backward(cfg):
    dtype, B, S, Hq, Hkv, D, layout = cfg
    announce(f"doc bwd {cfg}")
    q, k, v, do, cos, sin = _inputs(dtype, B, S, Hq, Hkv, D)
    doc = _doc_ids(B, S, layout)
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    out = ops.attention(qd, kd, vd, cos.to(DEV), sin.to(DEV), doc_ids=doc.to(DEV))
    out.backward(do.to(DEV))
    torch.cuda.synchronize()
    dq, dk, dv = ref.attention_bwd(q, k, v, cos, sin, do, doc_ids=doc)
    for got, want, name in ((qd.grad, dq, "dq"), (kd.grad, dk, "dk"), (vd.grad, dv, "dv")):
        check_grad(got, want, dtype, name, group=Hq // Hkv if name != "dq" else 1)


BF16_CASES = [c for c in CASES if c[0] == torch.bfloat16]


@pytest.mark.parametrize("cfg", BF16_CASES, ids=lambda c: "-".join(map(str, c)))
def test_backward_kept_and_recomputed_ds(cfg):
    """Packed documents through both dQ paths: the dS tiles the dK/dV pass keeps
    (written only for the listed query tiles; dQ reads only the listed key tiles)
    and the minimal workspace, where dQ recomputes S and dP.  dK and dV are the
    same arithmetic either way (bitwise equal)."""
    dtype, B, S, Hq, Hkv, D, layout = cfg
    announce(f"doc bwd kept/recomputed dS {cfg}")
    q, k, v, do, cos, sin = _inputs(dtype, B, S, Hq, Hkv, D)
    doc = _doc_ids(B, S, layout).to(DEV)
    args = [t.to(DEV) for t in (q, k, v, cos, sin)]
    out, lse = ops.fwd_raw(*args, causal=True, k_rotated=False, doc_ids=doc)
    kept = ops.bwd_raw(*args, out, lse, do.to(DEV), causal=True, doc_ids=doc)
    recomputed = ops.bwd_raw(*args, out, lse, do.to(DEV), causal=True, doc_ids=doc,
                             low_memory=True)
    torch.cuda.synchronize()
    assert torch.equal(kept[1], recomputed[1]) and torch.equal(kept[2], recomputed[2])
    refs = ref.attention_bwd(q, k, v, cos, sin, do, doc_ids=doc.cpu())
    for path, grads in (("kept", kept), ("recomputed", recomputed)):
        for got, want, name in zip(grads, refs, ("dq", "dk", "dv")):
            check_grad(got, want, dtype, f"{path} {name}", group=Hq // Hkv if name != "dq" else 1)


@pytest.mark.parametrize("cfg", [CASES[0], CASES[3], CASES[5]], ids=lambda c: "-".join(map(str, c)))
def test_capture(cfg):
    dtype, B, S, Hq, Hkv, D, layout = cfg
    announce(f"doc capture {cfg}")
    q, k, v, _, cos, sin = _inputs(dtype, B, S, Hq, Hkv, D)
    doc = _doc_ids(B, S, layout)
    out, p, _ = ops.capture_raw(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV),
                                causal=True, k_rotated=False, doc_ids=doc.to(DEV))
    o_ref, p_ref = ref.capture(q, k, v, cos, sin, doc_ids=doc)
    torch.cuda.synchronize()
    check_out(p, p_ref, 1e-5, "probs")
    assert max_abs(out, o_ref) <= TOL[dtype]
    # probabilities of other documents' keys are exactly zero
    other = (doc.unsqueeze(2) != doc.unsqueeze(1)).unsqueeze(1).expand_as(p_ref)
    assert p.cpu()[other].abs().max().item() == 0.0


def test_llama8b_shape_documents_independent():
    """C2 shape with packed documents: each document's rows equal the kernel run
    on that document alone (same absolute positions), and a single document
    equals plain causal attention."""
    B, S, Hq, Hkv, D = 2, 4096, 32, 8, 128
    announce("doc 8B shape")
    q, k, v, do, cos, sin = _inputs(torch.bfloat16, B, S, Hq, Hkv, D)
    q, k, v, do, cos, sin = (t.to(DEV) for t in (q, k, v, do, cos, sin))
    lens = [[1000, 1, 63, 64, 968, 2000], random_lengths(S, 5, 200, 1500)]
    doc = packed(B, lens).to(DEV)
    out, lse = ops.fwd_raw(q, k, v, cos, sin, causal=True, k_rotated=False, doc_ids=doc)
    for b in range(B):
        s0 = 0
        for n in lens[b]:
            sl = slice(s0, s0 + n)
            o_d, l_d = ops.fwd_raw(q[b:b + 1, sl].contiguous(), k[b:b + 1, sl].contiguous(),
                                   v[b:b + 1, sl].contiguous(), cos[sl].contiguous(),
                                   sin[sl].contiguous(), causal=True, k_rotated=False)
            assert (out[b:b + 1, sl].float() - o_d.float()).abs().max().item() <= 2e-2
            assert (lse[b:b + 1, :, sl] - l_d).abs().max().item() <= 1e-3
            s0 += n
    one = torch.zeros(B, S, dtype=torch.long, device=DEV)
    o1, l1 = ops.fwd_raw(q, k, v, cos, sin, causal=True, k_rotated=False, doc_ids=one)
    o0, l0 = ops.fwd_raw(q, k, v, cos, sin, causal=True, k_rotated=False)
    torch.cuda.synchronize()
    assert (o1.float() - o0.float()).abs().max().item() <= 2e-2
    assert (l1 - l0).abs().max().item() <= 1e-3


def test_llama8b_shape_backward_documents_independent():
    """Gradients with packed documents equal the per-document gradients."""
    B, S, Hq, Hkv, D = 1, 4096, 32, 8, 128
    announce("doc bwd 8B shape")
    q, k, v, do, cos, sin = _inputs(torch.bfloat16, B, S, Hq, Hkv, D, seed=4)
    q, k, v, do, cos, sin = (t.to(DEV) for t in (q, k, v, do, cos, sin))
    lens = [1500, 64, 1, 1000, 1531]
    doc = packed(B, [lens]).to(DEV)
    out, lse = ops.fwd_raw(q, k, v, cos, sin, causal=True, k_rotated=False, doc_ids=doc)
    dq, dk, dv = ops.bwd_raw(q, k, v, cos, sin, out, lse, do, causal=True, doc_ids=doc)
    s0 = 0
    for n in lens:
        sl = slice(s0, s0 + n)
        args = [t[:, sl].contiguous() for t in (q, k, v)] + [cos[sl].contiguous(),
                                                             sin[sl].contiguous()]
        o_d, l_d = ops.fwd_raw(*args, causal=True, k_rotated=False)
        g_d = ops.bwd_raw(*args, o_d, l_d, do[:, sl].contiguous(), causal=True)
        for got, want, name in zip((dq, dk, dv), g_d, ("dq", "dk", "dv")):
            check_grad(got[:, sl], want.float(), torch.bfloat16, f"doc of {n} {name}")
        s0 += n


def test_doc_ids_need_causal_self_attention():
    q, k, v, _, cos, sin = _inputs(torch.bfloat16, 1, 64, 4, 2, 128)
    doc = torch.zeros(1, 64, dtype=torch.long, device=DEV)
    with pytest.raises(KernelError):
        ops.fwd_raw(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV), causal=False,
                    k_rotated=False, doc_ids=doc)
    with pytest.raises(ValueError):
        ops.fwd_raw(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV), causal=True,
                    k_rotated=False, doc_ids=doc[:, :32])


def _module_reference(attn, x, cos, sin, doc):
    B, S, _ = x.shape
    xc = x.detach().cpu()
    W = {n: p.detach().cpu() for n, p in attn.named_parameters()}
    q = (xc @ W["q_proj.weight"].T).view(B, S, -1, attn.head_dim)
    k = (xc @ W["k_proj.weight"].T).view(B, S, -1, attn.head_dim)
    v = (xc @ W["v_proj.weight"].T).view(B, S, -1, attn.head_dim)
    o, _ = ref.attention_fwd(q, k, v, cos.cpu(), sin.cpu(), doc_ids=doc.cpu())
    return o.reshape(B, S, -1).to(xc.dtype) @ W["o_proj.weight"].T


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_module_doc_ids(dtype):
    """Attention.forward(doc_ids=...) on the kernels against the reference's
    explicit-mask branch restated on the CPU, plus capture of the same call."""
    announce(f"doc module {dtype}")
    torch.manual_seed(0)
    attn = Attention(256, 8, 2).to(DEV, dtype)
    S = 160
    cos, sin = precompute_rope_frequencies(32, S)
    cos, sin = cos.to(DEV), sin.to(DEV)
    x = torch.randn(2, S, 256, device=DEV, dtype=dtype)
    doc = packed(2, [[40, 1, 80, 39], [160]]).to(DEV)
    y = attn(x, cos, sin, doc_ids=doc)
    want = _module_reference(attn, x, cos, sin, doc)
    tol = 1e-4 if dtype == torch.float32 else 5e-2
    assert max_abs(y, want) <= tol
    attn.capture_attention_weights = True
    y2 = attn(x, cos, sin, doc_ids=doc)
    p = attn.last_attention_weights
    assert p.shape == (2, 8, S, S)
    assert max_abs(y2, want) <= tol
    assert p[0, :, 41:121, :41].abs().max().item() == 0.0  # third document sees no earlier one


@pytest.mark.parametrize("masks", ["doc", "kpm", "both"])
def test_module_capture_with_cache_and_masks(masks):
    """Capture with a KV cache and an explicit mask (kempnerforge/model/
    attention.py:169-170,252-271): on an empty cache the reference's masks
    broadcast and the result is the cache-free capture of the same call (the
    cache then holds this call's rotated keys), computed here by the capture
    kernel; on a non-empty cache the reference's mask construction raises, and
    so does the module, after appending as the reference does."""
    from kempnerforge_amd import KVCache

    announce(f"doc module capture + cache + {masks}")
    torch.manual_seed(1)
    dtype = torch.bfloat16
    attn = Attention(256, 8, 2).to(DEV, dtype)
    S = 96
    cos, sin = precompute_rope_frequencies(32, S)
    cos, sin = cos.to(DEV), sin.to(DEV)
    x = torch.randn(2, S, 256, device=DEV, dtype=dtype)
    kw = {}
    if masks in ("doc", "both"):
        kw["doc_ids"] = packed(2, [[30, 1, 65], [96]]).to(DEV)
    if masks in ("kpm", "both"):
        kpm = torch.ones(2, S, dtype=torch.bool, device=DEV)
        kpm[1, 10:20] = False
        kw["key_padding_mask"] = kpm
    attn.capture_attention_weights = True
    y_ref = attn(x, cos, sin, **kw)
    p_ref = attn.last_attention_weights
    cache = KVCache(2, 2 * S, 2, 32, dtype, DEV)
    y = attn(x, cos, sin, kv_cache=cache, **kw)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref) and torch.equal(attn.last_attention_weights, p_ref)
    assert cache.seq_len == S
    with pytest.raises(RuntimeError):
        attn(x, cos, sin, kv_cache=cache, **kw)
    assert cache.seq_len == 2 * S  # appended before the masks failed, as the reference
