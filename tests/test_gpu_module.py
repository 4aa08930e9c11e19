"""The drop-in Attention / KVCache on the GPU, checked the way the reference's
own tests check the module (kempnerforge tests/unit/test_model.py:114-187,
test_hooks.py:169-245, test_generate.py:33-273), plus autograd, activation
checkpointing and torch.compile compatibility."""

from __future__ import annotations

import pytest
import torch

from gpu_util import DEV, announce, max_abs
from kempnerforge_amd import Attention, KVCache, ops
from kempnerforge_amd.position import precompute_rope_frequencies
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu


def _reference_module_out(attn: Attention, x, cos, sin):
    """Reference Attention.forward restated with the module's weights (CPU, fp64 math)."""
    B, S, _ = x.shape
    xc = x.detach().cpu()
    W = {n: p.detach().cpu() for n, p in attn.named_parameters()}
    q = (xc @ W["q_proj.weight"].T).view(B, S, -1, attn.head_dim)
    k = (xc @ W["k_proj.weight"].T).view(B, S, -1, attn.head_dim)
    v = (xc @ W["v_proj.weight"].T).view(B, S, -1, attn.head_dim)
    o, _ = ref.attention_fwd(q, k, v, cos.cpu(), sin.cpu())
    return o.reshape(B, S, -1).to(xc.dtype) @ W["o_proj.weight"].T


@pytest.mark.parametrize("n_heads,n_kv", [(8, 8), (8, 2), (8, 1)])
def test_forward_shapes_and_values(n_heads, n_kv):
    announce(f"module fwd {n_heads}/{n_kv}")
    torch.manual_seed(0)
    attn = Attention(dim=256, n_heads=n_heads, n_kv_heads=n_kv).to(DEV)
    cos, sin = precompute_rope_frequencies(32, 64)
    x = torch.randn(2, 64, 256, device=DEV)
    out = attn(x, cos.to(DEV), sin.to(DEV))
    assert out.shape == (2, 64, 256)
    want = _reference_module_out(attn, x, cos, sin)
    assert max_abs(out, want) <= 1e-4


def test_bf16_module_no_warnings():
    import warnings

    torch.manual_seed(0)
    attn = Attention(dim=1024, n_heads=8, n_kv_heads=2).to(DEV).to(torch.bfloat16)
    cos, sin = precompute_rope_frequencies(128, 128, 5e5)
    x = torch.randn(1, 128, 1024, device=DEV, dtype=torch.bfloat16)
    with warnings.catch_warnings():
        warnings.filterwarnings("error")
        with torch.no_grad():
            out = attn(x, cos.to(DEV), sin.to(DEV))
    assert out.dtype == torch.bfloat16
    want = _reference_module_out(attn, x, cos, sin)
    assert max_abs(out, want.float()) <= 5e-2


def test_qk_norm_large_inputs_finite():
    torch.manual_seed(0)
    attn = Attention(dim=128, n_heads=4, n_kv_heads=4, qk_norm=True).to(DEV)
    cos, sin = precompute_rope_frequencies(32, 16)
    out = attn(torch.randn(1, 16, 128, device=DEV) * 100.0, cos.to(DEV), sin.to(DEV))
    assert out.isfinite().all()


def test_capture_matches_reference_hooks_tests():
    announce("module capture")
    torch.manual_seed(0)
    attn = Attention(64, 4, 4).to(DEV).eval()
    cos, sin = precompute_rope_frequencies(16, 32)
    cos, sin = cos[:16].to(DEV), sin[:16].to(DEV)
    x = torch.randn(2, 16, 64, device=DEV)
    out_sdpa = attn(x, cos, sin)
    assert attn.last_attention_weights is None
    attn.capture_attention_weights = True
    out_manual = attn(x, cos, sin)
    w = attn.last_attention_weights
    assert w.shape == (2, 4, 16, 16) and w.device == torch.device("cpu")
    assert torch.allclose(w.float().sum(-1), torch.ones(2, 4, 16), atol=1e-5)
    upper = torch.triu(torch.ones(16, 16), diagonal=1).bool()
    assert torch.allclose(w[0, 0][upper], torch.zeros(int(upper.sum())), atol=1e-6)
    assert torch.allclose(out_sdpa, out_manual, atol=1e-4)


def test_backward_through_module_and_checkpoint():
    announce("module backward + activation checkpointing")
    torch.manual_seed(0)
    attn = Attention(dim=512, n_heads=8, n_kv_heads=2).to(DEV).to(torch.bfloat16)
    cos, sin = precompute_rope_frequencies(64, 256, 5e5)
    cos, sin = cos.to(DEV), sin.to(DEV)
    x = torch.randn(2, 256, 512, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    y = attn(x, cos, sin)
    y.float().pow(2).mean().backward()
    g1 = [p.grad.clone() for p in attn.parameters()] + [x.grad.clone()]
    attn.zero_grad()
    x.grad = None
    from torch.utils.checkpoint import checkpoint

    y2 = checkpoint(lambda t: attn(t, cos, sin), x, use_reentrant=False)
    y2.float().pow(2).mean().backward()
    g2 = [p.grad for p in attn.parameters()] + [x.grad]
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


def test_torch_compile_fullgraph():
    announce("torch.compile")
    torch.manual_seed(0)
    B, S, Hq, Hkv, D = 1, 128, 4, 2, 64
    q = torch.randn(B, S, Hq, D, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    k = torch.randn(B, S, Hkv, D, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    v = torch.randn(B, S, Hkv, D, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    cos, sin = precompute_rope_frequencies(D, S)
    cos, sin = cos.to(DEV), sin.to(DEV)

    def f(q, k, v):
        return ops.attention(q, k, v, cos, sin).float().sum()

    eager = f(q, k, v)
    compiled = torch.compile(f, fullgraph=True, backend="aot_eager")(q, k, v)
    assert torch.equal(eager, compiled)
    compiled.backward()
    assert q.grad is not None and k.grad is not None and v.grad is not None


def test_generate_style_decode_matches_full_forward():
    """Prefill then single-token decode through KVCache equals one causal forward
    over the whole sequence (reference generate.py:100-124 flow)."""
    announce("module prefill + decode")
    torch.manual_seed(0)
    dim, H, Hkv, D = 512, 8, 2, 64
    attn = Attention(dim, H, Hkv).to(DEV).to(torch.bfloat16).eval()
    T, P = 40, 24
    cos, sin = precompute_rope_frequencies(D, 64, 5e5)
    cos, sin = cos.to(DEV), sin.to(DEV)
    x = torch.randn(2, T, dim, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        full = attn(x, cos[:T], sin[:T])
        cache = KVCache(2, T, Hkv, D, torch.bfloat16, DEV)
        outs = [attn(x[:, :P], cos[:P], sin[:P], kv_cache=cache)]
        for t in range(P, T):
            outs.append(attn(x[:, t:t + 1], cos[t:t + 1], sin[t:t + 1], kv_cache=cache))
    inc = torch.cat(outs, dim=1)
    assert cache.seq_len == T and cache.lens.tolist() == [T, T]
    assert (inc.float() - full.float()).abs().max().item() <= 3e-2
    with pytest.raises(ValueError):
        attn(x[:, :1], cos[:1], sin[:1], kv_cache=cache)


def test_chunked_prefill_masks_top_left():
    """A second multi-token chunk into a filled cache: the reference calls SDPA
    with is_causal=True on the [Sq, Sk] scores (attention.py:228-231), whose
    causal mask is top-left aligned (query row i sees keys 0..i).  Checked
    against a float32 CPU restatement of that call on the module's own bf16
    projections; 32 queries against 72 keys leave a ragged last 32-key tile."""
    announce("module chunked prefill (Sq 32, Sk 72)")
    torch.manual_seed(0)
    dim, H, Hkv, D = 512, 8, 2, 64
    attn = Attention(dim, H, Hkv).to(DEV).to(torch.bfloat16).eval()
    P, T = 40, 72
    cos, sin = precompute_rope_frequencies(D, 128, 5e5)
    cos, sin = cos.to(DEV), sin.to(DEV)
    x = torch.randn(2, T, dim, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        cache = KVCache(2, T, Hkv, D, torch.bfloat16, DEV)
        attn(x[:, :P], cos[:P], sin[:P], kv_cache=cache)
        got = attn(x[:, P:], cos[P:T], sin[P:T], kv_cache=cache).float().cpu()
        q = attn.q_proj(x[:, P:]).float().cpu().view(2, T - P, H, D).transpose(1, 2)
        k = attn.k_proj(x).float().cpu().view(2, T, Hkv, D).transpose(1, 2)
        v = attn.v_proj(x).float().cpu().view(2, T, Hkv, D).transpose(1, 2)
        wo = attn.o_proj.weight.float().cpu()
    c, s = cos.cpu(), sin.cpu()

    def rope(t, cc, ss):
        t1, t2 = t[..., :D // 2], t[..., D // 2:]
        return torch.cat([t1 * cc - t2 * ss, t2 * cc + t1 * ss], -1)

    q, k = rope(q, c[P:T], s[P:T]), rope(k, c[:T], s[:T])
    k, v = k.repeat_interleave(H // Hkv, 1), v.repeat_interleave(H // Hkv, 1)
    scores = (q @ k.transpose(-1, -2)) / D ** 0.5
    top_left = torch.ones(T - P, T, dtype=torch.bool).tril()
    p = scores.masked_fill(~top_left, float("-inf")).softmax(-1)
    want = (p @ v).transpose(1, 2).reshape(2, T - P, H * D) @ wo.t()
    err = (got - want).abs().max().item()
    print(f"chunked prefill max-abs err {err:.3e}")
    assert cache.seq_len == T and err <= 1.5e-2


def test_one_document_equals_causal():
    # packed-document path (reference :190-227) with one document equals plain
    # causal (reference tests/unit/test_packing.py:269-277); an all-True
    # key_padding_mask (the explicit-mask branch kept in PyTorch) too
    torch.manual_seed(0)
    attn = Attention(128, 4, 2).to(DEV)
    cos, sin = precompute_rope_frequencies(32, 32)
    cos, sin = cos.to(DEV), sin.to(DEV)
    x = torch.randn(2, 32, 128, device=DEV)
    a = attn(x, cos, sin)
    b = attn(x, cos, sin, doc_ids=torch.zeros(2, 32, dtype=torch.long, device=DEV))
    c = attn(x, cos, sin, key_padding_mask=torch.ones(2, 32, dtype=torch.bool, device=DEV))
    assert torch.allclose(a, b, atol=1e-4)
    assert torch.allclose(a, c, atol=1e-4)
