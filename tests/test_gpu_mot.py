"""MoTAttention on the GPU against the reference's Algorithm-1 composition
(kempnerforge tests/unit/test_mot.py:214-340): per-modality projections and
RoPE with positions restarting at 0 in every modality, concatenation, one
global SDPA, split, per-modality o_proj.  The restatement below runs on the
CPU in float64 with the oracle's eager-rounding RoPE, so it checks the
kernels' handling of modality-local positions independently of how the module
feeds them."""

from __future__ import annotations

import copy

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from gpu_util import DEV, announce, max_abs
from kempnerforge_amd import MoTAttention
from kempnerforge_amd.position import precompute_rope_frequencies
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu


def _rope(t, hd):
    cos, sin = precompute_rope_frequencies(hd, t)
    return cos.to(DEV), sin.to(DEV)


def _algorithm_1(attn, streams, rope, is_causal=True, key_padding_mask=None):
    """CPU float64 restatement of the reference forward (mot.py:139-207)."""
    W = {n: p.detach().cpu().double() for n, p in attn.named_parameters()}
    batch = next(iter(streams.values())).shape[0]
    qs, ks, vs, lens = [], [], [], []
    for m in attn.modalities:
        x = streams[m].detach().cpu()
        t = x.shape[1]
        xd = x.double()
        q = (xd @ W[f"q_proj.{m}.weight"].T).to(x.dtype).view(batch, t, -1, attn.head_dim)
        k = (xd @ W[f"k_proj.{m}.weight"].T).to(x.dtype).view(batch, t, -1, attn.head_dim)
        v = (xd @ W[f"v_proj.{m}.weight"].T).to(x.dtype).view(batch, t, -1, attn.head_dim)
        if attn.q_norm is not None:
            q = attn.q_norm[m].cpu()(q)
            k = attn.k_norm[m].cpu()(k)
            attn.to(DEV)
        cos, sin = (r.cpu() for r in rope[m])
        qs.append(ref.apply_rope(q.transpose(1, 2), cos[:t], sin[:t]).double())
        ks.append(ref.apply_rope(k.transpose(1, 2), cos[:t], sin[:t]).double())
        vs.append(v.transpose(1, 2).double())
        lens.append(t)
    q, k, v = torch.cat(qs, 2), torch.cat(ks, 2), torch.cat(vs, 2)
    k = k.repeat_interleave(attn.n_rep, dim=1)
    v = v.repeat_interleave(attn.n_rep, dim=1)
    total = q.shape[2]
    if key_padding_mask is not None:
        mask = torch.ones(total, total, dtype=torch.bool).tril().view(1, 1, total, total)
        mask = mask & key_padding_mask.cpu().view(batch, 1, 1, total)
        mask = mask | ~mask.any(dim=-1, keepdim=True)
        out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask)
    else:
        out = F.scaled_dot_product_attention(q, k, v, is_causal=is_causal)
    out = out.transpose(1, 2)
    res, off = {}, 0
    for m, t in zip(attn.modalities, lens):
        o = out[:, off:off + t].reshape(batch, t, -1)
        res[m] = o @ W[f"o_proj.{m}.weight"].T
        off += t
    return res


def _make(n_heads=4, n_kv=2, dim=256, qk_norm=False, dtype=torch.float32, seed=0):
    torch.manual_seed(seed)
    attn = MoTAttention(dim=dim, n_heads=n_heads, n_kv_heads=n_kv,
                        modalities=("image", "text"), qk_norm=qk_norm)
    for m in ("image", "text"):
        nn.init.normal_(attn.o_proj[m].weight, std=0.05)
        for p in (attn.q_proj, attn.k_proj, attn.v_proj):
            nn.init.normal_(p[m].weight, std=dim ** -0.5)
    return attn.to(DEV, dtype)


@pytest.mark.parametrize("n_heads,n_kv,dtype,qk_norm", [
    (4, 2, torch.float32, False), (4, 4, torch.float32, True), (8, 1, torch.float32, False),
    (2, 1, torch.bfloat16, False), (2, 2, torch.bfloat16, True)])
def test_matches_algorithm_1(n_heads, n_kv, dtype, qk_norm):
    announce(f"mot alg1 {n_heads}/{n_kv} {dtype} qk_norm={qk_norm}")
    attn = _make(n_heads, n_kv, qk_norm=qk_norm, dtype=dtype)
    hd = attn.head_dim
    streams = {"image": torch.randn(2, 70, 256, device=DEV, dtype=dtype),
               "text": torch.randn(2, 130, 256, device=DEV, dtype=dtype)}
    rope = {"image": _rope(70, hd), "text": _rope(130, hd)}
    got = attn(streams, rope)
    want = _algorithm_1(attn, streams, rope)
    tol = 1e-4 if dtype == torch.float32 else 5e-2
    for m in ("image", "text"):
        assert got[m].shape == streams[m].shape and got[m].dtype == dtype
        assert max_abs(got[m], want[m]) <= tol, m


def test_not_causal_and_all_valid_padding_mask():
    announce("mot non-causal / kpm")
    attn = _make()
    streams = {"image": torch.randn(1, 40, 256, device=DEV),
               "text": torch.randn(1, 60, 256, device=DEV)}
    rope = {"image": _rope(40, 64), "text": _rope(60, 64)}
    got = attn(streams, rope, is_causal=False)
    want = _algorithm_1(attn, streams, rope, is_causal=False)
    for m in ("image", "text"):
        assert max_abs(got[m], want[m]) <= 1e-4
    kpm = torch.ones(1, 100, dtype=torch.bool, device=DEV)
    kpm[0, 10:25] = False  # padded video frames' tokens
    got = attn(streams, rope, key_padding_mask=kpm)
    want = _algorithm_1(attn, streams, rope, key_padding_mask=kpm)
    for m in ("image", "text"):
        assert max_abs(got[m], want[m]) <= 1e-4


def test_cross_modality_flow_and_causality():
    """Text output depends on the image stream; image output does not depend on
    the text stream under causal masking (image first)."""
    announce("mot flow")
    attn = _make(4, 4)
    rope = {"image": _rope(16, 64), "text": _rope(24, 64)}
    image = torch.randn(1, 16, 256, device=DEV)
    text_a, text_b = torch.randn(2, 1, 24, 256, device=DEV)
    out_a = attn({"image": image, "text": text_a}, rope)
    out_b = attn({"image": image, "text": text_b}, rope)
    assert torch.equal(out_a["image"], out_b["image"])
    out_c = attn({"image": torch.randn_like(image), "text": text_a}, rope)
    assert not torch.allclose(out_a["text"], out_c["text"], atol=1e-6)


def test_text_invariant_to_image_weights_when_image_is_zero():
    announce("mot zero image")
    attn1 = _make(4, 4)
    attn2 = copy.deepcopy(attn1)
    for p in (attn2.q_proj, attn2.k_proj, attn2.v_proj, attn2.o_proj):
        nn.init.normal_(p["image"].weight)
    rope = {"image": _rope(8, 64), "text": _rope(16, 64)}
    zero = torch.zeros(1, 8, 256, device=DEV)
    text = torch.randn(1, 16, 256, device=DEV)
    o1 = attn1({"image": zero, "text": text}, rope)["text"]
    o2 = attn2({"image": zero, "text": text}, rope)["text"]
    assert max_abs(o1, o2.cpu()) <= 1e-6


def test_backward_matches_and_reaches_every_projection():
    """Gradients of every per-modality projection against autograd through the
    CPU restatement (float64)."""
    announce("mot backward")
    attn = _make(4, 2)
    rope = {"image": _rope(33, 64), "text": _rope(47, 64)}
    streams = {"image": torch.randn(2, 33, 256, device=DEV),
               "text": torch.randn(2, 47, 256, device=DEV)}
    out = attn(streams, rope)
    (out["image"].square().sum() + out["text"].sum()).backward()
    cpu = copy.deepcopy(attn).cpu().double()
    cpu.zero_grad()
    x_cpu = {m: s.detach().cpu().double() for m, s in streams.items()}
    # literal reference composition in float64 on the CPU, differentiated by autograd
    qs, ks, vs = [], [], []
    for m in ("image", "text"):
        x = x_cpu[m]
        t = x.shape[1]
        q = cpu.q_proj[m](x).view(2, t, -1, 64).transpose(1, 2)
        k = cpu.k_proj[m](x).view(2, t, -1, 64).transpose(1, 2)
        v = cpu.v_proj[m](x).view(2, t, -1, 64).transpose(1, 2)
        c, s = (r.cpu().double()[:t] for r in rope[m])
        qs.append(ref.apply_rope(q, c, s))
        ks.append(ref.apply_rope(k, c, s))
        vs.append(v)
    q, k, v = torch.cat(qs, 2), torch.cat(ks, 2), torch.cat(vs, 2)
    o = F.scaled_dot_product_attention(q, k.repeat_interleave(2, 1), v.repeat_interleave(2, 1),
                                       is_causal=True).transpose(1, 2)
    o_img = cpu.o_proj["image"](o[:, :33].reshape(2, 33, -1))
    o_txt = cpu.o_proj["text"](o[:, 33:].reshape(2, 47, -1))
    (o_img.square().sum() + o_txt.sum()).backward()
    for name, p in attn.named_parameters():
        want = dict(cpu.named_parameters())[name].grad
        assert p.grad is not None and p.grad.abs().sum() > 0, name
        # weight gradients sum over every position: per-element 1e-4 absolute
        # plus 1e-4 relative (module level, after the fp32 projections)
        err = (p.grad.detach().cpu().double() - want).abs()
        ratio = (err / (1e-4 * (1.0 + want.abs()))).max().item()
        print(f"[{name}] max-abs err {err.max().item():.3e}; worst err/bound {ratio:.3f}")
        assert ratio <= 1.0, name
