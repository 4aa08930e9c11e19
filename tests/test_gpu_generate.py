"""Ragged-batch decode, fused QK-norm and generation on the GPU.

The reference decodes one length for the whole batch (KVCache.seq_len,
kempnerforge/model/attention.py:52), normalises q and k in separate ops
(:155-157) and syncs the host every step (generate.py:116-121).  Checked here:
the fused QK-norm decode against RMSNorm followed by the plain decode and
against the oracle; a ragged batch against each sequence decoded alone; and
``generate`` against a cache-free greedy recomputation and against itself with
sparse end-of-sequence checks.
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch
import torch.nn as nn

from gpu_util import DEV, announce, max_abs, seeded
from kempnerforge_amd import Attention, KVCache, ops
from kempnerforge_amd.generate import generate
from kempnerforge_amd.norm import RMSNorm
from kempnerforge_amd.position import precompute_rope_frequencies
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("D,n_rep", [(128, 4), (64, 2), (32, 2)])
def test_fused_qk_norm_decode(D, n_rep):
    """kf_attn_decode with QK-norm weights == RMSNorm (reference module) then
    the plain decode, and == the oracle on the normalised rows."""
    announce(f"qk-norm decode D={D} n_rep={n_rep}")
    B, Hkv, Smax = 3, 2, 700
    Hq = Hkv * n_rep
    lens = torch.tensor([5, 333, 698], dtype=torch.int32)
    qn = seeded((B, 1, Hq, D), 0, torch.bfloat16) * 3
    kn = seeded((B, 1, Hkv, D), 1, torch.bfloat16) * 3
    vn = seeded((B, 1, Hkv, D), 2, torch.bfloat16)
    kc = seeded((B, Hkv, Smax, D), 3, torch.bfloat16)
    vc = seeded((B, Hkv, Smax, D), 4, torch.bfloat16)
    cos, sin = ref.rope_tables(D, Smax, 5e5)
    qnorm, knorm = RMSNorm(D), RMSNorm(D)
    with torch.no_grad():
        qnorm.weight.copy_(1 + 0.1 * torch.randn(D))
        knorm.weight.copy_(1 + 0.1 * torch.randn(D))
    qnorm, knorm = qnorm.to(DEV, torch.bfloat16), knorm.to(DEV, torch.bfloat16)
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
    assert max_abs(fused, plain.cpu()) <= 2e-2
    assert max_abs(fused, want) <= 2e-2
    # the cache row written for the new token: the rotated normalised key
    for b in range(B):
        L = int(lens[b])
        assert max_abs(kc1[b, :, L], kc_ref[b, :, L]) <= 2e-2


class TinyLM(nn.Module):
    """Minimal model with the reference Transformer's generation contract
    (kempnerforge/model/transformer.py:319-425): RoPE rows sliced at the first
    cache's fill level, one KVCache per layer, logits out."""

    def __init__(self, vocab=97, dim=256, n_layers=2, n_heads=4, n_kv=2, qk_norm=False,
                 max_seq_len=256):
        super().__init__()
        head_dim = dim // n_heads
        self.config = SimpleNamespace(max_seq_len=max_seq_len, n_layers=n_layers,
                                      n_kv_heads=n_kv, head_dim=head_dim, rope_theta=1e4)
        self.embed = nn.Embedding(vocab, dim)
        self.layers = nn.ModuleList(Attention(dim, n_heads, n_kv, qk_norm=qk_norm)
                                    for _ in range(n_layers))
        self.head = nn.Linear(dim, vocab, bias=False)
        self._rope_cos, self._rope_sin = precompute_rope_frequencies(head_dim, max_seq_len, 1e4)
        for p in self.parameters():
            nn.init.normal_(p, std=0.3)
        if qk_norm:
            for layer in self.layers:
                nn.init.normal_(layer.q_norm.weight, 1.0, 0.1)
                nn.init.normal_(layer.k_norm.weight, 1.0, 0.1)

    def forward(self, tokens, kv_caches=None):
        h = self.embed(tokens)
        start = kv_caches[0].seq_len if kv_caches is not None else 0
        S = tokens.shape[1]
        cos = self._rope_cos[start:start + S].to(h.device)
        sin = self._rope_sin[start:start + S].to(h.device)
        for i, layer in enumerate(self.layers):
            h = h + layer(h, cos, sin, kv_cache=kv_caches[i] if kv_caches is not None else None)
        return self.head(h)


def _greedy_no_cache(model, prompt, n):
    seq = prompt
    with torch.no_grad():
        for _ in range(n):
            nxt = model(seq)[:, -1].argmax(-1)
            seq = torch.cat([seq, nxt[:, None]], 1)
    return seq


@pytest.mark.parametrize("qk_norm", [False, True])
def test_generate_greedy_matches_recomputation(qk_norm):
    announce(f"generate greedy qk_norm={qk_norm}")
    torch.manual_seed(0)
    model = TinyLM(qk_norm=qk_norm).to(DEV)  # float32: generic kernels, 1e-6 agreement
    prompt = torch.randint(0, 97, (3, 11), device=DEV)
    out = generate(model, prompt, 20, temperature=0)
    assert torch.equal(out, _greedy_no_cache(model, prompt, 20))


@pytest.mark.parametrize("dtype,qk_norm", [(torch.float32, False), (torch.float32, True),
                                           (torch.bfloat16, True)])
def test_ragged_batch_matches_each_sequence_alone(dtype, qk_norm):
    """Right-padded prompts of lengths 3, 17, 9 decoded as one ragged batch
    give each sequence the continuation it gets alone (float32: identical
    tokens; bfloat16 on the MFMA decode with fused QK-norm: the first-step
    logits agree and the tokens of the first steps match)."""
    announce(f"ragged generate {dtype} qk_norm={qk_norm}")
    torch.manual_seed(1)
    n_heads, n_kv = (8, 2) if dtype == torch.bfloat16 else (4, 2)
    model = TinyLM(dim=1024 if dtype == torch.bfloat16 else 256, n_heads=n_heads, n_kv=n_kv,
                   qk_norm=qk_norm).to(DEV, dtype)
    lens = [3, 17, 9]
    prompt = torch.randint(0, 97, (3, 17), device=DEV)
    steps = 12 if dtype == torch.float32 else 4
    out = generate(model, prompt, steps, temperature=0, prompt_lens=lens)
    for b, n in enumerate(lens):
        alone = generate(model, prompt[b:b + 1, :n], steps, temperature=0)
        assert torch.equal(out[b, : n + steps], alone[0]), b
    # the per-sequence RoPE position is what makes this work: decoding the
    # ragged cache at the batch's single fill level would not match
    caches = [KVCache(3, 64, n_kv, model.config.head_dim, dtype, DEV) for _ in range(2)]
    with torch.no_grad():
        model(prompt, kv_caches=caches)
        for c in caches:
            c.set_lengths(lens)
        with pytest.raises(ValueError):
            model(prompt[:, :1], kv_caches=caches)  # ragged without full RoPE tables


def test_eos_checks_every_n_steps_same_output():
    announce("generate eos_check_every")
    torch.manual_seed(2)
    model = TinyLM(vocab=5).to(DEV)  # tiny vocabulary: EOS (token 0) comes soon
    prompt = torch.randint(1, 5, (4, 6), device=DEV)
    a = generate(model, prompt, 40, temperature=0, eos_token_id=0)
    b = generate(model, prompt, 40, temperature=0, eos_token_id=0, eos_check_every=7)
    assert torch.equal(a, b)
    torch.manual_seed(3)
    c = generate(model, prompt, 40, temperature=0.8, top_k=3, eos_token_id=0)
    torch.manual_seed(3)
    d = generate(model, prompt, 40, temperature=0.8, top_k=3, eos_token_id=0, eos_check_every=5)
    assert torch.equal(c, d)
