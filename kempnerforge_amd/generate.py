"""Autoregressive generation over the gfx950 KV-cache decode, with ragged batches.

``sample`` and ``generate`` keep the signatures and results of
``kempnerforge/model/generate.py:15-124`` (temperature, top-k, top-p sampling;
prefill, then one token per step through the model with one ``KVCache`` per
layer).  Two additions, both off by default:

* ``prompt_lens``: prompts of different lengths in one batch, right-padded in
  ``prompt_tokens``.  The prefill runs on the padded batch, then every layer's
  cache gets the per-sequence lengths and the model's full RoPE tables, so each
  sequence continues from its own last prompt token at its own position (the
  padding is overwritten as the sequence grows and is never attended).  The
  reference can only batch prompts of one length.
* ``eos_check_every``: how often the all-sequences-finished test reads back to
  the host.  The reference reads it every step (a device synchronisation per
  token); every N steps keeps the GPU queue full, and the output is cut at the
  step where the last sequence finished, so it is the same as the reference's
  (up to N - 1 decode steps are computed and discarded).

The model is the reference's ``Transformer`` contract: ``model(tokens,
kv_caches=...)`` returns logits ``(batch, seq, vocab)``, ``model.config`` has
``max_seq_len``, ``n_layers``, ``n_kv_heads``, ``head_dim`` and ``rope_theta``,
and the attention layers are ``kempnerforge_amd.Attention``.
"""

from __future__ import annotations

import torch

from kempnerforge_amd.attention import KVCache
from kempnerforge_amd.position import precompute_rope_frequencies


def sample(logits: torch.Tensor, temperature: float = 1.0, top_k: int = 0,
           top_p: float = 1.0) -> torch.Tensor:
    """Next token ids ``(batch,)`` from logits ``(batch, vocab)``: greedy at
    temperature 0, else temperature, top-k, then nucleus filtering and a
    multinomial draw (``kempnerforge/model/generate.py:15-56``)."""
    if temperature == 0:
        return logits.argmax(dim=-1)
    logits = logits / temperature
    if top_k > 0:
        top_k = min(top_k, logits.shape[-1])
        threshold = logits.topk(top_k, dim=-1).values[:, -1:]
        logits = logits.where(logits >= threshold, torch.full_like(logits, float("-inf")))
    if top_p < 1.0:
        sorted_logits, sorted_indices = logits.sort(dim=-1, descending=True)
        probs = sorted_logits.softmax(dim=-1)
        # drop tokens whose preceding cumulative mass already reaches top_p
        drop = (probs.cumsum(dim=-1) - probs) >= top_p
        sorted_logits[drop] = float("-inf")
        logits = torch.zeros_like(logits).scatter_(1, sorted_indices, sorted_logits)
    return torch.multinomial(logits.softmax(dim=-1), num_samples=1).squeeze(-1)


def _rope_tables(model, total_len: int, device):
    cos = getattr(model, "_rope_cos", None)
    sin = getattr(model, "_rope_sin", None)
    if cos is None or sin is None or cos.shape[0] < total_len:
        cfg = model.config
        cos, sin = precompute_rope_frequencies(cfg.head_dim, max(total_len, cfg.max_seq_len),
                                               theta=getattr(cfg, "rope_theta", 10000.0))
    return cos.to(device), sin.to(device)


@torch.no_grad()
def generate(
    model,
    prompt_tokens: torch.Tensor,
    max_new_tokens: int,
    *,
    temperature: float = 1.0,
    top_k: int = 0,
    top_p: float = 1.0,
    eos_token_id: int | None = None,
    prompt_lens: list[int] | None = None,
    eos_check_every: int = 1,
) -> torch.Tensor:
    """Prompt plus generated tokens, ``(batch, prompt_len + generated)``.

    Without ``prompt_lens`` this is the reference's ``generate``
    (``kempnerforge/model/generate.py:59-124``).  With it, sequence ``b``'s
    prompt is ``prompt_tokens[b, :prompt_lens[b]]``; the result holds, per row,
    the prompt followed directly by that sequence's generated tokens, padded on
    the right with ``eos_token_id`` (or 0) up to the longest row.
    """
    if eos_check_every < 1:
        raise ValueError("eos_check_every must be >= 1")
    was_training = model.training
    model.eval()
    device = prompt_tokens.device
    batch, prompt_len = prompt_tokens.shape
    cfg = model.config
    total_len = prompt_len + max_new_tokens
    if total_len > cfg.max_seq_len:
        raise ValueError(
            f"prompt ({prompt_len}) + max_new_tokens ({max_new_tokens}) = {total_len} "
            f"exceeds model max_seq_len ({cfg.max_seq_len})"
        )
    if prompt_lens is not None:
        prompt_lens = [int(n) for n in prompt_lens]
        if len(prompt_lens) != batch or min(prompt_lens) < 1 or max(prompt_lens) > prompt_len:
            raise ValueError("prompt_lens needs one length in [1, prompt_len] per sequence")
    dtype = next(model.parameters()).dtype
    caches = [KVCache(batch, total_len, cfg.n_kv_heads, cfg.head_dim, dtype, device)
              for _ in range(cfg.n_layers)]

    logits = model(prompt_tokens, kv_caches=caches)
    if prompt_lens is None:
        next_logits = logits[:, -1, :]
    else:
        last = torch.tensor([n - 1 for n in prompt_lens], device=device)
        next_logits = logits[torch.arange(batch, device=device), last]
        cos, sin = _rope_tables(model, total_len, device)
        for c in caches:
            c.set_lengths(prompt_lens)
            c.use_rope_tables(cos, sin)

    generated = []
    done = torch.zeros(batch, dtype=torch.bool, device=device)
    pending = []  # per step since the last check: all sequences finished?
    for step in range(max_new_tokens):
        token = sample(next_logits, temperature, top_k, top_p)
        generated.append(token)
        if eos_token_id is not None:
            done = done | (token == eos_token_id)
            pending.append(done.all())
            if len(pending) == eos_check_every or step + 1 == max_new_tokens:
                hits = torch.stack(pending).nonzero()
                if hits.numel():
                    # the reference stops right after the step that finished the batch
                    generated = generated[: step + 1 - len(pending) + int(hits[0, 0]) + 1]
                    break
                pending = []
        if step + 1 == max_new_tokens:
            break  # the reference's last forward only feeds a cache that is dropped
        next_logits = model(token.unsqueeze(1), kv_caches=caches)[:, -1, :]

    if was_training:
        model.train()
    gen = torch.stack(generated, dim=1) if generated else prompt_tokens[:, :0]
    if prompt_lens is None:
        return torch.cat([prompt_tokens, gen], dim=1)
    pad = eos_token_id if eos_token_id is not None else 0
    width = max(prompt_lens) + gen.shape[1]
    out = torch.full((batch, width), pad, dtype=prompt_tokens.dtype, device=device)
    for b, n in enumerate(prompt_lens):
        out[b, :n] = prompt_tokens[b, :n]
        out[b, n:n + gen.shape[1]] = gen[b]
    return out
