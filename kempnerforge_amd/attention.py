"""Drop-in ``Attention`` and ``KVCache`` running on the gfx950 HIP kernels.

Mirrors ``kempnerforge/model/attention.py``: same constructor and forward
signatures, attributes, submodule names (so state-dict keys
``{q,k,v,o}_proj.weight`` and ``{q,k}_norm.weight`` are unchanged), capture
flag and ``last_attention_weights`` on the CPU.  What changes is below the
projections: RoPE, the GQA expansion, the attention itself, the cache update
and the capture math run in the kernels of ``libkf_attn.so``.

Paths (reference lines in ``kempnerforge/model/attention.py``):

* training / no cache (``:228-231`` with ``is_causal=True``): ``kf::attn_fwd``,
  differentiable through ``kf::attn_bwd``;
* decode, one token with a cache (``:169-175,229-231``): ``kf_attn_decode``;
* prefill with a cache (``:169-175,229-231``): ``kf_kv_cache_append`` then the
  forward over the cache with the reference's top-left causal alignment;
* capture (``:184-189,238-280``): ``kf_attn_capture``;
* explicit masks without a cache (``:190-227``): ``doc_ids`` (packed
  documents) and ``key_padding_mask`` (padded keys, with the reference's NaN
  guard) run in the same kernels, the conditions applied per tile, so no
  ``[B,1,S,S]`` mask is built (capture included);
* capture with a cache and an explicit mask (``:169-170,252-271``): the
  reference appends to the cache and then builds an ``[S, S_kv]`` mask that
  only broadcasts against the ``[B,1,S,S]`` document / padding masks when the
  cache was empty.  Here the new tokens are appended likewise; on an empty
  cache the capture kernel runs with the masks (the cache then holds exactly
  this call's rotated keys), on a non-empty one a RuntimeError is raised, as
  the reference's mask construction raises one.
"""

from __future__ import annotations

import contextlib

import torch
import torch.nn as nn
from torch.nn.attention import SDPBackend, sdpa_kernel

from kempnerforge_amd import ops
from kempnerforge_amd.norm import RMSNorm

_SDPA_BACKENDS = {
    "flash": SDPBackend.FLASH_ATTENTION,
    "efficient": SDPBackend.EFFICIENT_ATTENTION,
    "cudnn": SDPBackend.CUDNN_ATTENTION,
    "math": SDPBackend.MATH,
}


class KVCache:
    """Pre-allocated KV cache ``[B, n_kv_heads, max_seq_len, head_dim]``.

    Same storage and API as ``kempnerforge/model/attention.py:29-70``: keys are
    stored after RoPE and before GQA expansion; ``seq_len`` is the batch's fill
    level.  ``lens`` is the fill level per sequence as an int32 device tensor,
    which the decode kernel reads without a host synchronisation.

    Beyond the reference (whose single ``seq_len`` forces one length for the
    whole batch): ``set_lengths`` gives each sequence its own fill level (a
    ragged batch, e.g. right-padded prompts of different lengths), and
    ``use_rope_tables`` hands over the full RoPE tables so that each sequence
    decodes at its own position.  ``seq_len`` is then the longest fill level.
    """

    def __init__(
        self,
        batch_size: int,
        max_seq_len: int,
        n_kv_heads: int,
        head_dim: int,
        dtype: torch.dtype,
        device: torch.device,
    ) -> None:
        self.k = torch.zeros(batch_size, n_kv_heads, max_seq_len, head_dim, dtype=dtype,
                             device=device)
        self.v = torch.zeros(batch_size, n_kv_heads, max_seq_len, head_dim, dtype=dtype,
                             device=device)
        self.lens = torch.zeros(batch_size, dtype=torch.int32, device=device)
        self._seq_len = 0
        self.rope_tables: tuple[torch.Tensor, torch.Tensor] | None = None
        self.ragged = False

    @property
    def max_seq_len(self) -> int:
        return self.k.shape[2]

    @property
    def seq_len(self) -> int:
        """Fill level of the batch (the longest sequence's for a ragged cache)."""
        return self._seq_len

    @seq_len.setter
    def seq_len(self, value: int) -> None:
        """Writable as in the reference (a caller may rewind a cache to reuse
        it): every sequence is set to this fill level, so the per-sequence
        ``lens`` the decode kernel reads follow (no host synchronisation)."""
        value = int(value)
        if not 0 <= value <= self.max_seq_len:
            raise ValueError(f"seq_len must lie in [0, {self.max_seq_len}] (got {value})")
        self._seq_len = value
        self.lens.fill_(value)
        self.ragged = False

    def update(self, k_new: torch.Tensor, v_new: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Append already-rotated ``(B, n_kv_heads, new_len, head_dim)`` keys and
        values; return the filled ``[:, :, :seq_len]`` views
        (``kempnerforge/model/attention.py:54-70``)."""
        new_len = k_new.shape[2]
        end = self.seq_len + new_len
        self.k[:, :, self.seq_len : end] = k_new
        self.v[:, :, self.seq_len : end] = v_new
        self._advance(new_len)
        return self.k[:, :, :end], self.v[:, :, :end]

    def set_lengths(self, lengths) -> None:
        """Per-sequence fill levels (a list of ints, or an int tensor at the
        cost of one host synchronisation).  Positions at or past a sequence's
        level are free: its next decode step writes there."""
        if isinstance(lengths, torch.Tensor):
            lengths = [int(x) for x in lengths.tolist()]
        lengths = [int(x) for x in lengths]
        if len(lengths) != self.lens.shape[0]:
            raise ValueError(f"need {self.lens.shape[0]} lengths (got {len(lengths)})")
        if min(lengths) < 0 or max(lengths) > self.max_seq_len:
            raise ValueError(f"lengths must lie in [0, {self.max_seq_len}]")
        self.lens.copy_(torch.tensor(lengths, dtype=torch.int32))
        self._seq_len = max(lengths)
        self.ragged = len(set(lengths)) > 1

    def use_rope_tables(self, cos: torch.Tensor, sin: torch.Tensor) -> None:
        """Full ``(positions, head_dim // 2)`` RoPE tables; decode then rotates
        each sequence at its own position ``lens[b]`` (needed for a ragged cache)."""
        self.rope_tables = (cos, sin)

    def _decode_tables(self, cos: torch.Tensor, sin: torch.Tensor):
        """(cos, sin, row offset) for a decode step: the caller's tables start
        at position ``seq_len``; attached full tables start at 0."""
        if self.rope_tables is not None:
            return self.rope_tables[0], self.rope_tables[1], 0
        if self.ragged:
            raise ValueError("a ragged KV cache needs the full RoPE tables: call use_rope_tables")
        return cos, sin, self.seq_len

    def _check_room(self, new_len: int) -> None:
        if self.seq_len + new_len > self.max_seq_len:
            raise ValueError(
                f"KV cache overflow: {self.seq_len} cached + {new_len} new tokens exceeds "
                f"max_seq_len {self.max_seq_len}"
            )

    def _advance(self, new_len: int) -> None:
        self._seq_len += new_len
        self.lens.add_(new_len)


class Attention(nn.Module):
    """Grouped-Query Attention with RoPE on gfx950 HIP kernels."""

    def __init__(
        self,
        dim: int,
        n_heads: int,
        n_kv_heads: int,
        head_dim: int | None = None,
        qk_norm: bool = False,
        sdpa_backend: str = "auto",
    ) -> None:
        super().__init__()
        self.n_heads = n_heads
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim or (dim // n_heads)
        self.n_rep = n_heads // n_kv_heads
        # Kept for configuration compatibility; the HIP path has one kernel per
        # operation and does not dispatch on it.
        self.sdpa_backend = sdpa_backend

        self.q_proj = nn.Linear(dim, n_heads * self.head_dim, bias=False)
        self.k_proj = nn.Linear(dim, n_kv_heads * self.head_dim, bias=False)
        self.v_proj = nn.Linear(dim, n_kv_heads * self.head_dim, bias=False)
        self.o_proj = nn.Linear(n_heads * self.head_dim, dim, bias=False)

        self.q_norm = RMSNorm(self.head_dim) if qk_norm else None
        self.k_norm = RMSNorm(self.head_dim) if qk_norm else None

        self.capture_attention_weights = False
        self.last_attention_weights: torch.Tensor | None = None

    def _sdpa_context(self):
        if self.sdpa_backend == "auto":
            return contextlib.nullcontext()
        return sdpa_kernel(_SDPA_BACKENDS[self.sdpa_backend])

    def forward(
        self,
        x: torch.Tensor,
        rope_cos: torch.Tensor,
        rope_sin: torch.Tensor,
        *,
        kv_cache: KVCache | None = None,
        doc_ids: torch.Tensor | None = None,
        key_padding_mask: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """x ``(B, S, dim)``, rope tables ``(S, head_dim // 2)`` for positions
        ``start_pos .. start_pos + S - 1`` → ``(B, S, dim)``."""
        batch, seq_len, _ = x.shape
        # BSHD views; -1 heads so tensor-parallel shards work (reference :148-152)
        q = self.q_proj(x).view(batch, seq_len, -1, self.head_dim)
        k = self.k_proj(x).view(batch, seq_len, -1, self.head_dim)
        v = self.v_proj(x).view(batch, seq_len, -1, self.head_dim)
        masked = doc_ids is not None or key_padding_mask is not None
        decode = (kv_cache is not None and seq_len == 1 and not masked
                  and not self.capture_attention_weights)
        # decode applies the QK-norm inside its kernels (one eps for both)
        fuse_norm = (decode and self.q_norm is not None
                     and self.q_norm.eps == self.k_norm.eps)  # type: ignore[union-attr]
        if self.q_norm is not None and not fuse_norm:
            q = self.q_norm(q)
            k = self.k_norm(k)  # type: ignore[reportOptionalCall]

        if self.capture_attention_weights:
            if masked and kv_cache is not None:
                # the reference appends first (:169-170), then builds the masks
                start = kv_cache.seq_len
                self._append(k, v, rope_cos, rope_sin, kv_cache)
                if start != 0:
                    raise RuntimeError(
                        "capture with doc_ids / key_padding_mask over a non-empty KV cache: "
                        f"the causal mask is [{seq_len}, {start + seq_len}] but the "
                        f"document / padding masks cover {seq_len} keys")
                # empty cache: its keys are this call's, rotated as the kernel rotates them
                kv_cache = None
            out, probs = self._capture(q, k, v, rope_cos, rope_sin, kv_cache, doc_ids,
                                       key_padding_mask)
            self.last_attention_weights = probs.to(q.dtype).detach().cpu()
        elif masked:
            assert kv_cache is None, (
                "doc_ids / key_padding_mask are not supported with kv_cache decode "
                "(would build an incorrect causal mask)."
            )
            out = ops.attention(q, k, v, rope_cos, rope_sin, causal=True, doc_ids=doc_ids,
                                key_padding_mask=key_padding_mask)
        elif kv_cache is None:
            out = ops.attention(q, k, v, rope_cos, rope_sin, causal=True)
        elif seq_len == 1:
            kv_cache._check_room(1)
            cos_t, sin_t, row0 = kv_cache._decode_tables(rope_cos, rope_sin)
            out = ops.decode_raw(
                q, k, v, kv_cache.k, kv_cache.v, kv_cache.lens, cos_t, sin_t,
                rope_row_offset=row0, max_len=kv_cache.seq_len + 1,
                q_norm_weight=self.q_norm.weight if fuse_norm else None,  # type: ignore[union-attr]
                k_norm_weight=self.k_norm.weight if fuse_norm else None,  # type: ignore[union-attr]
                norm_eps=self.q_norm.eps if fuse_norm else 1e-5)  # type: ignore[union-attr]
            kv_cache._advance(1)
        else:
            kc, vc = self._append(k, v, rope_cos, rope_sin, kv_cache)
            out, _ = ops.fwd_raw(q, kc, vc, rope_cos, rope_sin, causal=True, k_rotated=True,
                                 k_layout="bhsd")

        out = out.reshape(batch, seq_len, -1)
        return self.o_proj(out)

    @staticmethod
    def _append(k, v, rope_cos, rope_sin, kv_cache: KVCache):
        new_len = k.shape[1]
        if kv_cache.ragged:
            raise ValueError("prefill into a ragged KV cache is not supported; prefill the "
                             "right-padded batch first, then call set_lengths")
        kv_cache._check_room(new_len)
        start = kv_cache.seq_len
        ops.cache_append_raw(k, v, rope_cos, rope_sin, kv_cache.k, kv_cache.v, start)
        kv_cache._advance(new_len)
        end = kv_cache.seq_len
        return kv_cache.k[:, :, :end], kv_cache.v[:, :, :end]

    def _capture(self, q, k, v, rope_cos, rope_sin, kv_cache, doc_ids=None,
                 key_padding_mask=None):
        """Manual-attention replacement (``kempnerforge/model/attention.py:238-280``)."""
        if kv_cache is None:
            out, probs, _ = ops.capture_raw(q, k, v, rope_cos, rope_sin, causal=True,
                                            k_rotated=False, doc_ids=doc_ids,
                                            key_padding_mask=key_padding_mask)
            return out, probs
        seq_len = q.shape[1]
        kc, vc = self._append(k, v, rope_cos, rope_sin, kv_cache)
        out, probs, _ = ops.capture_raw(q, kc, vc, rope_cos, rope_sin, causal=seq_len > 1,
                                        k_rotated=True, k_layout="bhsd")
        return out, probs
