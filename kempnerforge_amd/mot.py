"""Drop-in ``MoTAttention`` (Mixture-of-Transformers global attention) on the
gfx950 kernels.

Mirrors ``kempnerforge/model/mot.py:35-207``: the same constructor, the same
per-modality ``nn.ModuleDict`` projections and optional per-modality QK norms
(so ``q_proj.{m}.weight`` ... ``k_norm.{m}.weight`` state-dict keys load
unchanged), zero-initialised ``o_proj``, and the same ``forward(streams, rope,
is_causal, key_padding_mask)`` contract.

Each modality's RoPE positions restart at 0 (``rope[m]`` counts from position
0 within that modality, ``kempnerforge/model/transformer.py:474-481``).  The
kernels index their RoPE tables by the token's row, so the per-token position
input is the concatenation of the per-modality tables in stream order: row s
of the concatenated table is the table row of token s's position inside its
modality.  With that, one ``kf::attn_fwd`` / ``kf::attn_bwd`` over the
concatenated sequence is the reference's RoPE + ``torch.cat`` +
``repeat_interleave`` + SDPA (``:162-186``), forward and backward.

With ``key_padding_mask`` (``:188-198``: causal AND valid keys, the NaN guard
unmasking rows that see no key) the same kernels apply the validity test per
tile instead of materialising the ``(B, 1, S, S)`` mask.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from kempnerforge_amd import ops
from kempnerforge_amd.norm import RMSNorm


class MoTAttention(nn.Module):
    """Per-modality Q/K/V/O projections; one global attention over all modalities."""

    def __init__(
        self,
        dim: int,
        n_heads: int,
        n_kv_heads: int,
        modalities: tuple[str, ...],
        head_dim: int | None = None,
        qk_norm: bool = False,
    ) -> None:
        super().__init__()
        if not modalities:
            raise ValueError("MoTAttention requires at least one modality")
        if n_kv_heads <= 0 or n_heads % n_kv_heads != 0:
            raise ValueError(
                f"MoTAttention: n_heads={n_heads} must be a positive multiple of "
                f"n_kv_heads={n_kv_heads}"
            )
        self.modalities = tuple(modalities)
        self.n_heads = n_heads
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim or (dim // n_heads)
        self.n_rep = n_heads // n_kv_heads
        hd = self.head_dim
        self.q_proj = nn.ModuleDict({m: nn.Linear(dim, n_heads * hd, bias=False)
                                     for m in self.modalities})
        self.k_proj = nn.ModuleDict({m: nn.Linear(dim, n_kv_heads * hd, bias=False)
                                     for m in self.modalities})
        self.v_proj = nn.ModuleDict({m: nn.Linear(dim, n_kv_heads * hd, bias=False)
                                     for m in self.modalities})
        self.o_proj = nn.ModuleDict({m: nn.Linear(n_heads * hd, dim, bias=False)
                                     for m in self.modalities})
        for m in self.modalities:
            nn.init.zeros_(self.o_proj[m].weight)
        if qk_norm:
            self.q_norm: nn.ModuleDict | None = nn.ModuleDict({m: RMSNorm(hd)
                                                               for m in self.modalities})
            self.k_norm: nn.ModuleDict | None = nn.ModuleDict({m: RMSNorm(hd)
                                                               for m in self.modalities})
        else:
            self.q_norm = None
            self.k_norm = None

    def forward(
        self,
        streams: dict[str, torch.Tensor],
        rope: dict[str, tuple[torch.Tensor, torch.Tensor]],
        is_causal: bool = True,
        key_padding_mask: torch.Tensor | None = None,
    ) -> dict[str, torch.Tensor]:
        """``streams[m]`` ``(B, T_m, dim)``, ``rope[m]`` ``(cos, sin)`` of shape
        ``(T_m, head_dim // 2)`` from position 0 -> per-modality ``(B, T_m, dim)``."""
        if set(streams.keys()) != set(self.modalities):
            raise ValueError(
                f"MoTAttention.forward: streams keys {sorted(streams.keys())} "
                f"do not match construction-time modalities {sorted(self.modalities)}"
            )
        batch = next(iter(streams.values())).shape[0]
        qs, ks, vs, coss, sins, lengths = [], [], [], [], [], []
        for m in self.modalities:
            x_m = streams[m]
            t_m = x_m.shape[1]
            q_m = self.q_proj[m](x_m).view(batch, t_m, -1, self.head_dim)
            k_m = self.k_proj[m](x_m).view(batch, t_m, -1, self.head_dim)
            v_m = self.v_proj[m](x_m).view(batch, t_m, -1, self.head_dim)
            if self.q_norm is not None:
                q_m = self.q_norm[m](q_m)
                k_m = self.k_norm[m](k_m)  # type: ignore[index]
            cos_m, sin_m = rope[m]
            qs.append(q_m)
            ks.append(k_m)
            vs.append(v_m)
            coss.append(cos_m[:t_m])
            sins.append(sin_m[:t_m])
            lengths.append(t_m)
        # BSHD, concatenated along the sequence in modality order; the tables
        # carry each token's own (modality-local) position
        q = torch.cat(qs, dim=1)
        k = torch.cat(ks, dim=1)
        v = torch.cat(vs, dim=1)
        cos = torch.cat(coss, dim=0)
        sin = torch.cat(sins, dim=0)
        if key_padding_mask is not None:
            # the reference's explicit mask is always causal (is_causal unused)
            out = ops.attention(q, k, v, cos, sin, causal=True,
                                key_padding_mask=key_padding_mask)
        else:
            out = ops.attention(q, k, v, cos, sin, causal=is_causal)
        out_streams: dict[str, torch.Tensor] = {}
        offset = 0
        for m, t_m in zip(self.modalities, lengths):
            o_m = out[:, offset:offset + t_m].reshape(batch, t_m, -1)
            out_streams[m] = self.o_proj[m](o_m)
            offset += t_m
        return out_streams
