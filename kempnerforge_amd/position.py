"""RoPE tables: the float32 cos/sin inputs the attention kernels read.

``precompute_rope_frequencies`` has the signature and values of
``kempnerforge/model/position.py:12-40``.  The rotation itself
(``kempnerforge/model/position.py:43-71``) is fused into the HIP kernels, which
cast the tables to the input dtype and round every op as the reference does.
"""

from __future__ import annotations

import torch


def precompute_rope_frequencies(
    head_dim: int,
    max_seq_len: int,
    theta: float = 10000.0,
    device: torch.device | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin tables, each float32 ``(max_seq_len, head_dim // 2)``:
    angle ``(pos, i) = pos * theta^(-2i/head_dim)``."""
    assert head_dim % 2 == 0, f"head_dim must be even, got {head_dim}"
    freqs = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device).float() / head_dim))
    positions = torch.arange(max_seq_len, device=device)
    angles = torch.outer(positions, freqs)
    return angles.cos(), angles.sin()
