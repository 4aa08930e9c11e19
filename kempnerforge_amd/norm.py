"""RMSNorm used for the optional per-head QK normalisation.

Same module, parameter name and arithmetic as
``kempnerforge/model/norm.py:11-27`` (float32 internally, cast back), so
``q_norm.weight`` / ``k_norm.weight`` state-dict keys load unchanged.
"""

from __future__ import annotations

import torch
import torch.nn as nn


class RMSNorm(nn.Module):
    """Root-mean-square layer normalisation (Llama style)."""

    def __init__(self, dim: int, eps: float = 1e-5) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        dtype = x.dtype
        x = x.float()
        norm = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps)
        return (norm * self.weight).to(dtype)
