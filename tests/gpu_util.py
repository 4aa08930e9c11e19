"""Shared helpers for the GPU parity tests."""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
if GOLDEN not in sys.path:
    sys.path.insert(0, GOLDEN)

DEV = torch.device("cuda:0") if torch.cuda.is_available() else None


def seeded(shape, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


def max_abs(got, want) -> float:
    return (got.detach().float().cpu().double() - want.double()).abs().max().item()


def rel_max(got, want) -> float:
    """max-abs error divided by max(1, max |want|): the tolerance scale used for
    gradients, whose magnitude grows with sequence length."""
    return max_abs(got, want) / max(1.0, want.abs().max().item())


def load_fixture(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


def announce(msg: str) -> None:
    print(f"[gpu case] {msg}", flush=True)
