"""The product's RoPE tables against the pinned oracle tables.

``kempnerforge_amd.position.precompute_rope_frequencies`` feeds every kernel
(and the module tests hand the same tables to the GPU and the oracle), so it
is checked here on its own: bit for bit against ``oracle.rope_tables`` (the
restatement of kempnerforge/model/position.py:12-40, pinned by a float64
closed form in test_oracle.py), and directly against that closed form.
"""

from __future__ import annotations

import math

import pytest
import torch

from kempnerforge_amd.position import precompute_rope_frequencies
from oracle import attention_ref as ref

# the configurations' tables: C1 (D=64, theta 1e4), C2-C4 (D=128, theta 5e5),
# C5 (S=16384), decode (8193 positions), an odd theta
CASES = [(64, 256, 1e4), (128, 4096, 5e5), (128, 16384, 5e5), (128, 8193, 5e5), (32, 100, 1234.5)]


@pytest.mark.parametrize("D,S,theta", CASES)
def test_equals_oracle_bit_for_bit(D, S, theta):
    cos, sin = precompute_rope_frequencies(D, S, theta)
    rc, rs = ref.rope_tables(D, S, theta)
    assert cos.dtype == torch.float32 and cos.shape == (S, D // 2)
    assert torch.equal(cos, rc) and torch.equal(sin, rs)


@pytest.mark.parametrize("D,S,theta", CASES)
def test_closed_form(D, S, theta):
    """cos/sin of pos * theta^(-2i/D) in float64, within the float32 rounding
    of the frequency (relative 2^-23) carried through pos * freq."""
    cos, sin = precompute_rope_frequencies(D, S, theta)
    pos = torch.arange(S, dtype=torch.float64).unsqueeze(1)
    i = torch.arange(D // 2, dtype=torch.float64).unsqueeze(0)
    ang = pos * theta ** (-2.0 * i / D)
    # float32 frequency and product: |d angle| <= 3 * 2^-24 * angle (+ argument rounding)
    tol = 3 * 2.0 ** -24 * ang.abs() + 2.0 ** -23
    assert ((cos.double() - ang.cos()).abs() <= tol + 1e-7).all()
    assert ((sin.double() - ang.sin()).abs() <= tol + 1e-7).all()
    assert math.isclose(float(cos[0, 0]), 1.0) and float(sin[0, 0]) == 0.0
