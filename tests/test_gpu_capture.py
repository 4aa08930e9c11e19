"""GPU parity of the capture path (kf_attn_capture): float32 probabilities
within 1e-5 of the oracle, rows summing to one, zeros above the diagonal."""

from __future__ import annotations

import pytest
import torch

import make_fixtures as mf
from gpu_util import DEV, announce, load_fixture, max_abs, seeded
from kempnerforge_amd import ops
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu


def _cap(q, k, v, cos, sin, causal=True):
    out, p, lse = ops.capture_raw(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV),
                                  causal=causal, k_rotated=False)
    torch.cuda.synchronize()
    return out, p, lse


def test_fixture_fp32():
    announce("capture fixture")
    fx = load_fixture("capture_fp32")
    c = mf.CAPTURE_CASE
    q, k, v, _, cos, sin = mf.attn_inputs(c["dtype"], c["B"], c["S"], c["Hq"], c["Hkv"], c["D"],
                                          c["theta"])
    out, p, _ = _cap(q, k, v, cos, sin)
    assert max_abs(p, torch.from_numpy(fx["probs"])) <= 1e-5
    assert max_abs(out, torch.from_numpy(fx["out"])) <= 1e-5


@pytest.mark.parametrize("cfg", [
    (torch.bfloat16, 1, 200, 8, 2, 128),
    (torch.bfloat16, 2, 130, 4, 4, 64),
    (torch.bfloat16, 1, 96, 8, 1, 128),
], ids=lambda c: "-".join(map(str, c)))
@pytest.mark.parametrize("causal", [True, False])
def test_shapes(cfg, causal):
    dtype, B, S, Hq, Hkv, D = cfg
    announce(f"capture {cfg} causal={causal}")
    q = seeded((B, S, Hq, D), 0, dtype)
    k = seeded((B, S, Hkv, D), 1, dtype)
    v = seeded((B, S, Hkv, D), 2, dtype)
    cos, sin = ref.rope_tables(D, S, 5e5)
    out, p, _ = _cap(q, k, v, cos, sin, causal)
    o_ref, p_ref = ref.capture(q, k, v, cos, sin, causal=causal)
    assert max_abs(p, p_ref) <= 1e-5
    assert max_abs(out, o_ref) <= 2e-2


def test_llama70b_capture_slice():
    """C5-cap: first 2048 tokens of the 70B shape, P [1,64,2048,2048] fp32."""
    B, S, Hq, Hkv, D = 1, 2048, 64, 8, 128
    announce("capture C5-cap")
    q = seeded((B, S, Hq, D), 0, torch.bfloat16)
    k = seeded((B, S, Hkv, D), 1, torch.bfloat16)
    v = seeded((B, S, Hkv, D), 2, torch.bfloat16)
    cos, sin = ref.rope_tables(D, S, 5e5)
    out, p, _ = _cap(q, k, v, cos, sin)
    rows = p.sum(-1)
    assert (rows - 1).abs().max().item() < 1e-5
    upper = torch.triu(torch.ones(S, S, dtype=torch.bool, device=DEV), diagonal=1)
    assert p[0][:, upper].abs().max().item() == 0.0
    g = 5  # one KV group (8 query heads) against the oracle
    hs = slice(g * 8, (g + 1) * 8)
    o_ref, p_ref = ref.capture(q[:, :, hs], k[:, :, g:g + 1], v[:, :, g:g + 1], cos, sin)
    assert max_abs(p[:, hs].cpu(), p_ref) <= 1e-5
    assert max_abs(out[:, :, hs].cpu(), o_ref) <= 2e-2
