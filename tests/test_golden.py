"""The oracle reproduces the committed golden fixtures (tests/golden/*.npz)."""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

from oracle import attention_ref as ref

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)
import make_fixtures as mf  # noqa: E402


def _load(name):
    return np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False)


@pytest.mark.parametrize("name", list(mf.ATTN_CASES))
def test_attention_fixture(name):
    fx = _load(name)
    q, k, v, do, cos, sin = mf.attn_inputs(*mf.ATTN_CASES[name])
    assert mf.digest(q, k, v, do) == str(fx["sha256"]), "input generator changed"
    out, lse = ref.attention_fwd(q, k, v, cos, sin)
    assert np.allclose(out.float().numpy(), fx["out"], atol=1e-6)
    assert np.allclose(lse.float().numpy(), fx["lse"], atol=1e-6)
    if name.startswith("c1"):  # backward is slow-ish; the bf16 case is checked on GPU
        dq, dk, dv = ref.attention_bwd(q, k, v, cos, sin, do)
        for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
            assert np.allclose(got.float().numpy(), fx[key], atol=1e-5), key


def test_decode_fixture():
    fx = _load("decode_bf16")
    q, kn, vn, kc, vc, lens, cos, sin = mf.decode_inputs(**mf.DECODE_CASE)
    assert mf.digest(q, kn, vn, kc, vc, lens) == str(fx["sha256"])
    out, kc2, _ = ref.decode_step(q, kn, vn, kc, vc, lens, cos, sin)
    assert np.allclose(out.float().numpy(), fx["out"], atol=1e-6)
    b = torch.arange(lens.numel())
    assert np.array_equal(kc2[b, :, lens.long()].float().numpy(), fx["k_written"])


def test_capture_fixture():
    fx = _load("capture_fp32")
    c = mf.CAPTURE_CASE
    q, k, v, _, cos, sin = mf.attn_inputs(c["dtype"], c["B"], c["S"], c["Hq"], c["Hkv"], c["D"],
                                          c["theta"])
    assert mf.digest(q, k, v) == str(fx["sha256"])
    out, p = ref.capture(q, k, v, cos, sin)
    assert np.allclose(p.float().numpy(), fx["probs"], atol=1e-7)
    assert np.allclose(out.float().numpy(), fx["out"], atol=1e-6)
