"""GPU parity of the backward (kf_attn_bwd via autograd of kf::attn_fwd).

Gradients grow with sequence length, so their tolerance is scaled: max-abs
error <= tol * max(1, max |reference|), tol = 1e-5 (float32) or 2e-2 (bf16),
against the float64 oracle from the same inputs.
"""

from __future__ import annotations

import pytest
import torch

import make_fixtures as mf
from gpu_util import DEV, announce, load_fixture, rel_max, seeded
from kempnerforge_amd import ops
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def _grads(q, k, v, do, cos, sin, causal=True):
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    out = ops.attention(qd, kd, vd, cos.to(DEV), sin.to(DEV), causal=causal)
    out.backward(do.to(DEV))
    torch.cuda.synchronize()
    return out, qd.grad, kd.grad, vd.grad


@pytest.mark.parametrize("name", list(mf.ATTN_CASES))
def test_fixture(name):
    announce(f"bwd fixture {name}")
    fx = load_fixture(name)
    dtype = mf.ATTN_CASES[name][0]
    q, k, v, do, cos, sin = mf.attn_inputs(*mf.ATTN_CASES[name])
    _, dq, dk, dv = _grads(q, k, v, do, cos, sin)
    for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        assert rel_max(got, torch.from_numpy(fx[key])) <= TOL[dtype], key


SHAPES = [
    (torch.bfloat16, 2, 200, 4, 4, 64),
    (torch.bfloat16, 1, 300, 8, 1, 128),
    (torch.bfloat16, 1, 130, 6, 2, 128),
    (torch.bfloat16, 1, 64, 4, 2, 32),
    (torch.float32, 1, 100, 8, 2, 128),
]


@pytest.mark.parametrize("cfg", SHAPES, ids=lambda c: "-".join(map(str, c)))
@pytest.mark.parametrize("causal", [True, False])
def test_shapes(cfg, causal):
    dtype, B, S, Hq, Hkv, D = cfg
    announce(f"bwd {cfg} causal={causal}")
    q = seeded((B, S, Hq, D), 0, dtype)
    k = seeded((B, S, Hkv, D), 1, dtype)
    v = seeded((B, S, Hkv, D), 2, dtype)
    do = seeded((B, S, Hq, D), 3, dtype)
    cos, sin = ref.rope_tables(D, S, 5e5)
    _, dq, dk, dv = _grads(q, k, v, do, cos, sin, causal)
    dq_r, dk_r, dv_r = ref.attention_bwd(q, k, v, cos, sin, do, causal=causal)
    assert rel_max(dq, dq_r) <= TOL[dtype]
    assert rel_max(dk, dk_r) <= TOL[dtype]
    assert rel_max(dv, dv_r) <= TOL[dtype]


def test_llama8b_shape_one_group():
    """C3 at full size (B=4, S=4096, Hq=32, Hkv=8, D=128): the backward of KV
    group (b=1, g=6) against the oracle (groups are independent), plus
    determinism of a second backward."""
    B, S, Hq, Hkv, D = 4, 4096, 32, 8, 128
    announce("bwd 8B shape")
    q = seeded((B, S, Hq, D), 0, torch.bfloat16)
    k = seeded((B, S, Hkv, D), 1, torch.bfloat16)
    v = seeded((B, S, Hkv, D), 2, torch.bfloat16)
    do = seeded((B, S, Hq, D), 3, torch.bfloat16)
    cos, sin = ref.rope_tables(D, S, 5e5)
    _, dq, dk, dv = _grads(q, k, v, do, cos, sin)
    _, dq2, dk2, dv2 = _grads(q, k, v, do, cos, sin)
    assert torch.equal(dq, dq2) and torch.equal(dk, dk2) and torch.equal(dv, dv2)
    b, g = 1, 6
    hs = slice(4 * g, 4 * g + 4)
    dq_r, dk_r, dv_r = ref.attention_bwd(q[b:b + 1, :, hs], k[b:b + 1, :, g:g + 1],
                                         v[b:b + 1, :, g:g + 1], cos, sin, do[b:b + 1, :, hs])
    assert rel_max(dq[b:b + 1, :, hs], dq_r) <= 2e-2
    assert rel_max(dk[b:b + 1, :, g:g + 1], dk_r) <= 2e-2
    assert rel_max(dv[b:b + 1, :, g:g + 1], dv_r) <= 2e-2
