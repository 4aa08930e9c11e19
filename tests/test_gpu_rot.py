"""GPU tests of the rotated-operand pair (kf_attn_fwd_rot / kf_attn_bwd_rot).

The forward also writes q and k after RoPE in the backward's layout, and the
backward reads them instead of q and k.  Checked here: rot holds exactly the
oracle's bf16 rotation of q and k (apply_rope, every product rounded as the
reference's eager ops round it) with zero rows past S, and out, lse, dq, dk,
dv equal the plain entry points' bit for bit (masked and unmasked, causal and
full, dS records kept or not, S not a multiple of 128).
"""

from __future__ import annotations

import pytest
import torch

from gpu_util import DEV, announce, seeded
from kempnerforge_amd import ops
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu

CASES = [
    # B, S, Hq, Hkv, D, causal, mask
    (2, 200, 8, 2, 128, True, None),
    (1, 130, 4, 4, 64, True, None),
    (1, 256, 8, 1, 128, False, None),
    (2, 320, 8, 2, 128, True, "doc"),
    (2, 192, 4, 2, 64, True, "kpm"),
    (1, 1024, 32, 8, 128, True, None),
]


def _inputs(B, S, Hq, Hkv, D, mask):
    q = seeded((B, S, Hq, D), 0, torch.bfloat16)
    k = seeded((B, S, Hkv, D), 1, torch.bfloat16)
    v = seeded((B, S, Hkv, D), 2, torch.bfloat16)
    do = seeded((B, S, Hq, D), 3, torch.bfloat16)
    cos, sin = ref.rope_tables(D, S, 5e5)
    extra = {}
    if mask == "doc":
        g = torch.Generator().manual_seed(5)
        cuts = torch.sort(torch.randint(1, S, (B, 3), generator=g), dim=1).values
        pos = torch.arange(S).expand(B, S)
        extra["doc_ids"] = (pos[:, :, None] >= cuts[:, None, :]).sum(-1).to(torch.int32).to(DEV)
    elif mask == "kpm":
        valid = torch.ones(B, S, dtype=torch.bool)
        valid[0, :17] = False
        valid[1, S - 40:] = False
        extra["key_padding_mask"] = valid.to(DEV)
    return [t.to(DEV) for t in (q, k, v, do, cos, sin)], extra


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(map(str, c)))
def test_rot_pair_matches_plain_entry_points(case):
    B, S, Hq, Hkv, D, causal, mask = case
    announce(f"rot pair {case}")
    (q, k, v, do, cos, sin), extra = _inputs(B, S, Hq, Hkv, D, mask)
    res = ops.fwd_rot_raw(q, k, v, cos, sin, causal=causal, **extra)
    assert res is not None, "the rotated-operand path should apply"
    out_r, lse_r, rot = res
    out, lse = ops.fwd_raw(q, k, v, cos, sin, causal=causal, k_rotated=False, **extra)
    torch.cuda.synchronize()
    assert torch.equal(out_r, out) and torch.equal(lse_r, lse)

    # rot: K [B*Hkv][P][D] then Q [B*Hq][P][D], the oracle's bf16 rotation
    P = (S + 127) // 128 * 128
    kr = rot[:B * Hkv * P * D].view(B, Hkv, P, D).cpu()
    qr = rot[B * Hkv * P * D:].view(B, Hq, P, D).cpu()
    cs, sn = cos.cpu(), sin.cpu()
    assert torch.equal(kr[:, :, :S], ref.apply_rope(k.cpu().transpose(1, 2), cs, sn))
    assert torch.equal(qr[:, :, :S], ref.apply_rope(q.cpu().transpose(1, 2), cs, sn))
    assert not kr[:, :, S:].any() and not qr[:, :, S:].any()

    for low_memory in (False, True):
        g_rot = ops.bwd_rot_raw(rot, v, cos, sin, out, lse, do, causal=causal,
                                low_memory=low_memory, **extra)
        g = ops.bwd_raw(q, k, v, cos, sin, out, lse, do, causal=causal, low_memory=low_memory,
                        **extra)
        torch.cuda.synchronize()
        for a, b, name in zip(g_rot, g, ("dq", "dk", "dv")):
            assert torch.equal(a, b), f"{name} differs (low_memory={low_memory})"


def test_autograd_saves_rot_not_q_and_k():
    """The differentiable op keeps rot in place of q and k and gives the same
    gradients as the plain backward."""
    announce("rot autograd")
    (q, k, v, do, cos, sin), _ = _inputs(2, 200, 8, 2, 128, None)
    qd, kd, vd = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = ops.attention(qd, kd, vd, cos, sin, causal=True)
    saved = out.grad_fn.saved_tensors
    ids = {t.data_ptr() for t in saved if isinstance(t, torch.Tensor) and t.numel()}
    assert len(ids) >= 4  # rot, v, out, lse (and the tables)
    assert qd.data_ptr() not in ids and kd.data_ptr() not in ids
    out.backward(do)
    out2, lse2 = ops.fwd_raw(q, k, v, cos, sin, causal=True, k_rotated=False)
    dq, dk, dv = ops.bwd_raw(q, k, v, cos, sin, out2, lse2, do, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(out.detach(), out2)
    assert torch.equal(qd.grad, dq) and torch.equal(kd.grad, dk) and torch.equal(vd.grad, dv)
