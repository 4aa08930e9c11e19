"""The ops under HIP graph capture.

The C ABI takes the caller's stream, allocates nothing and never synchronises
the host, so the forward, backward and decode launches can be captured into a
graph (torch.cuda.CUDAGraph) and replayed.  Each graph is replayed several
times with new data copied into its static inputs and eager work plus host
synchronisations between the replays; every replay must equal the eager call
on the same inputs bit for bit (the kernels are deterministic).
"""

from __future__ import annotations

import pytest
import torch

from gpu_util import DEV, announce, seeded
from kempnerforge_amd import ops
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu


def _capture(fn):
    """Warm up on a side stream, then capture fn() into a graph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = fn()
    return g, outs


@pytest.mark.parametrize("D,n_rep", [(128, 4), (64, 2)])
def test_fwd_bwd_graph_replays_equal_eager(D, n_rep):
    announce(f"graph fwd+bwd D={D} n_rep={n_rep}")
    B, S, Hkv = 2, 384, 2
    Hq = Hkv * n_rep
    cos, sin = (t.to(DEV) for t in ref.rope_tables(D, S, 5e5))
    q, k, v, do = (torch.empty(B, S, h, D, device=DEV, dtype=torch.bfloat16)
                   for h in (Hq, Hkv, Hkv, Hq))

    def step():
        out, lse = ops.fwd_raw(q, k, v, cos, sin, causal=True, k_rotated=False)
        dq, dk, dv = ops.bwd_raw(q, k, v, cos, sin, out, lse, do, causal=True)
        return out, lse, dq, dk, dv

    for t, seed in zip((q, k, v, do), range(4)):
        t.copy_(seeded(t.shape, seed, torch.bfloat16))
    g, outs = _capture(step)
    for rep in range(3):
        for t, seed in zip((q, k, v, do), range(10 * rep + 10, 10 * rep + 14)):
            t.copy_(seeded(t.shape, seed, torch.bfloat16))
        g.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outs]
        want = step()  # eager, same inputs
        torch.cuda.synchronize()
        for name, a, b in zip(("out", "lse", "dq", "dk", "dv"), got, want):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from eager"


def test_decode_graph_replays_equal_eager():
    announce("graph decode")
    B, Hq, Hkv, D, Smax = 4, 8, 2, 128, 1500
    lens = torch.tensor([3, 700, 1499 - 1, 1024], dtype=torch.int32, device=DEV)
    cos, sin = (t.to(DEV) for t in ref.rope_tables(D, Smax, 5e5))
    qn = torch.empty(B, 1, Hq, D, device=DEV, dtype=torch.bfloat16)
    kn = torch.empty(B, 1, Hkv, D, device=DEV, dtype=torch.bfloat16)
    vn = torch.empty_like(kn)
    kc = seeded((B, Hkv, Smax, D), 5, torch.bfloat16).to(DEV)
    vc = seeded((B, Hkv, Smax, D), 6, torch.bfloat16).to(DEV)

    def step():
        return ops.decode_raw(qn, kn, vn, kc, vc, lens, cos, sin, rope_row_offset=0,
                              max_len=Smax)

    for t, seed in zip((qn, kn, vn), range(3)):
        t.copy_(seeded(t.shape, seed, torch.bfloat16))
    g, out = _capture(step)
    for rep in range(3):
        for t, seed in zip((qn, kn, vn), range(10 * rep + 10, 10 * rep + 13)):
            t.copy_(seeded(t.shape, seed, torch.bfloat16))
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        kc_got = kc.clone()
        want = step()  # eager: rewrites the same cache slots with the same rows
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {rep}: decode output differs from eager"
        assert torch.equal(kc_got, kc), f"replay {rep}: cache rows differ from eager"
