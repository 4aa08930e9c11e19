"""Write the golden fixtures under tests/golden/ from the CPU oracle.

The reference ships no golden vectors for the attention path (its tests pin
shapes, invariants and tolerances only), so these fixtures are produced by the
oracle in ``oracle/attention_ref.py`` after that oracle is itself pinned by
``tests/test_oracle.py``.  Inputs are regenerated from seeds (torch CPU
generator; Q=0, K=1, V=2, dO=3, lengths=4) and a SHA-256 of the input bytes is
stored so a changed generator is detected rather than silently compared.

Run:  python tests/golden/make_fixtures.py
"""

from __future__ import annotations

import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import attention_ref as ref  # noqa: E402

# name: (dtype, B, S, Hq, Hkv, D, theta)
ATTN_CASES = {
    "c1_debug_fp32": (torch.float32, 2, 256, 4, 2, 64, 10000.0),
    "bf16_gqa4_d128": (torch.bfloat16, 1, 96, 8, 2, 128, 500000.0),
}
DECODE_CASE = dict(dtype=torch.bfloat16, B=4, Smax=80, Hq=8, Hkv=2, D=128, theta=500000.0,
                   lo=5, hi=70)
CAPTURE_CASE = dict(dtype=torch.float32, B=1, S=48, Hq=4, Hkv=2, D=64, theta=10000.0)


def seeded(shape, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


def attn_inputs(dtype, B, S, Hq, Hkv, D, theta):
    q = seeded((B, S, Hq, D), 0, dtype)
    k = seeded((B, S, Hkv, D), 1, dtype)
    v = seeded((B, S, Hkv, D), 2, dtype)
    do = seeded((B, S, Hq, D), 3, dtype)
    cos, sin = ref.rope_tables(D, S, theta)
    return q, k, v, do, cos, sin


def decode_inputs(dtype, B, Smax, Hq, Hkv, D, theta, lo, hi):
    g = torch.Generator().manual_seed(4)
    lens = torch.randint(lo, hi + 1, (B,), generator=g, dtype=torch.int32)
    q = seeded((B, 1, Hq, D), 0, dtype)
    kn = seeded((B, 1, Hkv, D), 1, dtype)
    vn = seeded((B, 1, Hkv, D), 2, dtype)
    kc = seeded((B, Hkv, Smax, D), 5, dtype)
    vc = seeded((B, Hkv, Smax, D), 6, dtype)
    cos, sin = ref.rope_tables(D, Smax, theta)
    return q, kn, vn, kc, vc, lens, cos, sin


def digest(*ts) -> str:
    h = hashlib.sha256()
    for t in ts:
        h.update(t.contiguous().view(torch.uint8).numpy().tobytes())
    return h.hexdigest()


def f32(t):
    return t.to(torch.float32).numpy()


def main() -> None:
    for name, cfg in ATTN_CASES.items():
        q, k, v, do, cos, sin = attn_inputs(*cfg)
        out, lse = ref.attention_fwd(q, k, v, cos, sin)
        dq, dk, dv = ref.attention_bwd(q, k, v, cos, sin, do)
        np.savez(os.path.join(HERE, f"{name}.npz"), sha256=np.array(digest(q, k, v, do)),
                 out=f32(out), lse=f32(lse), dq=f32(dq), dk=f32(dk), dv=f32(dv))
    q, kn, vn, kc, vc, lens, cos, sin = decode_inputs(**DECODE_CASE)
    out, kc2, vc2 = ref.decode_step(q, kn, vn, kc, vc, lens, cos, sin)
    b_idx = torch.arange(lens.numel())
    np.savez(os.path.join(HERE, "decode_bf16.npz"),
             sha256=np.array(digest(q, kn, vn, kc, vc, lens)), out=f32(out),
             k_written=f32(kc2[b_idx, :, lens.long()]), lens=lens.numpy())
    c = CAPTURE_CASE
    q, k, v, _, cos, sin = attn_inputs(c["dtype"], c["B"], c["S"], c["Hq"], c["Hkv"], c["D"],
                                       c["theta"])
    out, p = ref.capture(q, k, v, cos, sin)
    np.savez(os.path.join(HERE, "capture_fp32.npz"), sha256=np.array(digest(q, k, v)),
             out=f32(out), probs=f32(p))
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
