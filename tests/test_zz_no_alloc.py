"""kf_attn_decode_noalloc (the allocation-free decode, partials in the
library's static device array) against kf_attn_decode with a workspace: the
same kernels, so outputs and cache writes must be equal bit for bit; two calls
in a row, the second on a smaller batch with shorter caches (the array keeps
the first call's contents)."""

from __future__ import annotations

import ctypes

import pytest
import torch

from gpu_util import DEV, announce, seeded
from kempnerforge_amd import _lib, ops
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu


def _noalloc(q, kn, vn, kc, vc, lens, cos, sin, max_len):
    lib = _lib.load()
    B, _, Hq, D = q.shape
    Hkv, Smax = kc.shape[1], kc.shape[2]
    out = torch.empty_like(q)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(lib.kf_attn_decode_noalloc(p(q), p(kn), p(vn), p(kc), p(vc), p(lens), p(cos),
                                          p(sin), 0, cos.shape[0], p(out), B, Smax, Hq, Hkv, D,
                                          max_len, None, None, ctypes.c_float(1e-5),
                                          _lib.DTYPE_BF16, stream),
               "kf_attn_decode_noalloc")
    return out


@pytest.mark.parametrize("first,second", [
    ((16, 32, 8, 128, 3000, 6000), (3, 32, 8, 128, 100, 700)),
    ((8, 16, 2, 64, 1, 2500), (2, 16, 2, 64, 1, 40)),
])
def test_noalloc_equals_workspace_decode(first, second):
    for call, (B, Hq, Hkv, D, lo, hi) in enumerate((first, second)):
        announce(f"decode no-alloc call {call}: B={B} Hq={Hq} Hkv={Hkv} D={D} L~[{lo},{hi}]")
        g = torch.Generator().manual_seed(40 + call)
        lens = torch.randint(lo, hi + 1, (B,), generator=g, dtype=torch.int32)
        Smax = hi + 8
        q = seeded((B, 1, Hq, D), 50 + call, torch.bfloat16).to(DEV)
        kn = seeded((B, 1, Hkv, D), 60 + call, torch.bfloat16).to(DEV)
        vn = seeded((B, 1, Hkv, D), 70 + call, torch.bfloat16).to(DEV)
        kc = seeded((B, Hkv, Smax, D), 80 + call, torch.bfloat16).to(DEV)
        vc = seeded((B, Hkv, Smax, D), 90 + call, torch.bfloat16).to(DEV)
        cos, sin = (t.to(DEV) for t in ref.rope_tables(D, Smax, 5e5))
        ld = lens.to(DEV)
        kc1, vc1 = kc.clone(), vc.clone()
        want = ops.decode_raw(q, kn, vn, kc1, vc1, ld, cos, sin, rope_row_offset=0,
                              max_len=Smax)
        got = _noalloc(q, kn, vn, kc, vc, ld, cos, sin, Smax)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
        assert torch.equal(kc, kc1) and torch.equal(vc, vc1)
