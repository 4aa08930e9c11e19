"""ctypes binding of ``libkf_attn.so`` (the C ABI declared in ``include/kf_attn.h``).

The library is built in-tree by ``__graft_entry__.build()`` (``make`` in
``kempnerforge_amd/csrc``) into ``kempnerforge_amd/lib/libkf_attn.so``.  There is
no fallback: if the library is missing, every attention call raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

# In-tree build; KF_ATTN_LIB may name another build of the same library (an
# A/B comparison of two builds of the kernels on one device).
LIB_PATH = os.environ.get("KF_ATTN_LIB") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), "lib", "libkf_attn.so")

DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2

# Exported symbols and their signatures (must match include/kf_attn.h).
_c_int, _c_i64, _c_sz, _vp, _fp = (ctypes.c_int, ctypes.c_int64, ctypes.c_size_t,
                                    ctypes.c_void_p, ctypes.c_void_p)
_szp = ctypes.POINTER(ctypes.c_size_t)
SIGNATURES = {
    "kf_version": ([], _c_int),
    "kf_last_error": ([], ctypes.c_char_p),
    "kf_attn_fwd_workspace_size": ([_c_int] * 7 + [_szp], _c_int),
    "kf_attn_fwd": ([_vp, _vp, _vp, _fp, _fp, _vp, _fp, _vp, _c_sz] + [_c_int] * 6
                    + [_c_i64] * 6 + [_c_int] * 2 + [_vp, _vp, _c_int, _vp], _c_int),
    "kf_attn_bwd_workspace_size": ([_c_int] * 6 + [_szp], _c_int),
    "kf_attn_bwd_workspace_size_ds": ([_c_int] * 7 + [_szp], _c_int),
    "kf_attn_bwd": ([_vp, _vp, _vp, _fp, _fp, _vp, _fp, _vp, _vp, _vp, _vp, _vp, _c_sz]
                    + [_c_int] * 6 + [_vp, _vp, _c_int, _vp], _c_int),
    "kf_attn_rot_size": ([_c_int] * 8 + [_szp], _c_int),
    "kf_attn_fwd_rot": ([_vp, _vp, _vp, _fp, _fp, _vp, _fp, _vp, _vp, _c_sz] + [_c_int] * 6
                        + [_vp, _vp, _c_int, _vp], _c_int),
    "kf_attn_bwd_rot_workspace_size": ([_c_int] * 8 + [_szp], _c_int),
    "kf_attn_bwd_rot": ([_vp, _vp, _fp, _fp, _vp, _fp, _vp, _vp, _vp, _vp, _vp, _c_sz]
                        + [_c_int] * 6 + [_vp, _vp, _c_int, _vp], _c_int),
    "kf_attn_decode_workspace_size": ([_c_int] * 6 + [_szp], _c_int),
    "kf_attn_decode": ([_vp, _vp, _vp, _vp, _vp, _vp, _fp, _fp, _c_i64, _c_i64, _vp, _vp, _c_sz]
                       + [_c_int] * 6 + [_fp, _fp, ctypes.c_float, _c_int, _vp], _c_int),
    "kf_attn_decode_noalloc": ([_vp, _vp, _vp, _vp, _vp, _vp, _fp, _fp, _c_i64, _c_i64, _vp]
                               + [_c_int] * 6 + [_fp, _fp, ctypes.c_float, _c_int, _vp], _c_int),
    "kf_kv_cache_append": ([_vp, _vp, _fp, _fp, _vp, _vp] + [_c_int] * 7 + [_vp], _c_int),
    "kf_attn_capture_workspace_size": ([_c_int] * 7 + [_szp], _c_int),
    "kf_attn_capture": ([_vp, _vp, _vp, _fp, _fp, _fp, _vp, _fp, _vp, _c_sz] + [_c_int] * 6
                        + [_c_i64] * 6 + [_c_int] * 2 + [_vp, _vp, _c_int, _vp], _c_int),
    "kf_prof_enable": ([_c_int], _c_int),
    "kf_prof_collect": ([ctypes.c_char_p, ctypes.POINTER(ctypes.c_float),
                         ctypes.POINTER(ctypes.c_int), _c_int], _c_int),
}

_lock = threading.Lock()
_lib = None


class KernelError(RuntimeError):
    """A C-ABI entry point returned an error code."""


def load() -> ctypes.CDLL:
    """Load the library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"kempnerforge_amd: native library not found at {LIB_PATH}; "
                    "build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                    "(there is no CPU or PyTorch fallback for the attention path)"
                )
            lib = ctypes.CDLL(LIB_PATH)
            for name, (argtypes, restype) in SIGNATURES.items():
                if os.environ.get("KF_ATTN_LIB") and not hasattr(lib, name):
                    continue  # another build may predate an entry point
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = restype
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().kf_last_error().decode(errors="replace")
        raise KernelError(f"{what} failed (code {rc}): {msg}")


def size_out() -> ctypes.c_size_t:
    return ctypes.c_size_t(0)


class KernelTimer:
    """Per-kernel HIP-event timing of the library's launches.

    ``with KernelTimer() as t: ...`` enables the library's event bracketing;
    on exit ``t.stats`` maps kernel name -> (total_ms, launches).
    """

    CAP = 64

    def __enter__(self):
        lib = load()
        lib.kf_prof_collect(None, None, None, 0)  # drop anything recorded before
        lib.kf_prof_enable(1)
        self.stats = {}
        return self

    def __exit__(self, *exc):
        lib = load()
        lib.kf_prof_enable(0)
        names = ctypes.create_string_buffer(64 * self.CAP)
        tot = (ctypes.c_float * self.CAP)()
        cnt = (ctypes.c_int * self.CAP)()
        n = lib.kf_prof_collect(names, tot, cnt, self.CAP)
        for i in range(min(n, self.CAP)):
            name = names.raw[64 * i: 64 * (i + 1)].split(b"\0", 1)[0].decode()
            self.stats[name] = (float(tot[i]), int(cnt[i]))
        return False
