"""PyTorch operators over the C ABI (``include/kf_attn.h``).

``attention`` is a ``torch.library`` custom op with a fake (meta) kernel and an
autograd formula, so it works under ``torch.compile`` (the reference compiles
the model, ``kempnerforge/distributed/parallel.py:590-592``) and under
non-reentrant activation checkpointing (``kempnerforge/distributed/parallel.py:104``):
the forward saves q, k, v (pre-RoPE), out and lse and is deterministic, so a
recomputed forward reproduces the saved tensors bit for bit.

All ops launch on ``torch.cuda.current_stream()``, allocate outputs and
workspace through PyTorch's caching allocator, and never synchronise.  They
only accept GPU tensors: there is no CPU path.
"""

from __future__ import annotations

import ctypes
import weakref
from typing import Optional

import torch

from kempnerforge_amd import _lib

_DTYPES = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16,
           torch.float16: _lib.DTYPE_F16}


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"kempnerforge_amd attention: unsupported dtype {t.dtype}") from None


def _require_gpu(*ts: torch.Tensor) -> None:
    for t in ts:
        if t.device.type != "cuda":
            raise RuntimeError(
                "kempnerforge_amd attention runs only on a ROCm GPU (gfx950); got a tensor on "
                f"{t.device}. There is no CPU fallback."
            )


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """t itself when its data starts on a 16-byte boundary (the MFMA kernels'
    vector loads need it), else a fresh copy (the allocator aligns those)."""
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def _doc_ids(doc_ids, B: int, S: int, device) -> torch.Tensor | None:
    """Packed-sequence document ids as the contiguous int32 [B, S] the kernels read."""
    if doc_ids is None:
        return None
    if tuple(doc_ids.shape) != (B, S):
        raise ValueError(f"doc_ids must be [batch, seq_len] = [{B}, {S}] (got {tuple(doc_ids.shape)})")
    if doc_ids.device != device:
        raise RuntimeError("doc_ids must be on the same device as q")
    return doc_ids.to(torch.int32).contiguous()


def _key_valid(key_padding_mask, B: int, S: int, device) -> torch.Tensor | None:
    """``key_padding_mask [B, S]`` (True = attend) as the int32 flags the kernels read."""
    if key_padding_mask is None:
        return None
    if tuple(key_padding_mask.shape) != (B, S):
        raise ValueError(f"key_padding_mask must be [batch, seq_len] = [{B}, {S}] "
                         f"(got {tuple(key_padding_mask.shape)})")
    if key_padding_mask.device != device:
        raise RuntimeError("key_padding_mask must be on the same device as q")
    return key_padding_mask.to(torch.int32).contiguous()


def _rope_table(t: torch.Tensor, rows: int, half: int, name: str) -> torch.Tensor:
    if t.dtype != torch.float32:
        t = t.float()
    t = t.contiguous()
    if t.dim() != 2 or t.shape[0] < rows or t.shape[1] != half:
        raise ValueError(f"{name} must be [>= {rows}, {half}] (got {tuple(t.shape)})")
    return t


# --------------------------------------------------------------------------- raw calls
def fwd_raw(q, k, v, cos, sin, *, causal: bool, k_rotated: bool, k_layout: str = "bshd",
            doc_ids=None, key_padding_mask=None):
    """out, lse = attention(q, k, v) with RoPE fused (``kf_attn_fwd``).

    q ``[B,Sq,Hq,D]``; k/v ``[B,Sk,Hkv,D]`` (``k_layout="bshd"``) or
    ``[B,Hkv,Sk,D]`` views into a KV cache (``k_layout="bhsd"``, keys already
    rotated).  ``doc_ids [B,S]`` restricts each query to keys of its own
    document (packed sequences), ``key_padding_mask [B,S]`` (True = attend) to
    valid keys, a row left with no key attending every key.  Returns out
    ``[B,Sq,Hq,D]`` and lse ``[B,Hq,Sq]`` float32.
    """
    _require_gpu(q, k, v)
    lib = _lib.load()
    q = q.contiguous()
    B, Sq, Hq, D = q.shape
    if k_layout == "bshd":
        Sk, Hkv = k.shape[1], k.shape[2]
        kstr = (k.stride(0), k.stride(1), k.stride(2))
        vstr = (v.stride(0), v.stride(1), v.stride(2))
    else:
        Hkv, Sk = k.shape[1], k.shape[2]
        kstr = (k.stride(0), k.stride(2), k.stride(1))
        vstr = (v.stride(0), v.stride(2), v.stride(1))
    if k.stride(-1) != 1 or v.stride(-1) != 1 or tuple(v.shape) != tuple(k.shape):
        raise ValueError("k and v must have the same shape and a contiguous head dim")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("q, k, v must share a dtype")
    cos = _rope_table(cos, Sq, D // 2, "rope_cos")
    sin = _rope_table(sin, Sq, D // 2, "rope_sin")
    doc = _doc_ids(doc_ids, B, Sq, q.device)
    kv = _key_valid(key_padding_mask, B, Sq, q.device)
    dt = _dtype_code(q)
    out = torch.empty_like(q)
    lse = torch.empty(B, Hq, Sq, dtype=torch.float32, device=q.device)
    nbytes = _lib.size_out()
    _lib.check(lib.kf_attn_fwd_workspace_size(B, Sq, Sk, Hq, Hkv, D, dt, ctypes.byref(nbytes)),
               "kf_attn_fwd_workspace_size")
    ws = _workspace(nbytes.value, q.device)
    _lib.check(lib.kf_attn_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(cos), _ptr(sin), _ptr(out),
                               _ptr(lse), _ptr(ws), ws.numel(), B, Sq, Sk, Hq, Hkv, D, *kstr,
                               *vstr, int(k_rotated), int(causal), _ptr(doc), _ptr(kv), dt,
                               _stream(q)),
               "kf_attn_fwd")
    return out, lse


_BWD_LOW_MEMORY = False
# Largest share of the memory available to the caching allocator (free device
# memory plus what it holds unused) that the kept dS tiles may take.
_DS_BUDGET_FRACTION: float | None = 0.5


def set_backward_low_memory(enabled: bool) -> None:
    """Default of ``bwd_raw``'s ``low_memory`` (and so of the autograd backward of
    :func:`attention` and the ``Attention`` module): True never keeps the dS
    tiles (about B*Hq*S*S bytes), trading ~5-11% of backward time for memory."""
    global _BWD_LOW_MEMORY
    _BWD_LOW_MEMORY = bool(enabled)
    _DS_DECISIONS.clear()


def set_backward_ds_budget(fraction: float | None) -> None:
    """Share (0..1] of the memory the allocator can still hand out that the
    backward's kept dS tiles may take (default 0.5); above it the backward
    falls back to recomputing S and dP for dQ.  None keeps them whenever the
    library offers them, whatever the free memory (a policy that does not
    depend on the allocator's state at all).  The decision is made once per
    backward shape and then reused, so that dQ's last bits do not change from
    step to step; setting the budget starts over."""
    global _DS_BUDGET_FRACTION
    if fraction is not None and not 0.0 < fraction <= 1.0:
        raise ValueError(f"fraction must lie in (0, 1] or be None (got {fraction})")
    _DS_BUDGET_FRACTION = None if fraction is None else float(fraction)
    _DS_DECISIONS.clear()


def available_bytes(device) -> int | None:
    """Bytes the caching allocator can hand out without growing past the
    device: free device memory plus memory it reserves but does not use
    (None if the runtime cannot say, e.g. inside some stream captures)."""
    try:
        free, _ = torch.cuda.mem_get_info(device)
    except RuntimeError:
        return None
    idle = torch.cuda.memory_reserved(device) - torch.cuda.memory_allocated(device)
    return int(free) + max(int(idle), 0)


# The keep-dS decision per backward shape, made once (the first backward of
# that shape) and reused: the kept-tile and recompute dQ paths differ in the
# last bits, so deciding again from the allocator's state at every call could
# switch paths from one step to the next.  Cleared by set_backward_ds_budget
# and set_backward_low_memory.
_DS_DECISIONS: dict[tuple, bool] = {}


def _keep_ds_for(key: tuple, extra_bytes: int, device) -> bool:
    hit = _DS_DECISIONS.get(key)
    if hit is None:
        if _DS_BUDGET_FRACTION is None:
            hit = extra_bytes > 0
        else:
            hit = keep_ds_tiles(extra_bytes, available_bytes(device))
        _DS_DECISIONS[key] = hit
    return hit


def keep_ds_tiles(extra_bytes: int, available: int | None, fraction: float | None = None) -> bool:
    """Whether the backward keeps its dS tiles: their ``extra_bytes`` must fit in
    ``fraction`` of the ``available`` bytes (the memory-aware default; the
    reference's SDPA backward needs O(S) memory, so an unconditional O(S^2)
    store could run a model that fits with the reference out of memory).
    Unknown availability keeps them if the library offers them."""
    fraction = _DS_BUDGET_FRACTION if fraction is None else fraction
    if extra_bytes <= 0:
        return False
    if fraction is None:
        return True
    return available is None or extra_bytes <= fraction * available


def bwd_raw(q, k, v, cos, sin, out, lse, dout, *, causal: bool, doc_ids=None,
            key_padding_mask=None, low_memory: bool | None = None):
    """dq, dk, dv for :func:`fwd_raw` with un-rotated BSHD k (``kf_attn_bwd``).

    By default the workspace is sized so that the dK/dV pass keeps its bf16 dS
    tiles for dQ (``kf_attn_bwd_workspace_size_ds``: about B*Hq*S*S bytes
    for causal attention, 2.2 GB at B=4, S=4096, Hq=32) when those fit in the
    budget of :func:`set_backward_ds_budget` (half the memory the allocator can
    still hand out); otherwise, or with ``low_memory=True``, it passes the
    minimal workspace and dQ recomputes S and dP (None: the default set by
    :func:`set_backward_low_memory`, initially False).  dK and dV are the same
    bits either way.
    """
    _require_gpu(q, k, v, out, lse, dout)
    lib = _lib.load()
    q, k, v, out, dout = (t.contiguous() for t in (q, k, v, out, dout))
    lse = lse.contiguous()
    B, S, Hq, D = q.shape
    Hkv = k.shape[2]
    cos = _rope_table(cos, S, D // 2, "rope_cos")
    sin = _rope_table(sin, S, D // 2, "rope_sin")
    doc = _doc_ids(doc_ids, B, S, q.device)
    kv = _key_valid(key_padding_mask, B, S, q.device)
    dt = _dtype_code(q)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    nbytes = _lib.size_out()
    _lib.check(lib.kf_attn_bwd_workspace_size(B, S, Hq, Hkv, D, dt, ctypes.byref(nbytes)),
               "kf_attn_bwd_workspace_size")
    low_memory = _BWD_LOW_MEMORY if low_memory is None else low_memory
    # key padding keeps dS only causally, and only for the batch rows whose key
    # 0 is valid (decided on the device; the others recompute)
    if not low_memory and (kv is None or causal):
        with_ds = _lib.size_out()
        _lib.check(lib.kf_attn_bwd_workspace_size_ds(B, S, Hq, Hkv, D, dt, int(causal),
                                                     ctypes.byref(with_ds)),
                   "kf_attn_bwd_workspace_size_ds")
        key = ("bwd", q.device, B, S, Hq, Hkv, D, q.dtype, bool(causal), doc is not None,
               kv is not None)
        if _keep_ds_for(key, with_ds.value - nbytes.value, q.device):
            nbytes = with_ds
    ws = _workspace(nbytes.value, q.device)
    _lib.check(lib.kf_attn_bwd(_ptr(q), _ptr(k), _ptr(v), _ptr(cos), _ptr(sin), _ptr(out),
                               _ptr(lse), _ptr(dout), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(ws),
                               ws.numel(), B, S, Hq, Hkv, D, int(causal), _ptr(doc), _ptr(kv),
                               dt, _stream(q)),
               "kf_attn_bwd")
    return dq, dk, dv


_KF_ERR_UNSUPPORTED = 2


def rot_size(B: int, S: int, Hq: int, Hkv: int, D: int, dtype: torch.dtype, has_doc: bool,
             has_key_padding: bool) -> int:
    """Bytes of the rotated-operand buffer of :func:`fwd_rot_raw`, or 0 when that
    path does not take these sizes, dtype or mask kinds (``kf_attn_rot_size``)."""
    lib = _lib.load()
    if dtype not in _DTYPES or not hasattr(lib, "kf_attn_rot_size"):  # (a KF_ATTN_LIB build
        return 0                                                        # predating the pair)
    n = _lib.size_out()
    rc = lib.kf_attn_rot_size(B, S, Hq, Hkv, D, _DTYPES[dtype], int(has_doc),
                                      int(has_key_padding), ctypes.byref(n))
    if rc == _KF_ERR_UNSUPPORTED:
        return 0
    _lib.check(rc, "kf_attn_rot_size")
    return n.value


def _rot_shapes_ok(q, k, v) -> bool:
    """Self-attention shapes and one dtype: what the rotated-operand pair takes
    before kf_attn_rot_size's own size / dtype / mask checks."""
    if q.dim() != 4 or k.dim() != 4:
        return False
    B, S, Hq, D = q.shape
    return (k.shape[0] == B and k.shape[1] == S and k.shape[3] == D
            and tuple(v.shape) == tuple(k.shape) and k.dtype == q.dtype and v.dtype == q.dtype)


def fwd_rot_raw(q, k, v, cos, sin, *, causal: bool, doc_ids=None, key_padding_mask=None):
    """out, lse, rot for self-attention (``kf_attn_fwd_rot``): :func:`fwd_raw` with
    un-rotated BSHD k that also returns ``rot``, q and k after RoPE as the
    backward reads them, so that :func:`bwd_rot_raw` needs neither q nor k.
    None when that path does not apply (dtype, head_dim, alignment): then use
    :func:`fwd_raw` and :func:`bwd_raw`."""
    _require_gpu(q, k, v)
    lib = _lib.load()
    if not _rot_shapes_ok(q, k, v):
        return None
    # misaligned views are copied, so that whenever rot_size() is non-zero the
    # call below takes the rotated-operand path (the fake kernel relies on it)
    q, k, v = (_aligned(t.contiguous()) for t in (q, k, v))
    B, S, Hq, D = q.shape
    Hkv = k.shape[2]
    cos = _aligned(_rope_table(cos, S, D // 2, "rope_cos"))
    sin = _aligned(_rope_table(sin, S, D // 2, "rope_sin"))
    doc = _doc_ids(doc_ids, B, S, q.device)
    kv = _key_valid(key_padding_mask, B, S, q.device)
    nrot = rot_size(B, S, Hq, Hkv, D, q.dtype, doc is not None, kv is not None)
    if nrot == 0:
        return None
    dt = _dtype_code(q)
    out = torch.empty_like(q)
    lse = torch.empty(B, Hq, S, dtype=torch.float32, device=q.device)
    rot = torch.empty(nrot // q.element_size(), dtype=q.dtype, device=q.device)
    nbytes = _lib.size_out()
    _lib.check(lib.kf_attn_fwd_workspace_size(B, S, S, Hq, Hkv, D, dt, ctypes.byref(nbytes)),
               "kf_attn_fwd_workspace_size")
    ws = _workspace(nbytes.value, q.device)
    rc = lib.kf_attn_fwd_rot(_ptr(q), _ptr(k), _ptr(v), _ptr(cos), _ptr(sin), _ptr(out),
                             _ptr(lse), _ptr(rot), _ptr(ws), ws.numel(), B, S, Hq, Hkv, D,
                             int(causal), _ptr(doc), _ptr(kv), dt, _stream(q))
    if rc == _KF_ERR_UNSUPPORTED:
        return None
    _lib.check(rc, "kf_attn_fwd_rot")
    return out, lse, rot


def bwd_rot_raw(rot, v, cos, sin, out, lse, dout, *, causal: bool, doc_ids=None,
                key_padding_mask=None, low_memory: bool | None = None):
    """dq, dk, dv for :func:`fwd_rot_raw` from its ``rot`` (``kf_attn_bwd_rot``);
    workspace policy as in :func:`bwd_raw`.  The results equal :func:`bwd_raw`'s
    bit for bit."""
    _require_gpu(rot, v, out, lse, dout)
    lib = _lib.load()
    v, out, dout, lse = (t.contiguous() for t in (v, out, dout, lse))
    dout = _aligned(dout)
    B, S, Hq, D = out.shape
    Hkv = v.shape[2]
    cos = _rope_table(cos, S, D // 2, "rope_cos")
    sin = _rope_table(sin, S, D // 2, "rope_sin")
    doc = _doc_ids(doc_ids, B, S, out.device)
    kv = _key_valid(key_padding_mask, B, S, out.device)
    # the C ABI takes rot without a length: check it here, before any launch,
    # so a rot from another shape or mask kind cannot send the kernels out of bounds
    want = rot_size(B, S, Hq, Hkv, D, out.dtype, doc is not None, kv is not None)
    if (rot.dtype != out.dtype or not rot.is_contiguous() or rot.device != out.device
            or rot.data_ptr() % 16 or want == 0 or rot.numel() * rot.element_size() != want):
        raise ValueError(
            f"rot must be the contiguous, 16-byte aligned {out.dtype} buffer fwd_rot_raw "
            f"returns for these shapes and masks ({want} bytes on {out.device}); got "
            f"{rot.numel() * rot.element_size()} bytes of {rot.dtype} on {rot.device}")
    dt = _dtype_code(out)
    dq, dk, dv = torch.empty_like(out), torch.empty_like(v), torch.empty_like(v)
    nbytes = _lib.size_out()
    _lib.check(lib.kf_attn_bwd_rot_workspace_size(B, S, Hq, Hkv, D, dt, int(causal), 0,
                                                  ctypes.byref(nbytes)),
               "kf_attn_bwd_rot_workspace_size")
    low_memory = _BWD_LOW_MEMORY if low_memory is None else low_memory
    if not low_memory and (kv is None or causal):  # as in bwd_raw
        with_ds = _lib.size_out()
        _lib.check(lib.kf_attn_bwd_rot_workspace_size(B, S, Hq, Hkv, D, dt, int(causal), 1,
                                                      ctypes.byref(with_ds)),
                   "kf_attn_bwd_rot_workspace_size")
        key = ("bwd_rot", out.device, B, S, Hq, Hkv, D, out.dtype, bool(causal), doc is not None,
               kv is not None)
        if _keep_ds_for(key, with_ds.value - nbytes.value, out.device):
            nbytes = with_ds
    ws = _workspace(nbytes.value, out.device)
    _lib.check(lib.kf_attn_bwd_rot(_ptr(rot), _ptr(v), _ptr(cos), _ptr(sin), _ptr(out),
                                   _ptr(lse), _ptr(dout), _ptr(dq), _ptr(dk), _ptr(dv),
                                   _ptr(ws), ws.numel(), B, S, Hq, Hkv, D, int(causal),
                                   _ptr(doc), _ptr(kv), dt, _stream(out)),
               "kf_attn_bwd_rot")
    return dq, dk, dv


def decode_raw(q_new, k_new, v_new, k_cache, v_cache, lens, cos, sin, *, rope_row_offset: int,
               max_len: int, q_norm_weight=None, k_norm_weight=None, norm_eps: float = 1e-5):
    """One decode step (``kf_attn_decode``); writes the rotated new k and v into
    the caches at ``lens[b]`` and returns out ``[B,1,Hq,D]``.  With the QK-norm
    weights (``[D]``, any float dtype) q_new and k_new are RMS-normalised in the
    kernels first, as ``Attention.q_norm`` / ``k_norm`` would."""
    _require_gpu(q_new, k_new, v_new, k_cache, v_cache, lens)
    lib = _lib.load()
    q_new, k_new, v_new = (t.contiguous() for t in (q_new, k_new, v_new))
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("KV caches must be contiguous [B, n_kv_heads, max_seq_len, head_dim]")
    if lens.dtype != torch.int32 or not lens.is_contiguous():
        raise TypeError("lens must be a contiguous int32 tensor")
    B, _, Hq, D = q_new.shape
    Hkv, Smax = k_cache.shape[1], k_cache.shape[2]
    cos = _rope_table(cos, 1, D // 2, "rope_cos")
    sin = _rope_table(sin, 1, D // 2, "rope_sin")
    if (q_norm_weight is None) != (k_norm_weight is None):
        raise ValueError("QK-norm needs both q_norm_weight and k_norm_weight")
    qnw = knw = None
    if q_norm_weight is not None:
        qnw, knw = (_norm_weight(w, D, q_new.device) for w in (q_norm_weight, k_norm_weight))
    dt = _dtype_code(q_new)
    out = torch.empty_like(q_new)
    nbytes = _lib.size_out()
    _lib.check(lib.kf_attn_decode_workspace_size(B, Hq, Hkv, D, max_len, dt, ctypes.byref(nbytes)),
               "kf_attn_decode_workspace_size")
    ws = _workspace(nbytes.value, q_new.device)
    _lib.check(lib.kf_attn_decode(_ptr(q_new), _ptr(k_new), _ptr(v_new), _ptr(k_cache),
                                  _ptr(v_cache), _ptr(lens), _ptr(cos), _ptr(sin),
                                  int(rope_row_offset), cos.shape[0], _ptr(out), _ptr(ws),
                                  ws.numel(), B, Smax, Hq, Hkv, D, int(max_len), _ptr(qnw),
                                  _ptr(knw), float(norm_eps), dt, _stream(q_new)),
               "kf_attn_decode")
    return out


_NORM_CACHE: dict[int, tuple] = {}  # id(weight) -> (weakref, version, float32 copy)


def _norm_weight(w: torch.Tensor, D: int, device) -> torch.Tensor:
    """RMSNorm weight as the float32 [D] vector the kernels read (exact for any
    float storage dtype), cached per parameter version so that a decode step
    does not launch the conversion again."""
    if w.shape != (D,):
        raise ValueError(f"QK-norm weight must be [{D}] (got {tuple(w.shape)})")
    if w.device != device:
        raise RuntimeError("QK-norm weight must be on the same device as q")
    if w.dtype == torch.float32 and w.is_contiguous():
        return w
    hit = _NORM_CACHE.get(id(w))
    if hit is not None and hit[0]() is w and hit[1] == w._version:
        return hit[2]
    f = w.detach().to(torch.float32).contiguous()
    if len(_NORM_CACHE) > 1024:  # drop entries of freed weights
        for k in [k for k, e in _NORM_CACHE.items() if e[0]() is None]:
            del _NORM_CACHE[k]
    _NORM_CACHE[id(w)] = (weakref.ref(w), w._version, f)
    return f


def cache_append_raw(k_new, v_new, cos, sin, k_cache, v_cache, start: int) -> None:
    """Rotate ``k_new [B,S,Hkv,D]`` and write it and ``v_new`` into the caches at
    positions ``start..start+S-1`` (``kf_kv_cache_append``)."""
    _require_gpu(k_new, v_new, k_cache, v_cache)
    lib = _lib.load()
    k_new, v_new = k_new.contiguous(), v_new.contiguous()
    B, Snew, Hkv, D = k_new.shape
    Smax = k_cache.shape[2]
    cos = _rope_table(cos, Snew, D // 2, "rope_cos")
    sin = _rope_table(sin, Snew, D // 2, "rope_sin")
    _lib.check(lib.kf_kv_cache_append(_ptr(k_new), _ptr(v_new), _ptr(cos), _ptr(sin),
                                      _ptr(k_cache), _ptr(v_cache), int(start), B, Snew, Hkv,
                                      Smax, D, _dtype_code(k_new), _stream(k_new)),
               "kf_kv_cache_append")


def capture_raw(q, k, v, cos, sin, *, causal: bool, k_rotated: bool, k_layout: str = "bshd",
                doc_ids=None, key_padding_mask=None):
    """out, probs, lse with probs the float32 softmax matrix ``[B,Hq,Sq,Sk]``
    (``kf_attn_capture``)."""
    _require_gpu(q, k, v)
    lib = _lib.load()
    q = q.contiguous()
    B, Sq, Hq, D = q.shape
    if k_layout == "bshd":
        Sk, Hkv = k.shape[1], k.shape[2]
        kstr = (k.stride(0), k.stride(1), k.stride(2))
        vstr = (v.stride(0), v.stride(1), v.stride(2))
    else:
        Hkv, Sk = k.shape[1], k.shape[2]
        kstr = (k.stride(0), k.stride(2), k.stride(1))
        vstr = (v.stride(0), v.stride(2), v.stride(1))
    if k.stride(-1) != 1 or v.stride(-1) != 1:
        raise ValueError("k and v need a contiguous head dim")
    cos = _rope_table(cos, Sq, D // 2, "rope_cos")
    sin = _rope_table(sin, Sq, D // 2, "rope_sin")
    doc = _doc_ids(doc_ids, B, Sq, q.device)
    kv = _key_valid(key_padding_mask, B, Sq, q.device)
    dt = _dtype_code(q)
    out = torch.empty_like(q)
    lse = torch.empty(B, Hq, Sq, dtype=torch.float32, device=q.device)
    probs = torch.empty(B, Hq, Sq, Sk, dtype=torch.float32, device=q.device)
    nbytes = _lib.size_out()
    _lib.check(lib.kf_attn_capture_workspace_size(B, Sq, Sk, Hq, Hkv, D, dt, ctypes.byref(nbytes)),
               "kf_attn_capture_workspace_size")
    ws = _workspace(nbytes.value, q.device)
    _lib.check(lib.kf_attn_capture(_ptr(q), _ptr(k), _ptr(v), _ptr(cos), _ptr(sin), _ptr(probs),
                                   _ptr(out), _ptr(lse), _ptr(ws), ws.numel(), B, Sq, Sk, Hq, Hkv,
                                   D, *kstr, *vstr, int(k_rotated), int(causal), _ptr(doc),
                                   _ptr(kv), dt, _stream(q)),
               "kf_attn_capture")
    return out, probs, lse


# --------------------------------------------------------------------------- custom ops
@torch.library.custom_op("kf::attn_fwd", mutates_args=(), device_types="cuda")
def attn_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor,
             sin: torch.Tensor, causal: bool, doc_ids: Optional[torch.Tensor] = None,
             key_padding_mask: Optional[torch.Tensor] = None, keep_rot: bool = True
             ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """out, lse and rot: the rotated q and k for the backward, written only
    when ``keep_rot`` (a backward will run) and the rotated-operand path takes
    these inputs; empty otherwise."""
    if keep_rot:
        res = fwd_rot_raw(q, k, v, cos, sin, causal=causal, doc_ids=doc_ids,
                          key_padding_mask=key_padding_mask)
        if res is not None:
            return res
    out, lse = fwd_raw(q, k, v, cos, sin, causal=causal, k_rotated=False, doc_ids=doc_ids,
                       key_padding_mask=key_padding_mask)
    return out, lse, q.new_empty(0)


@attn_fwd.register_fake
def _(q, k, v, cos, sin, causal, doc_ids=None, key_padding_mask=None, keep_rot=True):
    # the same decision as the real kernel: rot exactly when keep_rot, the
    # shapes and dtypes fit and kf_attn_rot_size accepts the sizes (the real
    # op copies misaligned inputs, so alignment never changes it)
    B, S, Hq, D = q.shape
    nrot = rot_size(B, S, Hq, k.shape[2], D, q.dtype, doc_ids is not None,
                    key_padding_mask is not None) if keep_rot and _rot_shapes_ok(q, k, v) else 0
    return (torch.empty_like(q), q.new_empty(B, Hq, S, dtype=torch.float32),
            q.new_empty(nrot // q.element_size()))


@torch.library.custom_op("kf::attn_bwd", mutates_args=(), device_types="cuda")
def attn_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor,
             sin: torch.Tensor, out: torch.Tensor, lse: torch.Tensor, dout: torch.Tensor,
             causal: bool, doc_ids: Optional[torch.Tensor] = None,
             key_padding_mask: Optional[torch.Tensor] = None
             ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return bwd_raw(q, k, v, cos, sin, out, lse, dout, causal=causal, doc_ids=doc_ids,
                   key_padding_mask=key_padding_mask)


@attn_bwd.register_fake
def _(q, k, v, cos, sin, out, lse, dout, causal, doc_ids=None, key_padding_mask=None):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


@torch.library.custom_op("kf::attn_bwd_rot", mutates_args=(), device_types="cuda")
def attn_bwd_rot(rot: torch.Tensor, v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                 out: torch.Tensor, lse: torch.Tensor, dout: torch.Tensor, causal: bool,
                 doc_ids: Optional[torch.Tensor] = None,
                 key_padding_mask: Optional[torch.Tensor] = None
                 ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return bwd_rot_raw(rot, v, cos, sin, out, lse, dout, causal=causal, doc_ids=doc_ids,
                       key_padding_mask=key_padding_mask)


@attn_bwd_rot.register_fake
def _(rot, v, cos, sin, out, lse, dout, causal, doc_ids=None, key_padding_mask=None):
    return torch.empty_like(out), torch.empty_like(v), torch.empty_like(v)


def _setup_context(ctx, inputs, output):
    q, k, v, cos, sin, causal, doc_ids, key_padding_mask, _keep_rot = inputs
    out, lse, rot = output
    # only out carries a gradient: no zero-filled gradients for lse and rot
    ctx.mark_non_differentiable(lse, rot)
    ctx.set_materialize_grads(False)
    # with rot the backward needs neither q nor k: keep rot in their place
    ctx.use_rot = rot.numel() > 0
    if ctx.use_rot:
        ctx.save_for_backward(rot, v, cos, sin, out, lse, doc_ids, key_padding_mask)
    else:
        ctx.save_for_backward(q, k, v, cos, sin, out, lse, doc_ids, key_padding_mask)
    ctx.causal = causal


def _backward(ctx, dout, dlse, drot):
    if ctx.use_rot:
        rot, v, cos, sin, out, lse, doc_ids, key_padding_mask = ctx.saved_tensors
        dq, dk, dv = attn_bwd_rot(rot, v, cos, sin, out, lse, dout.contiguous(), ctx.causal,
                                  doc_ids, key_padding_mask)
    else:
        q, k, v, cos, sin, out, lse, doc_ids, key_padding_mask = ctx.saved_tensors
        dq, dk, dv = attn_bwd(q, k, v, cos, sin, out, lse, dout.contiguous(), ctx.causal,
                              doc_ids, key_padding_mask)
    return dq, dk, dv, None, None, None, None, None, None


attn_fwd.register_autograd(_backward, setup_context=_setup_context)


def attention(q, k, v, rope_cos, rope_sin, *, causal: bool = True, doc_ids=None,
              key_padding_mask=None) -> torch.Tensor:
    """Differentiable RoPE + GQA + (causal) attention on BSHD tensors.

    Equivalent to the reference's ``apply_rope`` on q and k
    (``kempnerforge/model/attention.py:165-166``), ``repeat_interleave``
    (``:173-175``) and ``F.scaled_dot_product_attention(..., is_causal=causal)``
    (``:231``), returning BSHD instead of BHSD.  With ``doc_ids [B,S]`` it is the
    reference's packed-sequence branch instead (``:204-227``): causal and
    same-document, without materialising the ``[B,1,S,S]`` mask; with
    ``key_padding_mask [B,S]`` (True = attend) its padded-key branch
    (``:214-225``, ``kempnerforge/model/mot.py:188-198``), NaN guard included.
    """
    # rot only when a backward can run: under no_grad / inference it would be
    # written (q and k rotated, (B*Hkv + B*Hq)*S*D elements) and never read
    keep_rot = torch.is_grad_enabled() and (q.requires_grad or k.requires_grad
                                            or v.requires_grad)
    out, _, _ = attn_fwd(q, k, v, rope_cos, rope_sin, causal, doc_ids, key_padding_mask,
                         keep_rot)
    return out
