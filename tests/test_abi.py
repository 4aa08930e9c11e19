"""CPU checks of the boundary: the C-ABI library loads and exports every entry
point include/kf_attn.h declares, and the drop-in module keeps the reference's
contract (kempnerforge/model/attention.py:29-114) without touching a GPU."""

from __future__ import annotations

import ctypes
import inspect
import os
import re

import pytest
import torch

import kempnerforge_amd
from kempnerforge_amd import _lib
from kempnerforge_amd.attention import Attention, KVCache

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kf_attn.h")


def _declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:int|const char\*)\s+(kf_\w+)\(", text, re.M)))


def test_header_declares_the_entry_points():
    assert set(_declared_symbols()) >= {
        "kf_version", "kf_last_error", "kf_attn_fwd", "kf_attn_bwd", "kf_attn_decode",
        "kf_kv_cache_append", "kf_attn_capture", "kf_attn_fwd_workspace_size",
        "kf_attn_bwd_workspace_size", "kf_attn_decode_workspace_size",
        "kf_attn_capture_workspace_size", "kf_attn_rot_size", "kf_attn_fwd_rot",
        "kf_attn_bwd_rot_workspace_size", "kf_attn_bwd_rot",
    }


def test_library_exports_every_declared_symbol():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared_symbols():
        assert hasattr(lib, name), name
    assert set(_lib.SIGNATURES) == set(_declared_symbols())


def test_host_only_calls():
    """Entry points that never touch the device: version, workspace sizing and
    argument validation (which rejects before any launch)."""
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    lib = _lib.load()
    assert lib.kf_version() >= 100
    n = _lib.size_out()
    assert lib.kf_attn_fwd_workspace_size(4, 4096, 4096, 32, 8, 128, 1, ctypes.byref(n)) == 0
    # rotated K and V (bf16), then one int2 document range per batch row and 64-key tile,
    # then int32 counts and order of up to one query block per position
    assert n.value == 2 * 4 * 8 * 4096 * 128 * 2 + 4 * 64 * 8 + 2 * 4 * 4096 * 4
    assert lib.kf_attn_fwd_workspace_size(1, 8, 8, 6, 4, 64, 1, ctypes.byref(n)) == 1
    assert b"multiple" in lib.kf_last_error()
    assert lib.kf_attn_fwd_workspace_size(1, 8, 8, 4, 4, 63, 1, ctypes.byref(n)) == 1
    assert lib.kf_attn_decode_workspace_size(32, 32, 8, 128, 8193, 1, ctypes.byref(n)) == 0
    # (o[D], m, l) per query head of a KV group for each partial slot: one per
    # wavefront of the stream kernel (at most 2048) plus one per (sequence, KV head)
    assert n.value == (2048 + 32 * 8) * 4 * (128 + 2) * 4
    # backward: rotated K (per KV head) and Q (per query head) bf16 [P][D], then
    # lse and Delta float32 [P] per query head, then the int2 tile records and
    # the int32 counts and order of the dK/dV items (V and dO are read in place)
    B, S, Hq, Hkv, D, P = 4, 4096, 32, 8, 128, 4096
    base = (B * Hkv + B * Hq) * P * D * 2 + 2 * B * Hq * P * 4 + B * (P // 64) * 8 \
        + 2 * B * (P // 128) * 4  # + the dK/dV items' counts and order (packed documents)
    assert lib.kf_attn_bwd_workspace_size(B, S, Hq, Hkv, D, 1, ctypes.byref(n)) == 0
    assert n.value == base
    # kept dS tiles: bf16 over the causal 64-row x 32-key blocks, P * (P + 64) bytes per
    # query head, after the base rounded up to 256 bytes; full attention: 2 * P * P
    assert lib.kf_attn_bwd_workspace_size_ds(B, S, Hq, Hkv, D, 1, 1, ctypes.byref(n)) == 0
    assert n.value == (base + 255) // 256 * 256 + B * Hq * P * (P + 64)
    assert lib.kf_attn_bwd_workspace_size_ds(B, 4000, Hq, Hkv, D, 1, 0, ctypes.byref(n)) == 0
    assert n.value == (base + 255) // 256 * 256 + B * Hq * 2 * P * P  # P = 4096 for S = 4000
    # past 32 GiB of tiles dQ recomputes (bf16 at 65536 positions, fp32 at C5's 16384)
    for args in ((1, 65536, 32, 8, 128, 1, 1), (1, 16384, 64, 8, 128, 0, 1)):
        small, big = _lib.size_out(), _lib.size_out()
        assert lib.kf_attn_bwd_workspace_size(*args[:6], ctypes.byref(small)) == 0
        assert lib.kf_attn_bwd_workspace_size_ds(*args, ctypes.byref(big)) == 0
        assert big.value == small.value
    # fp32: rotated Q and K float32 [Sp][D] (Sp = S rounded up to 64), two floats of
    # row statistics per query row, float64 group sums of dK and dV per key row,
    # then the mask records (an int2 per batch row and 32-position tile, an int32
    # per batch row); kept dS: float32 [32][64] blocks, tile t holding t // 2 + 1
    al = lambda x: (x + 255) // 256 * 256  # noqa: E731
    f32 = al(al((B * Hq * P * D + B * Hkv * P * D + B * Hq * P * 2) * 4)
             + B * S * Hkv * D * 2 * 8) + B * (S // 32) * 8 + B * 4
    assert lib.kf_attn_bwd_workspace_size(B, S, Hq, Hkv, D, 0, ctypes.byref(n)) == 0
    assert n.value == f32
    assert lib.kf_attn_bwd_workspace_size_ds(B, S, Hq, Hkv, D, 0, 1, ctypes.byref(n)) == 0
    blocks = sum(t // 2 + 1 for t in range(S // 32))
    assert n.value == al(f32) + B * Hq * blocks * 32 * 64 * 4
    # rotated operands kept from the forward: K per KV head then Q per query head,
    # bf16 [P][D]; the backward reading them needs that much less workspace
    assert lib.kf_attn_rot_size(B, S, Hq, Hkv, D, 1, 0, 0, ctypes.byref(n)) == 0
    rot = (B * Hkv + B * Hq) * P * D * 2
    assert n.value == rot
    assert lib.kf_attn_rot_size(B, 4000, Hq, Hkv, D, 1, 1, 0, ctypes.byref(n)) == 0
    assert n.value == rot  # P = 4096 for S = 4000
    assert lib.kf_attn_bwd_rot_workspace_size(B, S, Hq, Hkv, D, 1, 1, 0, ctypes.byref(n)) == 0
    assert n.value == base - rot
    assert lib.kf_attn_bwd_rot_workspace_size(B, S, Hq, Hkv, D, 1, 1, 1, ctypes.byref(n)) == 0
    assert n.value == (base - rot + 255) // 256 * 256 + B * Hq * P * (P + 64)
    # only the bf16 MFMA kernels take that path (fp32, head_dim 96, both masks)
    for args in ((B, S, Hq, Hkv, D, 0, 0, 0), (B, S, Hq, Hkv, 96, 1, 0, 0),
                 (B, S, Hq, Hkv, D, 1, 1, 1)):
        assert lib.kf_attn_rot_size(*args, ctypes.byref(n)) == 2
    assert lib.kf_attn_bwd_rot_workspace_size(B, S, Hq, Hkv, 96, 1, 1, 0, ctypes.byref(n)) == 2
    # kv-cache overflow is rejected on the host (reference generate.py:92-96 guard)
    rc = lib.kf_kv_cache_append(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                                ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                                10, 1, 8, 2, 16, 64, 1, None)
    assert rc == 1 and b"overflow" in lib.kf_last_error()


def test_attention_constructor_contract():
    sig = inspect.signature(Attention.__init__)
    assert list(sig.parameters) == ["self", "dim", "n_heads", "n_kv_heads", "head_dim",
                                    "qk_norm", "sdpa_backend"]
    fsig = inspect.signature(Attention.forward)
    assert list(fsig.parameters) == ["self", "x", "rope_cos", "rope_sin", "kv_cache", "doc_ids",
                                     "key_padding_mask"]
    a = Attention(dim=256, n_heads=8, n_kv_heads=2, qk_norm=True, sdpa_backend="math")
    assert (a.n_heads, a.n_kv_heads, a.head_dim, a.n_rep) == (8, 2, 32, 4)
    assert a.sdpa_backend == "math" and a.capture_attention_weights is False
    assert a.last_attention_weights is None
    assert sorted(a.state_dict()) == ["k_norm.weight", "k_proj.weight", "o_proj.weight",
                                      "q_norm.weight", "q_proj.weight", "v_proj.weight"]
    assert a.q_proj.weight.shape == (256, 256) and a.k_proj.weight.shape == (64, 256)
    assert Attention(dim=128, n_heads=4, n_kv_heads=4).q_norm is None


def test_kvcache_contract_cpu():
    # reference tests/unit/test_generate.py:33-89 (storage and update semantics)
    c = KVCache(2, 16, 4, 8, torch.float32, torch.device("cpu"))
    assert c.k.shape == (2, 4, 16, 8) and c.seq_len == 0 and (c.k == 0).all()
    k1, v1 = torch.randn(2, 4, 3, 8), torch.randn(2, 4, 3, 8)
    ka, va = c.update(k1, v1)
    assert ka.shape == (2, 4, 3, 8) and torch.equal(ka, k1) and c.seq_len == 3
    k2, v2 = torch.randn(2, 4, 1, 8), torch.randn(2, 4, 1, 8)
    ka, va = c.update(k2, v2)
    assert torch.equal(ka, torch.cat([k1, k2], 2)) and torch.equal(va, torch.cat([v1, v2], 2))
    assert c.lens.tolist() == [4, 4]


def test_cpu_tensors_are_rejected_loudly():
    a = Attention(dim=64, n_heads=4, n_kv_heads=2)
    cos, sin = kempnerforge_amd.precompute_rope_frequencies(16, 8)
    with pytest.raises(RuntimeError):
        a(torch.randn(1, 8, 64), cos, sin)


def test_oracle_not_imported_by_product():
    pkg = os.path.join(ROOT, "kempnerforge_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith(".py"):
                src = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in src, f


def test_kept_ds_budget_decision():
    """The backward keeps its dS tiles only within the memory budget (half of
    what the allocator can still hand out by default)."""
    from kempnerforge_amd import ops

    gib = 1 << 30
    assert ops.keep_ds_tiles(2 * gib, 10 * gib)
    assert not ops.keep_ds_tiles(6 * gib, 10 * gib)
    assert ops.keep_ds_tiles(6 * gib, 10 * gib, fraction=0.8)
    assert not ops.keep_ds_tiles(0, 10 * gib)  # the library offers none (key padding, caps)
    assert ops.keep_ds_tiles(1, None)          # availability unknown: keep
    with pytest.raises(ValueError):
        ops.set_backward_ds_budget(0.0)


def test_noalloc_rejects_oversized_partials():
    """kf_attn_decode_noalloc refuses partials beyond its 32 MiB static array on
    the host, before it looks up the array or launches anything: the pointers
    here are never dereferenced (no device is touched)."""
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    lib = _lib.load()
    nbytes = _lib.size_out()
    B, Hq, Hkv, D = 4096, 64, 8, 128
    assert lib.kf_attn_decode_workspace_size(B, Hq, Hkv, D, 1024, _lib.DTYPE_BF16,
                                             ctypes.byref(nbytes)) == 0
    assert nbytes.value > 32 << 20
    p = ctypes.c_void_p(1 << 20)  # non-null, never dereferenced
    rc = lib.kf_attn_decode_noalloc(p, p, p, p, p, p, p, p, 0, 1, p, B, 1024, Hq, Hkv, D, 1024,
                                    None, None, ctypes.c_float(1e-5), _lib.DTYPE_BF16,
                                    ctypes.c_void_p(0))
    assert rc == 4 and b"static scratch" in lib.kf_last_error()
