"""MFU accounting and profiler kernel classification that know MI355X.

Mirrors ``kempnerforge/metrics/mfu.py:25-175`` (peak table, PaLM-style flops
per token, ``compute_mfu``) and the kernel bucketing of
``kempnerforge/profiling/profiler.py:75-114`` with the same function names,
arguments and return values.  What changes:

* the peak table has the AMD Instinct parts (dense bf16, no sparsity), and an
  unknown AMD GPU is estimated from its gfx architecture and CU count instead
  of falling through to the CUDA compute-capability guess (ROCm reports gfx950
  as capability 9.5, which the reference would read as a Hopper, 989 TFLOPS);
* the classifier recognises the ROCm library kernel names (Tensile ``Cijk_``,
  hipBLASLt, CK), RCCL, the HIP runtime's copy/fill kernels and this package's
  attention kernels, which get a bucket of their own.

``config`` arguments are duck-typed: any object with the reference
``ModelConfig`` fields used below (``dim``, ``n_layers``, ``n_heads``,
``n_kv_heads``, ``head_dim``, ``vocab_size``, ``computed_ffn_hidden_dim``,
``is_moe``, ``max_seq_len`` and, for MoE, ``moe_frequency``, ``moe_top_k``,
``moe_shared_experts``).
"""

from __future__ import annotations

import logging

import torch

logger = logging.getLogger(__name__)

# Dense bf16 peak TFLOPS per GPU (one logical device).  AMD: CUs x peak engine
# clock x dense bf16 MFMA flops per CU per clock (gfx950 4096, gfx942 2048,
# gfx90a 1024); NVIDIA entries as in the reference table.
_GPU_PEAK_TFLOPS: dict[str, float] = {
    # AMD Instinct
    "MI355X": 2516.6,  # 256 CU x 2.4 GHz x 4096
    "MI350X": 2306.9,  # 256 CU x 2.2 GHz x 4096
    "MI325X": 1307.4,  # 304 CU x 2.1 GHz x 2048
    "MI300X": 1307.4,  # 304 CU x 2.1 GHz x 2048
    "MI300A": 980.6,   # 228 CU x 2.1 GHz x 2048
    "MI250X": 191.5,   # per GCD: 110 CU x 1.7 GHz x 1024
    "MI250": 181.0,    # per GCD: 104 CU x 1.7 GHz x 1024
    "MI210": 181.0,    # 104 CU x 1.7 GHz x 1024
    # NVIDIA (reference table)
    "H200": 989.0,
    "H100": 989.0,
    "H100 SXM": 989.0,
    "H100 PCIe": 756.0,
    "H800": 989.0,
    "A100": 312.0,
    "A100 SXM": 312.0,
    "A100 PCIe": 312.0,
    "A100-SXM4-80GB": 312.0,
    "A100-SXM4-40GB": 312.0,
    "A100-PCIE-80GB": 312.0,
    "A100-PCIE-40GB": 312.0,
    "A10G": 125.0,
    "L40S": 362.0,
    "RTX 4090": 330.0,
    "RTX 3090": 142.0,
}

# gfx architecture -> (dense bf16 flops per CU per clock, peak engine clock GHz)
_AMD_ARCH: dict[str, tuple[int, float]] = {
    "gfx950": (4096, 2.4),
    "gfx942": (2048, 2.1),
    "gfx941": (2048, 2.1),
    "gfx940": (2048, 2.1),
    "gfx90a": (1024, 1.7),
}


def _amd_arch(device: int) -> str | None:
    if torch.version.hip is None:
        return None
    arch = getattr(torch.cuda.get_device_properties(device), "gcnArchName", "") or ""
    return arch.split(":")[0] or None


def get_gpu_peak_tflops(device: int = 0) -> float:
    """Peak dense bf16 TFLOPS of ``device`` (reference ``mfu.py:48-87``).

    Name match first (longest names first, so "MI300X" does not match an
    "MI300A"); then, on ROCm, an estimate from the gfx architecture and the CU
    count; then the reference's compute-capability guess for CUDA devices.
    Returns 1.0 without a GPU.
    """
    if not torch.cuda.is_available():
        return 1.0
    name = torch.cuda.get_device_name(device)
    for gpu_name in sorted(_GPU_PEAK_TFLOPS, key=len, reverse=True):
        if gpu_name in name:
            tflops = _GPU_PEAK_TFLOPS[gpu_name]
            logger.info(f"Detected GPU: {name} -> {tflops} bf16 TFLOPS")
            return tflops
    arch = _amd_arch(device)
    if arch is not None:
        per_cu, ghz = _AMD_ARCH.get(arch, (1024, 1.5))
        cus = torch.cuda.get_device_properties(device).multi_processor_count
        tflops = round(cus * ghz * per_cu / 1e3, 1)
        logger.warning(f"Unknown AMD GPU: {name} ({arch}, {cus} CUs). Using estimated "
                       f"{tflops} bf16 TFLOPS. Add it to _GPU_PEAK_TFLOPS for accuracy.")
        return tflops
    major, minor = torch.cuda.get_device_capability(device)
    tflops = 989.0 if major >= 9 else 312.0 if major >= 8 else 100.0
    logger.warning(f"Unknown GPU: {name} (cc {major}.{minor}). Using estimated {tflops} bf16 "
                   "TFLOPS. Add this GPU to _GPU_PEAK_TFLOPS for accuracy.")
    return tflops


def _attn_params(config) -> int:
    head_dim = config.head_dim
    return (config.dim * (config.n_heads * head_dim)
            + 2 * config.dim * (config.n_kv_heads * head_dim)
            + (config.n_heads * head_dim) * config.dim)


def estimate_model_flops_per_token(config, seq_len: int | None = None) -> int:
    """Forward+backward flops per token, ``6*P_active + 12*L*D*S`` (PaLM), as in
    the reference (``mfu.py:90-147``): embedding excluded, output projection
    included, MoE counting the top-k routed plus shared experts of the MoE
    layers, GQA not discounted in the attention term."""
    s = seq_len if seq_len is not None else config.max_seq_len
    mlp_params = 3 * config.dim * config.computed_ffn_hidden_dim  # SwiGLU
    attn = _attn_params(config)
    output_params = config.vocab_size * config.dim
    if getattr(config, "is_moe", False):
        n_moe = sum(1 for i in range(config.n_layers) if (i + 1) % config.moe_frequency == 0)
        n_dense = config.n_layers - n_moe
        shared = config.moe_shared_experts * mlp_params
        active = (n_dense * (attn + mlp_params)
                  + n_moe * (attn + config.moe_top_k * mlp_params + shared) + output_params)
    else:
        active = config.n_layers * (attn + mlp_params) + output_params
    return 6 * active + 12 * config.n_layers * config.dim * s


def compute_mfu(config, tokens_per_sec: float, num_gpus: int = 1,
                gpu_peak_tflops: float | None = None, seq_len: int | None = None) -> float:
    """Model flops utilisation in [0, 1] (reference ``mfu.py:150-175``)."""
    if gpu_peak_tflops is None:
        gpu_peak_tflops = get_gpu_peak_tflops()
    achieved = estimate_model_flops_per_token(config, seq_len=seq_len) * tokens_per_sec / 1e12
    peak = gpu_peak_tflops * num_gpus
    return 0.0 if peak == 0 else achieved / peak


def causal_attention_pairs(batch: int, n_heads: int, seq_len: int, doc_lengths=None) -> int:
    """Visible (query, key) pairs of causal attention over ``batch`` sequences,
    or, with ``doc_lengths`` (one list of document lengths per sequence, packed
    documents), of the same-document causal pairs only."""
    if doc_lengths is None:
        return batch * n_heads * seq_len * (seq_len + 1) // 2
    return n_heads * sum(n * (n + 1) // 2 for lens in doc_lengths for n in lens)


def attention_kernel_flops(pairs: int, head_dim: int, backward: bool = True) -> float:
    """Matmul flops of exact attention over ``pairs`` visible pairs: 4*D per
    pair forward (QK^T and PV), 10*D more backward (recomputed QK^T, dP, dV,
    dK, dQ)."""
    return (14.0 if backward else 4.0) * head_dim * pairs


# ---------------------------------------------------------------- profiler
_ATTN_KEYS = ("fwd_mfma", "bwd_dkdv", "bwd_dq", "q_prep_bwd", "kv_prep", "decode_stream",
              "decode_merge", "decode_generic", "capture_probs", "fwd_generic",
              "bwd_dq_generic", "bwd_dkdv_generic", "cache_append", "append_kernel",
              "doc_block_tiles", "order_by_count",
              "kf::attn", "flash", "fmha", "attention")
_MATMUL_KEYS = ("gemm", "mm", "matmul", "dot", "bmm", "cublas", "nvjet", "cutlass",
                "cijk_", "hipblaslt", "rocblas", "ck_tile", "wvsplitk")
_COMM_KEYS = ("nccl", "rccl", "allreduce", "allgather", "reduce_scatter", "alltoall")
_MEMORY_KEYS = ("memcpy", "memset", "copybuffer", "fillbuffer")


def classify_kernel(name: str) -> str:
    """Bucket of a profiler event: "attention", "matmul", "comm", "memory" or
    "other" (the reference's buckets, ``profiler.py:92-103``, plus attention)."""
    n = name.lower()
    if any(k in n for k in _ATTN_KEYS):
        return "attention"
    if any(k in n for k in _MATMUL_KEYS):
        return "matmul"
    if any(k in n for k in _COMM_KEYS):
        return "comm"
    if any(k in n for k in _MEMORY_KEYS):
        return "memory"
    return "other"


def analyze_profiler(prof) -> dict:
    """Aggregate device time per bucket of a finished ``torch.profiler`` run,
    with the keys of the reference's ``_analyze_profiler`` (``profiler.py:
    75-114``) plus ``attention_time_us`` / ``attention_pct``."""
    times = {"matmul": 0, "attention": 0, "comm": 0, "memory": 0, "other": 0}
    total_time = 0
    total_flops = 0
    for evt in prof.key_averages():
        name = evt.key
        if "profilerstep" in name.lower():
            continue
        us = evt.self_device_time_total
        total_time += us
        total_flops += evt.flops if evt.flops else 0
        times[classify_kernel(name)] += us
    denom = max(total_time, 1)
    peak = get_gpu_peak_tflops()
    achieved = total_flops / (total_time / 1e6) / 1e12 if total_time > 0 else 0.0
    out = {"total_cuda_time_us": total_time}
    for k in ("matmul", "comm", "memory", "other", "attention"):
        out[f"{k}_time_us"] = times[k]
    for k in ("matmul", "comm", "memory", "other", "attention"):
        out[f"{k}_pct"] = 100 * times[k] / denom
    out.update(total_flops=total_flops, achieved_tflops=achieved, peak_tflops=peak,
               kernel_efficiency_pct=100 * achieved / peak if peak > 0 else 0.0)
    return out
