"""MFU peak detection and profiler classification on the real MI355X."""

from __future__ import annotations

import pytest
import torch

from gpu_util import DEV, announce, seeded
from kempnerforge_amd import mfu, ops
from kempnerforge_amd.position import precompute_rope_frequencies

pytestmark = pytest.mark.gpu


def test_peak_is_mi355x():
    announce("mfu peak")
    assert mfu.get_gpu_peak_tflops() == pytest.approx(2516.6, abs=0.1)


def test_profiler_buckets_attention_kernels():
    announce("mfu profiler")
    B, S, Hq, Hkv, D = 1, 256, 8, 2, 128
    q = seeded((B, S, Hq, D), 0, torch.bfloat16).to(DEV).requires_grad_(True)
    k = seeded((B, S, Hkv, D), 1, torch.bfloat16).to(DEV).requires_grad_(True)
    v = seeded((B, S, Hkv, D), 2, torch.bfloat16).to(DEV).requires_grad_(True)
    cos, sin = precompute_rope_frequencies(D, S)
    cos, sin = cos.to(DEV), sin.to(DEV)
    w = torch.randn(D, D, device=DEV, dtype=torch.bfloat16)
    acts = [torch.profiler.ProfilerActivity.CPU, torch.profiler.ProfilerActivity.CUDA]
    with torch.profiler.profile(activities=acts) as prof:
        out = ops.attention(q, k, v, cos, sin)
        (out @ w).float().sum().backward()
        torch.cuda.synchronize()
    s = mfu.analyze_profiler(prof)
    assert s["attention_time_us"] > 0
    assert s["matmul_time_us"] > 0
    assert s["total_cuda_time_us"] >= s["attention_time_us"] + s["matmul_time_us"]
