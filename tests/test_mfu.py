"""MFU accounting and kernel classification on MI355X (kempnerforge_amd.mfu),
checked the way the reference checks its own (tests/unit/test_performance.py:
31-157, 226-260) plus the AMD cases it cannot cover."""

from __future__ import annotations

import math
from dataclasses import dataclass
from types import SimpleNamespace
from unittest.mock import MagicMock

import pytest
import torch

from kempnerforge_amd import mfu


@dataclass
class Cfg:
    """The ModelConfig fields the flops formula reads (reference
    kempnerforge/config/model.py:28-125): head_dim = dim // n_heads, Llama FFN
    width 4*dim*2/3 rounded up to a multiple of 256 unless given."""

    dim: int
    n_layers: int
    n_heads: int
    vocab_size: int
    max_seq_len: int = 2048
    n_kv_heads: int | None = None
    ffn_hidden_dim: int | None = None
    num_experts: int = 0
    moe_top_k: int = 2
    moe_frequency: int = 1
    moe_shared_experts: int = 0

    def __post_init__(self):
        if self.n_kv_heads is None:
            self.n_kv_heads = self.n_heads

    @property
    def is_moe(self):
        return self.num_experts > 0

    @property
    def head_dim(self):
        return self.dim // self.n_heads

    @property
    def computed_ffn_hidden_dim(self):
        if self.ffn_hidden_dim is not None:
            return self.ffn_hidden_dim
        return 256 * math.ceil(int(4 * self.dim * (2 / 3)) / 256)


SMALL = Cfg(dim=256, n_layers=4, n_heads=4, vocab_size=1000, max_seq_len=128)


class TestFlops:
    def test_closed_form_small(self):
        # attn 4*256*256, mlp 3*256*768 (ffn 683 -> 768), 4 layers, output 256*1000
        attn, mlp = 4 * 256 * 256, 3 * 256 * 768
        active = 4 * (attn + mlp) + 1000 * 256
        assert mfu.estimate_model_flops_per_token(SMALL) == 6 * active + 12 * 4 * 256 * 128

    def test_llama_7b_reasonable(self):
        cfg = Cfg(dim=4096, n_layers=32, n_heads=32, vocab_size=32000, ffn_hidden_dim=11008)
        assert 30e9 < mfu.estimate_model_flops_per_token(cfg) < 60e9

    def test_gqa_counts_fewer_kv_params(self):
        mha = Cfg(dim=512, n_layers=2, n_heads=8, vocab_size=100)
        gqa = Cfg(dim=512, n_layers=2, n_heads=8, n_kv_heads=2, vocab_size=100)
        # K and V projections shrink by 6/8 of 2*dim*dim per layer
        diff = mfu.estimate_model_flops_per_token(mha) - mfu.estimate_model_flops_per_token(gqa)
        assert diff == 6 * 2 * (2 * 512 * 512 * 6 // 8)

    def test_moe_active_params(self):
        base = dict(dim=256, n_layers=4, n_heads=4, vocab_size=1000, max_seq_len=128)
        dense = mfu.estimate_model_flops_per_token(Cfg(**base))
        moe = mfu.estimate_model_flops_per_token(Cfg(**base, num_experts=8, moe_top_k=2))
        assert dense < moe < 4 * dense
        half = mfu.estimate_model_flops_per_token(Cfg(**base, num_experts=8, moe_frequency=2))
        assert half < moe
        shared = mfu.estimate_model_flops_per_token(Cfg(**base, num_experts=8,
                                                        moe_shared_experts=1))
        assert shared - moe == 6 * 4 * 3 * 256 * 768

    def test_seq_len_override(self):
        assert (mfu.estimate_model_flops_per_token(SMALL, seq_len=256)
                - mfu.estimate_model_flops_per_token(SMALL, seq_len=64)) == 12 * 4 * 256 * 192

    def test_compute_mfu(self):
        m1 = mfu.compute_mfu(SMALL, 1e6, 1, gpu_peak_tflops=2516.6)
        m4 = mfu.compute_mfu(SMALL, 1e6, 4, gpu_peak_tflops=2516.6)
        assert 0 < m1 < 1 and m4 == pytest.approx(m1 / 4)
        assert mfu.compute_mfu(SMALL, 0.0, 1, gpu_peak_tflops=312.0) == 0.0
        assert mfu.compute_mfu(SMALL, 1e6, 1, gpu_peak_tflops=0.0) == 0.0

    def test_attention_pairs_and_flops(self):
        assert mfu.causal_attention_pairs(1, 1, 4) == 10
        # packed documents: only same-document causal pairs
        assert mfu.causal_attention_pairs(2, 3, 6, [[2, 4], [6]]) == 3 * (3 + 10 + 21)
        assert mfu.attention_kernel_flops(10, 128) == 14 * 128 * 10
        assert mfu.attention_kernel_flops(10, 128, backward=False) == 4 * 128 * 10


def _fake_gpu(monkeypatch, name, arch=None, cus=256, cc=(9, 5)):
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "get_device_name", lambda d=0: name)
    monkeypatch.setattr(torch.cuda, "get_device_capability", lambda d=0: cc)
    props = SimpleNamespace(gcnArchName=arch or "", multi_processor_count=cus)
    monkeypatch.setattr(torch.cuda, "get_device_properties", lambda d=0: props)
    monkeypatch.setattr(torch.version, "hip", "7.0" if arch else None)


class TestPeak:
    def test_cpu_only_dummy(self, monkeypatch):
        monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
        assert mfu.get_gpu_peak_tflops() == 1.0

    @pytest.mark.parametrize("name,want", [("AMD Instinct MI355X", 2516.6),
                                           ("AMD Instinct MI350X", 2306.9),
                                           ("AMD Instinct MI300X", 1307.4),
                                           ("AMD Instinct MI300A", 980.6),
                                           ("NVIDIA H100 80GB HBM3", 989.0)])
    def test_name_table(self, monkeypatch, name, want):
        _fake_gpu(monkeypatch, name, arch="gfx950:sramecc+:xnack-" if "AMD" in name else None)
        assert mfu.get_gpu_peak_tflops() == want

    def test_unknown_gfx950_uses_arch_not_capability(self, monkeypatch):
        # ROCm reports gfx950 as capability 9.5; the reference would guess 989
        _fake_gpu(monkeypatch, "AMD Radeon Graphics", arch="gfx950:sramecc+:xnack-", cus=256)
        assert mfu.get_gpu_peak_tflops() == pytest.approx(2516.6, abs=0.1)
        _fake_gpu(monkeypatch, "AMD Radeon Graphics", arch="gfx942", cus=304)
        assert mfu.get_gpu_peak_tflops() == pytest.approx(1307.4, abs=0.1)

    def test_unknown_cuda_fallbacks(self, monkeypatch):
        for cc, want in (((9, 0), 989.0), ((8, 0), 312.0), ((7, 5), 100.0)):
            _fake_gpu(monkeypatch, "Fake-Unknown-GPU-9000", cc=cc)
            assert mfu.get_gpu_peak_tflops() == want

    def test_compute_mfu_auto_detects(self, monkeypatch):
        monkeypatch.setattr(mfu, "get_gpu_peak_tflops", lambda device=0: 100.0)
        assert mfu.compute_mfu(SMALL, 1e6, 1) > 0


class TestClassifier:
    @pytest.mark.parametrize("name,bucket", [
        ("aten::mm", "matmul"),
        ("Cijk_Alik_Bljk_BBS_BH_MT128x128x64_MI16x16x1", "matmul"),
        ("hipblasLt gemm", "matmul"),
        ("ncclDevKernel_Generic", "comm"),
        ("rccl allreduce", "comm"),
        ("__amd_rocclr_copyBuffer", "memory"),
        ("__amd_rocclr_fillBufferAligned", "memory"),
        ("Memcpy DtoD", "memory"),
        ("fwd_mfma_kernel<128, false>", "attention"),
        ("bwd_dkdv_kernel<128, false>", "attention"),
        ("decode_stream_kernel<128, false>", "attention"),
        ("kf::attn_fwd", "attention"),
        ("aten::relu", "other"),
    ])
    def test_buckets(self, name, bucket):
        assert mfu.classify_kernel(name) == bucket

    def test_analyze_profiler(self, monkeypatch):
        monkeypatch.setattr(mfu, "get_gpu_peak_tflops", lambda device=0: 2516.6)

        def evt(key, us, flops=0):
            e = MagicMock()
            e.key, e.self_device_time_total, e.flops = key, us, flops
            return e

        prof = MagicMock()
        prof.key_averages.return_value = [
            evt("aten::mm", 5000, int(1e12)), evt("nccl:allreduce", 2000),
            evt("aten::relu", 1000), evt("fwd_mfma_kernel<128, false>", 2000),
            evt("ProfilerStep#3", 99999)]
        s = mfu.analyze_profiler(prof)
        assert s["matmul_time_us"] == 5000 and s["comm_time_us"] == 2000
        assert s["other_time_us"] == 1000 and s["attention_time_us"] == 2000
        assert s["total_cuda_time_us"] == 10000 and s["total_flops"] == int(1e12)
        assert s["matmul_pct"] == pytest.approx(50.0)
        assert s["achieved_tflops"] == pytest.approx(100.0)
        assert s["peak_tflops"] == 2516.6
