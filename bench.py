"""Benchmark of the gfx950 attention path on one GPU; prints one JSON line.

Step = one training-step attention pass of the Llama-3-8B shape (BASELINE
config C3): causal GQA forward (RoPE fused) + backward, bf16, B=4, S=4096,
32 query heads, 8 KV heads, head_dim 128, RoPE theta 5e5, seeded N(0,1)
synthetic inputs resident in HBM.  Algorithmic work per step is 14*D*P flops
with P = B*Hq*S*(S+1)/2 causal (query, key) pairs (forward 4*D*P, backward
10*D*P; GQA not discounted).

Also reported: per-kernel HIP-event timings (the library brackets each launch
on its own stream), the roofline of the dominant kernel, the forward alone
(C2), the C3 step on packed documents (C3-doc; flops of same-document pairs
only), with an all-True key_padding_mask (C3-kpm), in float16 (C3-fp16) and in
float32 (C3-fp32; the decode and capture lines also carry float32 runs), one
rank's share of the reference's TP = 4 training configs at S = 4096, the
Llama-3-70B shape fwd+bwd (C5: B=1, S=16384, 64 query heads) and its
2048-token probability capture (C5-cap), the KV-cache decode configuration C4
in GB/s, and the reference's PyTorch paths timed on the host CPU (C3 sample,
C4 decode, C5-cap capture) next to them.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu-baseline]
    python bench.py --only c3|c2|c3doc|c3kpm|c3fp16|c3fp32|c5|c5cap|c4|tp4_70b|tp4_29b|tp4_13b|tp4_7b
                    [--steps K] [--warmup W]
        one workload: W untimed steps, K timed steps, then K steps with the
        per-kernel event timing (the shape profiling runs use)
    python bench.py --rocprof-summary DIR [DIR ...] --warmup W --steps K
        markdown table of rocprofv3 outputs of --only runs (kernel trace and
        --pmc counter collections), launches of the W warm-up steps dropped
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "causal GQA attn TFLOP/s fwd+bwd (8B shape) + decode HBM GB/s, 1 MI355X"
PEAK_BF16_TFLOPS = 2516.6  # 256 CU x 2.4 GHz x 4096 flop/clk, dense
PEAK_HBM_GBPS = 8000.0
SHORT_WARM, SHORT_STEPS = 50, 200  # minimum warm-up / timed calls of the sub-ms lines

C3 = dict(B=4, S=4096, Hq=32, Hkv=8, D=128, theta=500000.0)
C4 = dict(B=32, Hq=32, Hkv=8, D=128, lo=1024, hi=8192, theta=500000.0)
C5 = dict(B=1, S=16384, Hq=64, Hkv=8, D=128, theta=500000.0, cap_tokens=2048)
# one rank's share of the reference's tensor-parallel training configs (TP = 4:
# query and KV heads divided by 4; configs/train/70b_32gpu_tp4.toml,
# 29b_32gpu_tp4_pp2.toml, 13b_32gpu_tp4_pp2.toml, 7b_12gpu_tp4.toml)
TP4_SHARES = {"70b": dict(B=2, Hq=16, Hkv=2), "29b": dict(B=1, Hq=12, Hkv=2),
              "13b": dict(B=4, Hq=10, Hkv=2), "7b": dict(B=4, Hq=8, Hkv=2)}

# what bounds each kernel (the roofline its "achieved" figure is quoted on)
BOUND = {"fwd_mfma": "mfma", "bwd_dkdv": "mfma", "bwd_dq": "mfma", "bwd_dq_ds": "hbm",
         "q_prep_bwd": "hbm", "kv_prep": "hbm", "decode_stream": "hbm", "decode_merge": "hbm",
         "capture_probs": "hbm"}


def pairs(B, Hq, S):
    return B * Hq * S * (S + 1) // 2


def ds_record_bytes(B, Hq, S):
    """Bytes of the dS records the dK/dV kernel keeps for a causal launch."""
    P = (S + 127) // 128 * 128
    return B * Hq * P * (P + 64)


def measured_traffic():
    """HBM bytes per launch of each kernel per workload, from the rocprofv3
    FETCH_SIZE / WRITE_SIZE runs recorded in profiles/hbm_traffic.json (scaled by
    a device copy of known size); {} when that file is absent."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        return {k: v["bytes"] for k, v in json.load(f)["kernels"].items()}


def seeded(shape, seed, dtype, dev):
    import torch

    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype).to(dev)


# --------------------------------------------------------------------------- workloads
class Workloads:
    """Inputs and step functions of every benchmarked configuration."""

    def __init__(self, dev):
        import torch

        from kempnerforge_amd import ops
        from kempnerforge_amd.position import precompute_rope_frequencies

        self.torch, self.ops, self.dev = torch, ops, dev
        self.rope = precompute_rope_frequencies
        self.bf16 = torch.bfloat16
        self._c3 = self._c5 = self._c4 = self._doc = self._ones = self._c3h = None
        self._c3f = None

    # C3 / C2 / C3-doc share the 8B-shape tensors
    def c3_inputs(self):
        if self._c3 is None:
            B, S, Hq, Hkv, D = (C3[k] for k in ("B", "S", "Hq", "Hkv", "D"))
            q = seeded((B, S, Hq, D), 0, self.bf16, self.dev).requires_grad_(True)
            k = seeded((B, S, Hkv, D), 1, self.bf16, self.dev).requires_grad_(True)
            v = seeded((B, S, Hkv, D), 2, self.bf16, self.dev).requires_grad_(True)
            do = seeded((B, S, Hq, D), 3, self.bf16, self.dev)
            cos, sin = self.rope(D, S, C3["theta"])
            self._c3 = (q, k, v, do, cos.to(self.dev), sin.to(self.dev))
        return self._c3

    def c3_step(self):
        q, k, v, do, cos, sin = self.c3_inputs()
        out = self.ops.attention(q, k, v, cos, sin, causal=True)
        self.torch.autograd.grad(out, (q, k, v), do)

    def c3fp16_step(self):
        # the C3 step in float16 (the reference's mixed_precision = "fp16"):
        # the same seeded values, stored as fp16
        if self._c3h is None:
            self._c3h = tuple(t.detach().to(self.torch.float16).requires_grad_(t.requires_grad)
                              if t.is_floating_point() and t.dtype == self.bf16 else t
                              for t in self.c3_inputs())
        q, k, v, do, cos, sin = self._c3h
        out = self.ops.attention(q, k, v, cos, sin, causal=True)
        self.torch.autograd.grad(out, (q, k, v), do)

    def c3fp32_step(self):
        # the C3 step in float32 (the reference's mixed_precision = "fp32"): the
        # same seeded values, on the fp32 matrix-core kernels
        if self._c3f is None:
            self._c3f = tuple(t.detach().float().requires_grad_(t.requires_grad)
                              if t.is_floating_point() and t.dtype == self.bf16 else t
                              for t in self.c3_inputs())
        q, k, v, do, cos, sin = self._c3f
        out = self.ops.attention(q, k, v, cos, sin, causal=True)
        self.torch.autograd.grad(out, (q, k, v), do)

    def tp4_step(self, name):
        # C3's length and head_dim on one rank's share of a TP = 4 config
        if getattr(self, "_tp", (None,))[0] != name:
            self._tp = None
            sh, S, D = TP4_SHARES[name], C3["S"], C3["D"]
            B, Hq, Hkv = sh["B"], sh["Hq"], sh["Hkv"]
            q = seeded((B, S, Hq, D), 0, self.bf16, self.dev).requires_grad_(True)
            k = seeded((B, S, Hkv, D), 1, self.bf16, self.dev).requires_grad_(True)
            v = seeded((B, S, Hkv, D), 2, self.bf16, self.dev).requires_grad_(True)
            do = seeded((B, S, Hq, D), 3, self.bf16, self.dev)
            cos, sin = self.rope(D, S, C3["theta"])
            self._tp = (name, q, k, v, do, cos.to(self.dev), sin.to(self.dev))
        _, q, k, v, do, cos, sin = self._tp
        out = self.ops.attention(q, k, v, cos, sin, causal=True)
        self.torch.autograd.grad(out, (q, k, v), do)

    def c2_step(self):
        q, k, v, _, cos, sin = self.c3_inputs()
        self.ops.fwd_raw(q.detach(), k.detach(), v.detach(), cos, sin, causal=True,
                         k_rotated=False)

    def c3_raw_step(self):
        # the kernels the autograd step runs: the rotated-operand pair
        q, k, v, do, cos, sin = self.c3_inputs()
        qn, kn, vn = q.detach(), k.detach(), v.detach()
        o, l, rot = self.ops.fwd_rot_raw(qn, kn, vn, cos, sin, causal=True)
        return self.ops.bwd_rot_raw(rot, vn, cos, sin, o, l, do, causal=True)

    def doc_inputs(self):
        """C3 on packed sequences: documents of 64..2048 tokens (seed 7)."""
        if self._doc is None:
            torch = self.torch
            B, S, Hq = C3["B"], C3["S"], C3["Hq"]
            g = torch.Generator().manual_seed(7)
            rows, vis = [], 0
            for _ in range(B):
                lens, left = [], S
                while left:
                    n = min(left, int(torch.randint(64, 2049, (1,), generator=g)))
                    lens.append(n)
                    left -= n
                vis += Hq * sum(n * (n + 1) // 2 for n in lens)
                rows.append(torch.cat([torch.full((n,), i, dtype=torch.int32)
                                       for i, n in enumerate(lens)]))
            ndocs = sum(int(r.max()) + 1 for r in rows)
            self._doc = (torch.stack(rows).to(self.dev), vis, ndocs)
        return self._doc

    def c3doc_step(self):
        q, k, v, do, cos, sin = self.c3_inputs()
        doc = self.doc_inputs()[0]
        out = self.ops.attention(q, k, v, cos, sin, causal=True, doc_ids=doc)
        self.torch.autograd.grad(out, (q, k, v), do)

    def c3kpm_step(self):
        # the image-prefix VLM arches pass a key_padding_mask on every step,
        # all-True when nothing is padded
        q, k, v, do, cos, sin = self.c3_inputs()
        if self._ones is None:
            self._ones = self.torch.ones(q.shape[0], q.shape[1], dtype=self.torch.bool,
                                         device=self.dev)
        out = self.ops.attention(q, k, v, cos, sin, causal=True, key_padding_mask=self._ones)
        self.torch.autograd.grad(out, (q, k, v), do)

    def c5_inputs(self):
        if self._c5 is None:
            B, S, Hq, Hkv, D = (C5[k] for k in ("B", "S", "Hq", "Hkv", "D"))
            q = seeded((B, S, Hq, D), 0, self.bf16, self.dev).requires_grad_(True)
            k = seeded((B, S, Hkv, D), 1, self.bf16, self.dev).requires_grad_(True)
            v = seeded((B, S, Hkv, D), 2, self.bf16, self.dev).requires_grad_(True)
            do = seeded((B, S, Hq, D), 3, self.bf16, self.dev)
            cos, sin = self.rope(D, S, C5["theta"])
            Sc = C5["cap_tokens"]
            cap = tuple(t.detach()[:, :Sc].contiguous() for t in (q, k, v))
            self._c5 = (q, k, v, do, cos.to(self.dev), sin.to(self.dev), cap)
        return self._c5

    def c5_step(self):
        q, k, v, do, cos, sin, _ = self.c5_inputs()
        out = self.ops.attention(q, k, v, cos, sin, causal=True)
        self.torch.autograd.grad(out, (q, k, v), do)

    def c5cap_step(self):
        _, _, _, _, cos, sin, (qc, kc, vc) = self.c5_inputs()
        Sc = C5["cap_tokens"]
        self.ops.capture_raw(qc, kc, vc, cos[:Sc], sin[:Sc], causal=True, k_rotated=False)

    def c5_free(self):
        self._c5 = None

    def c4_inputs(self):
        if self._c4 is None:
            torch = self.torch
            g = torch.Generator().manual_seed(4)
            B, Hq, Hkv, D = C4["B"], C4["Hq"], C4["Hkv"], C4["D"]
            lens = torch.randint(C4["lo"], C4["hi"] + 1, (B,), generator=g, dtype=torch.int32)
            Smax = C4["hi"] + 1
            qn = seeded((B, 1, Hq, D), 0, self.bf16, self.dev)
            kn = seeded((B, 1, Hkv, D), 1, self.bf16, self.dev)
            vn = seeded((B, 1, Hkv, D), 2, self.bf16, self.dev)
            # the caches from the same seeded CPU generator as everything else
            # (drawn one sequence at a time, to bound host memory)
            kc = torch.empty(B, Hkv, Smax, D, device=self.dev, dtype=self.bf16)
            vc = torch.empty_like(kc)
            for b in range(B):
                kc[b].copy_(torch.randn(Hkv, Smax, D, generator=g, dtype=self.bf16))
                vc[b].copy_(torch.randn(Hkv, Smax, D, generator=g, dtype=self.bf16))
            cos, sin = self.rope(D, Smax, C4["theta"])
            nbytes = sum(4 * (int(L) + 1) * Hkv * D for L in lens) + 4 * B * Hq * D \
                + 4 * B * Hkv * D
            self._c4 = (qn, kn, vn, kc, vc, lens, lens.to(self.dev), cos.to(self.dev),
                        sin.to(self.dev), Smax, nbytes)
        return self._c4

    def c4_step(self):
        qn, kn, vn, kc, vc, _, lens_d, cos, sin, Smax, _ = self.c4_inputs()
        self.ops.decode_raw(qn, kn, vn, kc, vc, lens_d, cos, sin, rope_row_offset=0,
                            max_len=Smax)


def timed(torch, fn, warm, iters):
    """Seconds per call of fn over iters calls after warm untimed ones,
    bracketed by device synchronisations."""
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    t = time.perf_counter()
    for _ in range(iters):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t) / iters


def kernel_stats(torch, fn, iters):
    """Per-kernel HIP-event averages over iters calls of fn."""
    from kempnerforge_amd import _lib

    with _lib.KernelTimer() as kt:
        for _ in range(iters):
            fn()
        torch.cuda.synchronize()
    return {n: {"avg_us": t / c * 1e3, "launches": c} for n, (t, c) in kt.stats.items()}


def roofline(kstats, algo, traffic, suffix):
    """Roofline object of the kernel taking the most time: algorithmic flops
    (mfma) or bytes (hbm) per launch over its event-timed average duration."""
    dom = max(kstats, key=lambda n: kstats[n]["avg_us"] * kstats[n]["launches"])
    if dom not in algo:
        return None
    bound = BOUND.get(dom, "mfma")
    secs = kstats[dom]["avg_us"] * 1e-6
    if bound == "mfma":
        ach, peak, unit = algo[dom] / secs / 1e12, PEAK_BF16_TFLOPS, "TFLOP/s"
    else:
        ach, peak, unit = algo[dom] / secs / 1e9, PEAK_HBM_GBPS, "GB/s"
    return {"kernel": dom, "bound": bound, "achieved": round(ach, 1), "peak": peak,
            "unit": unit, "frac": round(ach / peak, 4),
            "traffic": traffic.get(f"{dom}@{suffix}"),
            "traffic_source": "profiles/hbm_traffic.json (rocprofv3 --pmc FETCH_SIZE, "
                              "WRITE_SIZE; scaled by a device copy)",
            "avg_us": round(kstats[dom]["avg_us"], 1)}


# --------------------------------------------------------------------------- CPU legs
def cpu_legs(args, torch, wl):
    """The reference's PyTorch paths on the host CPU, on bounded samples."""
    from oracle import cpu_baseline as cb

    cores = cb.cpu_threads()
    model = cb.cpu_model()
    bf16 = torch.bfloat16
    D = C3["D"]
    out = {}
    # C3: 1/16 of the step (one batch row, one KV group pair)
    sample = dict(B=1, S=C3["S"], Hq=8, Hkv=2)
    secs, reps, used = cb.time_fwd_bwd(sample["B"], sample["S"], sample["Hq"], sample["Hkv"], D,
                                       C3["theta"], bf16, min_seconds=args.cpu_seconds)
    fl = 14.0 * D * pairs(sample["B"], sample["Hq"], sample["S"])
    out["c3"] = {"value": round(fl / secs / 1e12, 4), "unit": "TFLOP/s", "cores": cores,
                 "kind": "port", "cpu": model,
                 "sample": (f"reference PyTorch path (apply_rope -> repeat_interleave -> SDPA "
                            f"is_causal, autograd) fwd+bwd on CPU, {str(used)[6:]}, B=1 "
                            f"S={sample['S']} Hq=8 Hkv=2 D={D} (1/16 of C3), median of {reps}")}
    # C4: the whole decode batch, one sequence at a time
    lens = [int(x) for x in wl.c4_inputs()[5]]
    Hq, Hkv = C4["Hq"], C4["Hkv"]
    secs, reps, used = cb.time_decode(lens, Hq, Hkv, D, C4["theta"], bf16,
                                      min_seconds=args.cpu_seconds, max_reps=10)
    nbytes = wl.c4_inputs()[-1]
    out["c4"] = {"value": round(nbytes / secs / 1e9, 3), "unit": "GB/s", "cores": cores,
                 "kind": "port", "cpu": model,
                 "sample": (f"reference decode step (RoPE at L_b, KVCache.update, "
                            f"repeat_interleave of the cache, SDPA is_causal=False) on CPU, "
                            f"{str(used)[6:]}, all {len(lens)} C4 sequences one at a time, "
                            f"median of {reps}")}
    # C5-cap: the whole 2048-token capture
    Sc = C5["cap_tokens"]
    secs, reps, used = cb.time_capture(Sc, C5["Hq"], C5["Hkv"], D, C5["theta"], bf16,
                                       min_seconds=args.cpu_seconds, max_reps=10)
    cap_bytes = capture_bytes()
    out["c5cap"] = {"value": round(cap_bytes / secs / 1e9, 3), "unit": "GB/s", "cores": cores,
                    "kind": "port", "cpu": model,
                    "sample": (f"reference _attention_with_weights (matmul, scale, "
                               f"masked_fill, softmax, matmul) on CPU, {str(used)[6:]}, the "
                               f"full C5-cap slice [1,64,2048,2048], median of {reps}; bytes "
                               f"counted as for the GPU (fp32 P written)")}
    return out


def capture_bytes():
    Sc, Hq, Hkv, D = C5["cap_tokens"], C5["Hq"], C5["Hkv"], C5["D"]
    return 4 * Hq * Sc * Sc + Sc * (Hq + 2 * Hkv) * D * 2 + Sc * Hq * D * 2


# --------------------------------------------------------------------------- modes
def run_only(args, torch, wl):
    """One workload: W untimed steps, K timed steps, K event-timed steps."""
    steps = {"c3": wl.c3_step, "c2": wl.c2_step, "c3doc": wl.c3doc_step,
             "c3kpm": wl.c3kpm_step, "c3fp16": wl.c3fp16_step, "c3fp32": wl.c3fp32_step,
             "c5": wl.c5_step,
             **{f"tp4_{n}": (lambda n=n: wl.tp4_step(n)) for n in TP4_SHARES},
             "c5cap": wl.c5cap_step, "c4": wl.c4_step}
    fn = steps[args.only]
    secs = timed(torch, fn, args.warmup, args.steps)
    ks = kernel_stats(torch, fn, args.steps)
    print(json.dumps({"workload": args.only, "steps": args.steps, "warmup": args.warmup,
                      "ms_per_step": round(secs * 1e3, 4),
                      "kernels_us": {n: round(s["avg_us"], 1) for n, s in ks.items()},
                      "launches": {n: s["launches"] for n, s in ks.items()}}), flush=True)
    return 0


def run_full(args, torch, wl):
    B, S, Hq, Hkv, D = (C3[k] for k in ("B", "S", "Hq", "Hkv", "D"))
    P = pairs(B, Hq, S)
    flops_step = 14.0 * D * P
    traffic = measured_traffic()

    # C3: the headline step (autograd forward + backward)
    secs = timed(torch, wl.c3_step, args.warmup, args.steps)
    ms_step = secs * 1e3
    value = flops_step / secs / 1e12
    kstats = kernel_stats(torch, wl.c3_step, args.steps)
    algo = {"fwd_mfma": 4.0 * D * P, "bwd_dkdv": 8.0 * D * P, "bwd_dq": 2.0 * D * P,
            "bwd_dq_ds": float(ds_record_bytes(B, Hq, S))}
    roof = roofline(kstats, algo, traffic, "C3")
    fwd_us = kstats.get("fwd_mfma", {}).get("avg_us")

    # C2: forward only (out + LSE) on the same tensors
    c2_s = timed(torch, wl.c2_step, args.warmup, args.steps)
    c2 = {"config": "C2 llama3-8b fwd B=4 S=4096 Hq=32 Hkv=8 D=128", "ms": round(c2_s * 1e3, 4),
          "TFLOP/s": round(4.0 * D * P / c2_s / 1e12, 1)}

    # C3 replayed from a HIP graph (the raw rotated-operand forward + backward
    # captured once): the same kernels without per-launch host overhead or autograd
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            wl.c3_raw_step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        wl.c3_raw_step()
    c3g_s = timed(torch, graph.replay, args.warmup, args.steps)
    c3_graph = {"config": "C3 step as one HIP graph replay (fwd_rot_raw + bwd_rot_raw)",
                "ms": round(c3g_s * 1e3, 4), "TFLOP/s": round(flops_step / c3g_s / 1e12, 1)}
    del graph

    # C3-doc: flops count only same-document causal pairs
    _, vis, ndocs = wl.doc_inputs()
    doc_s = timed(torch, wl.c3doc_step, args.warmup, args.steps)
    c3doc = {"config": f"C3-doc C3 with packed documents of 64..2048 tokens (seed 7), "
                       f"{ndocs} documents",
             "ms": round(doc_s * 1e3, 4), "TFLOP/s": round(14.0 * D * vis / doc_s / 1e12, 1),
             "visible_pair_frac": round(vis / P, 4),
             "speedup_vs_dense_causal": round(ms_step / (doc_s * 1e3), 2)}

    # C3-kpm: the C3 step with an all-True key_padding_mask (what the VLM arches
    # pass when nothing is padded): the explicit-mask kernels, dS records kept
    kpm_s = timed(torch, wl.c3kpm_step, args.warmup, args.steps)
    kk = kernel_stats(torch, wl.c3kpm_step, args.steps)
    c3kpm = {"config": "C3-kpm C3 with an all-True key_padding_mask",
             "ms": round(kpm_s * 1e3, 4), "TFLOP/s": round(flops_step / kpm_s / 1e12, 1),
             "vs_unmasked_step": round(kpm_s * 1e3 / ms_step, 3),
             "kernels_us": {n: round(s["avg_us"], 1) for n, s in kk.items()},
             "launches_per_step": {n: s["launches"] // args.steps for n, s in kk.items()}}

    # C3-fp16: the C3 step on float16 inputs (mixed_precision = "fp16")
    h_s = timed(torch, wl.c3fp16_step, args.warmup, args.steps)
    kh = kernel_stats(torch, wl.c3fp16_step, args.steps)
    c3fp16 = {"config": "C3-fp16 C3 with float16 q/k/v/dO (the same seeded values)",
              "ms": round(h_s * 1e3, 4), "TFLOP/s": round(flops_step / h_s / 1e12, 1),
              "vs_bf16_step": round(h_s * 1e3 / ms_step, 3),
              "kernels_us": {n: round(s["avg_us"], 1) for n, s in kh.items()}}
    wl._c3h = None

    # C3-fp32: the C3 step on float32 inputs (mixed_precision = "fp32"), whose
    # matrix-core peak is 157.3 TFLOP/s (dense fp32)
    f_s = timed(torch, wl.c3fp32_step, 2, max(2, args.steps // 4))
    kf = kernel_stats(torch, wl.c3fp32_step, max(2, args.steps // 4))
    c3fp32 = {"config": "C3-fp32 C3 with float32 q/k/v/dO (the same seeded values)",
              "ms": round(f_s * 1e3, 3), "TFLOP/s": round(flops_step / f_s / 1e12, 1),
              "frac_of_fp32_peak": round(flops_step / f_s / 157.3e12, 3),
              "kernels_us": {n: round(s["avg_us"], 1) for n, s in kf.items()}}
    wl._c3f = None

    # one rank's share of the reference's TP = 4 training configs at S = 4096
    tp4 = {}
    for name, sh in TP4_SHARES.items():
        step = lambda name=name: wl.tp4_step(name)  # noqa: E731
        t_s = timed(torch, step, args.warmup, args.steps)
        Pn = pairs(sh["B"], sh["Hq"], S)
        tp4[name] = {"B": sh["B"], "Hq": sh["Hq"], "Hkv": sh["Hkv"], "ms": round(t_s * 1e3, 4),
                     "TFLOP/s": round(14.0 * D * Pn / t_s / 1e12, 1)}
        if name == "70b":
            tp4[name]["kernels_us"] = {n: round(s_["avg_us"], 1)
                                       for n, s_ in kernel_stats(torch, step, args.steps).items()}
    wl._tp = None
    tp4 = {"config": "fwd+bwd at S=4096, D=128 on one rank's heads of the reference's TP=4 "
                     "training configs", **tp4}

    # C5 and C5-cap
    P5 = pairs(C5["B"], C5["Hq"], C5["S"])
    c5_s = timed(torch, wl.c5_step, 2, max(5, args.steps // 2))
    k5 = kernel_stats(torch, wl.c5_step, max(3, args.steps // 4))
    algo5 = {"fwd_mfma": 4.0 * D * P5, "bwd_dkdv": 8.0 * D * P5, "bwd_dq": 2.0 * D * P5,
             "bwd_dq_ds": float(ds_record_bytes(C5["B"], C5["Hq"], C5["S"]))}
    c5 = {"config": "C5 llama3-70b fwd+bwd B=1 S=16384 Hq=64 Hkv=8 D=128",
          "ms": round(c5_s * 1e3, 3), "TFLOP/s": round(14.0 * D * P5 / c5_s / 1e12, 1),
          "frac_of_peak": round(14.0 * D * P5 / c5_s / 1e12 / PEAK_BF16_TFLOPS, 4),
          "kernels_us": {n: round(s["avg_us"], 1) for n, s in k5.items()},
          "roofline": roofline(k5, algo5, traffic, "C5")}
    # The capture and decode lines time at least SHORT_STEPS calls after
    # SHORT_WARM untimed ones: a capture call is ~0.3 ms, and its first few
    # dozen calls on a fresh buffer run ~13% slower than the steady state.
    cap_s = timed(torch, wl.c5cap_step, max(args.warmup, SHORT_WARM), max(args.steps, SHORT_STEPS))
    kcap = kernel_stats(torch, wl.c5cap_step, args.steps)
    cap_b = capture_bytes()
    c5cap = {"config": "C5-cap first 2048 tokens of C5, P [1,64,2048,2048] fp32",
             "us": round(cap_s * 1e6, 1), "bytes": cap_b, "GB/s": round(cap_b / cap_s / 1e9, 1),
             "frac_of_hbm_peak": round(cap_b / cap_s / 1e9 / PEAK_HBM_GBPS, 4),
             "kernels_us": {n: round(s["avg_us"], 1) for n, s in kcap.items()},
             "capture_kernel_traffic": traffic.get("capture_probs@C5CAP")}
    # the same capture on float32 inputs (the fp32 kernels: forward, then P)
    cap32 = [t.float() for t in wl.c5_inputs()[6]]
    Sc = C5["cap_tokens"]
    cos5, sin5 = wl.c5_inputs()[4][:Sc], wl.c5_inputs()[5][:Sc]
    cap32_step = lambda: wl.ops.capture_raw(*cap32, cos5, sin5, causal=True,  # noqa: E731
                                            k_rotated=False)
    cap32_s = timed(torch, cap32_step, 3, 10)
    c5cap["fp32"] = {"config": "C5-cap with float32 q/k/v (the same seeded values)",
                     "us": round(cap32_s * 1e6, 1),
                     "kernels_us": {n: round(s["avg_us"], 1)
                                    for n, s in kernel_stats(torch, cap32_step, 10).items()}}
    del cap32
    wl.c5_free()

    # C4 decode
    dec_bytes = wl.c4_inputs()[-1]
    n_dec = max(args.steps, SHORT_STEPS)
    dec_s = timed(torch, wl.c4_step, max(args.warmup, SHORT_WARM), n_dec)
    dstats = kernel_stats(torch, wl.c4_step, n_dec)
    stream_us = dstats.get("decode_stream", {}).get("avg_us")
    decode = {"config": "C4 B=32 Hq=32 Hkv=8 D=128 L~U[1024,8192] seed 4",
              "bytes": dec_bytes, "us_per_step": round(dec_s * 1e6, 1),
              "GB/s": round(dec_bytes / dec_s / 1e9, 1),
              "frac_of_hbm_peak": round(dec_bytes / dec_s / 1e9 / PEAK_HBM_GBPS, 4),
              "kernels_us": {n: round(s["avg_us"], 1) for n, s in dstats.items()},
              "stream_kernel_GB/s": round(dec_bytes / (stream_us * 1e-6) / 1e9, 1)
              if stream_us else None,
              "stream_kernel_traffic": traffic.get("decode_stream@C4")}
    # the same decode on float32 inputs and caches (twice the bytes)
    qn4, kn4, vn4, kc4, vc4, _, lens4, cos4, sin4, Smax4, _ = wl.c4_inputs()
    dec32 = [t.float() for t in (qn4, kn4, vn4, kc4, vc4)]
    dec32_step = lambda: wl.ops.decode_raw(*dec32, lens4, cos4, sin4,  # noqa: E731
                                           rope_row_offset=0, max_len=Smax4)
    d32_s = timed(torch, dec32_step, SHORT_WARM, SHORT_STEPS)
    decode["fp32"] = {"config": "C4 with float32 q/k/v and caches", "bytes": 2 * dec_bytes,
                      "us_per_step": round(d32_s * 1e6, 1),
                      "GB/s": round(2 * dec_bytes / d32_s / 1e9, 1),
                      "kernels_us": {n: round(s["avg_us"], 1) for n, s in
                                     kernel_stats(torch, dec32_step, SHORT_STEPS).items()}}
    del dec32

    cpu = None
    if not args.no_cpu_baseline:
        legs = cpu_legs(args, torch, wl)
        cpu = legs["c3"]
        decode["cpu_baseline"] = legs["c4"]
        c5cap["cpu_baseline"] = legs["c5cap"]

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v/dO, resident in HBM)",
        "config": {"workload": "llama3-8b causal GQA attention fwd+bwd (C3)", "batch": B,
                   "seq_len": S, "n_heads": Hq, "n_kv_heads": Hkv, "head_dim": D,
                   "rope_theta": C3["theta"], "parallelism": "single GPU"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "frac_of_peak_step": round(value / PEAK_BF16_TFLOPS, 4),
        "kernels_us": {n: round(s["avg_us"], 1) for n, s in kstats.items()},
        "fwd_tflops": round(4.0 * D * P / (fwd_us * 1e-6) / 1e12, 1) if fwd_us else None,
        "c2_fwd": c2,
        "c3_graph": c3_graph,
        "c3_doc": c3doc,
        "c3_kpm": c3kpm,
        "c3_fp16": c3fp16,
        "c3_fp32": c3fp32,
        "tp4_shares": tp4,
        "c5": c5,
        "c5_cap": c5cap,
        "decode": decode,
    }
    print(json.dumps(line), flush=True)
    return 0


# --------------------------------------------------------------------------- rocprof summary
def _short(name: str) -> str:
    """Kernel symbol -> the launcher's name (kf::..._kernel<...> -> ...)."""
    m = re.search(r"(fwd_f32|bwd_dq_rec_f32|bwd_dq_f32|bwd_dkdv_f32|rows_f32|stats_f32|"
                  r"mask_prep_f32|capture_f32|decode_merge_f32|decode_f32|"
                  r"kv_prep|fwd_mfma|fwd32|q_prep_bwd|bwd_dkdv|bwd_dq_ds2|bwd_dq_ds|bwd_dq|decode_stream|"
                  r"decode_merge|capture_probs_mfma|kv_append|append|doc_block_tiles|"
                  r"order_by_count|kpm_row_flags|dkdv_reduce)_kernel", name)
    if m:
        # fwd32_kernel is the unmasked forward's kernel, launched as fwd_mfma;
        # bwd_dq_ds2_kernel (two query tiles per workgroup) as bwd_dq_ds
        return {"capture_probs_mfma": "capture_probs", "append": "kv_append",
                "fwd32": "fwd_mfma", "bwd_dq_ds2": "bwd_dq_ds"}.get(m.group(1), m.group(1))
    return "copy" if "copyBuffer" in name else name[:40]


def _ours(name: str) -> bool:
    """A kernel of this library (rocprofv3 reports some names mangled, some
    demangled)."""
    return "_ZN2kf" in name or "kf::" in name


def _drop_warmup(rows, warmup, steps, key):
    """Per kernel, drop the launches of the warm-up steps (the first
    warmup * launches-per-step of that kernel)."""
    by = {}
    for r in rows:
        by.setdefault(key(r), []).append(r)
    out = {}
    for k, rs in by.items():
        per = len(rs) // (warmup + 2 * steps) if len(rs) % (warmup + 2 * steps) == 0 else 0
        out[k] = rs[warmup * per:] if per else rs
    return out


def _run_shape(d, warmup, steps):
    """(warmup, steps) of the --only run profiled into d, read from the JSON
    line it printed into d + ".log" when present."""
    log = d.rstrip("/") + ".log"
    if os.path.exists(log):
        with open(log) as f:
            for line in f:
                if line.startswith("{") and '"warmup"' in line:
                    j = json.loads(line)
                    return j["warmup"], j["steps"]
    return warmup, steps


COPY_KIB = 262144.0  # --copy-calibration copies 256 MiB


def rocprof_summary(dirs, warmup, steps, traffic_json=None):
    lines = []
    traffic = {}
    for d in dirs:
        wl = os.path.basename(d.rstrip("/"))
        warmup, steps = _run_shape(d, warmup, steps)
        trace = sorted(glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True))
        pmc = sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True))
        if trace:
            with open(trace[0]) as f:
                rows = [r for r in csv.DictReader(f) if _ours(r["Kernel_Name"])]
            rows.sort(key=lambda r: int(r["Start_Timestamp"]))
            by = _drop_warmup(rows, warmup, steps, lambda r: _short(r["Kernel_Name"]))
            lines.append(f"\n{wl}: kernel trace ({trace[0]})\n")
            lines.append("| kernel | launches | avg us | median us | min us | LDS B |")
            lines.append("|---|---|---|---|---|---|")
            for k, rs in sorted(by.items(), key=lambda kv: -sum(
                    int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in kv[1])):
                us = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in rs]
                r0 = rs[0]
                lines.append(f"| {k} | {len(us)} | {statistics.mean(us):.1f} | "
                             f"{statistics.median(us):.1f} | {min(us):.1f} | "
                             f"{r0['LDS_Block_Size']} |")
        for path in pmc:
            with open(path) as f:
                rows = list(csv.DictReader(f))
            # the 256 MiB device copy of --copy-calibration (the largest copy)
            calib = {}
            for r in rows:
                if "copyBuffer" in r["Kernel_Name"]:
                    calib[r["Counter_Name"]] = max(calib.get(r["Counter_Name"], 0.0),
                                                   float(r["Counter_Value"]))
            rows = [r for r in rows if _ours(r["Kernel_Name"])]
            disp = {}
            for r in rows:
                e = disp.setdefault((int(r["Dispatch_Id"]), _short(r["Kernel_Name"])), {})
                e[r["Counter_Name"]] = float(r["Counter_Value"])
                e["dispatch_us"] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            items = [(k[1], v) for k, v in sorted(disp.items())]
            by = _drop_warmup(items, warmup, steps, lambda it: it[0])
            names = sorted({c for _, v in items for c in v})
            lines.append(f"\n{wl}: counters ({path})"
                         + (f"; copy calibration {calib}" if calib else "") + "\n")
            lines.append("| kernel | dispatches | " + " | ".join(names) + " |")
            lines.append("|---|---|" + "---|" * len(names))
            # byte counters scaled by what they read for the copy of known size
            scale = {c: COPY_KIB / calib[c] * 1024 for c in ("FETCH_SIZE", "WRITE_SIZE")
                     if calib.get(c, 0) > COPY_KIB / 4}
            if scale:
                names += [f"{c} bytes" for c in scale]
                lines[-2] = "| kernel | dispatches | " + " | ".join(names) + " |"
                lines[-1] = "|---|---|" + "---|" * len(names)
            for k, its in sorted(by.items()):
                vals = [statistics.mean(v[c] for _, v in its if c in v)
                        for c in names if not c.endswith(" bytes")]
                vals += [statistics.mean(v[c] for _, v in its) * f for c, f in scale.items()]
                lines.append(f"| {k} | {len(its)} | " + " | ".join(f"{x:.6g}" for x in vals)
                             + " |")
                for c, f in scale.items():
                    traffic.setdefault(f"{k}@{wl.split('_')[-1].upper()}", {})[c] = round(
                        statistics.mean(v[c] for _, v in its) * f)
    print("\n".join(lines))
    if traffic_json:
        out = {k: {"bytes": v.get("FETCH_SIZE", 0) + v.get("WRITE_SIZE", 0),
                   "fetch_bytes": v.get("FETCH_SIZE"), "write_bytes": v.get("WRITE_SIZE")}
               for k, v in sorted(traffic.items())}
        with open(traffic_json, "w") as f:
            json.dump({"source": "rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE of bench.py "
                                 "--only runs, scaled by a 256 MiB device copy in the same run",
                       "kernels": out}, f, indent=1)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--only", choices=("c3", "c2", "c3doc", "c3kpm", "c3fp16", "c3fp32", "c5",
                                         "c5cap", "c4", *(f"tp4_{n}" for n in TP4_SHARES)))
    ap.add_argument("--rocprof-summary", nargs="+", metavar="DIR")
    ap.add_argument("--traffic-json", metavar="PATH",
                    help="with --rocprof-summary: write HBM bytes per launch per kernel")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run one 256 MiB device-to-device copy (a kernel of known "
                         "traffic, for scaling HBM byte counters)")
    args = ap.parse_args()
    if args.rocprof_summary:
        return rocprof_summary(args.rocprof_summary, args.warmup, args.steps, args.traffic_json)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the attention path "
              "shards over (batch x KV-head group) with no exchange, so each GPU runs this "
              "same single-GPU workload.", file=sys.stderr)
        return 2

    import torch

    dev = torch.device("cuda:0")
    if args.copy_calibration:
        src = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    wl = Workloads(dev)
    if args.only:
        return run_only(args, torch, wl)
    return run_full(args, torch, wl)


if __name__ == "__main__":
    sys.exit(main())
