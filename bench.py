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
only), the Llama-3-70B shape fwd+bwd (C5: B=1, S=16384, 64 query heads) and its
2048-token probability capture (C5-cap), the KV-cache decode configuration C4
in GB/s, and the reference's PyTorch path timed on the host CPU on a bounded
sample of the same workload.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "causal GQA attn TFLOP/s fwd+bwd (8B shape) + decode HBM GB/s, 1 MI355X"
PEAK_BF16_TFLOPS = 2516.6  # 256 CU x 2.4 GHz x 4096 flop/clk, dense
PEAK_HBM_GBPS = 8000.0

C3 = dict(B=4, S=4096, Hq=32, Hkv=8, D=128, theta=500000.0)
C4 = dict(B=32, Hq=32, Hkv=8, D=128, lo=1024, hi=8192, theta=500000.0)
C5 = dict(B=1, S=16384, Hq=64, Hkv=8, D=128, theta=500000.0, cap_tokens=2048)


def pairs(B, Hq, S):
    return B * Hq * S * (S + 1) // 2


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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run one 256 MiB device-to-device copy (a kernel of known "
                         "traffic, for scaling HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the attention path "
              "shards over (batch x KV-head group) with no exchange, so each GPU runs this "
              "same single-GPU workload.", file=sys.stderr)
        return 2

    import torch

    from kempnerforge_amd import _lib, ops
    from kempnerforge_amd.position import precompute_rope_frequencies

    dev = torch.device("cuda:0")
    bf16 = torch.bfloat16
    if args.copy_calibration:
        src = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    B, S, Hq, Hkv, D = (C3[k] for k in ("B", "S", "Hq", "Hkv", "D"))
    q = seeded((B, S, Hq, D), 0, bf16, dev).requires_grad_(True)
    k = seeded((B, S, Hkv, D), 1, bf16, dev).requires_grad_(True)
    v = seeded((B, S, Hkv, D), 2, bf16, dev).requires_grad_(True)
    do = seeded((B, S, Hq, D), 3, bf16, dev)
    cos, sin = precompute_rope_frequencies(D, S, C3["theta"])
    cos, sin = cos.to(dev), sin.to(dev)
    P = pairs(B, Hq, S)
    flops_step = 14.0 * D * P

    def step():
        out = ops.attention(q, k, v, cos, sin, causal=True)
        torch.autograd.grad(out, (q, k, v), do)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    secs = time.perf_counter() - t0
    ms_step = secs / args.steps * 1e3
    value = flops_step / (ms_step * 1e-3) / 1e12

    # per-kernel timing over the same number of steps (separate pass: the event
    # records would otherwise sit inside the timed region)
    with _lib.KernelTimer() as kt:
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
    kstats = {n: {"avg_us": t / c * 1e3, "launches": c} for n, (t, c) in kt.stats.items()}
    # algorithmic flops per launch of each MFMA kernel (the backward's 10*D*P is
    # 4*D*P of recomputed S and dP plus dV, dK -> dkdv kernel 8*D*P; dQ 2*D*P)
    algo = {"fwd_mfma": 4.0 * D * P, "bwd_dkdv": 8.0 * D * P, "bwd_dq": 2.0 * D * P,
            "bwd_dq_ds": 2.0 * D * P}
    dom = max(kstats, key=lambda n: kstats[n]["avg_us"] * kstats[n]["launches"])
    traffic = measured_traffic()
    roof = None
    if dom in algo:
        ach = algo[dom] / (kstats[dom]["avg_us"] * 1e-6) / 1e12
        roof = {"kernel": dom, "bound": "mfma", "achieved": round(ach, 1),
                "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(ach / PEAK_BF16_TFLOPS, 4),
                "traffic": traffic.get(f"{dom}@C3"),
                "avg_us": round(kstats[dom]["avg_us"], 1)}
    fwd_us = kstats.get("fwd_mfma", {}).get("avg_us")

    def wall(fn, warm, iters):
        for _ in range(warm):
            fn()
        torch.cuda.synchronize()
        t = time.perf_counter()
        for _ in range(iters):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t) / iters

    # C2: forward only (out + LSE) on the same tensors
    qn_, kn_, vn_ = q.detach(), k.detach(), v.detach()
    c2_s = wall(lambda: ops.fwd_raw(qn_, kn_, vn_, cos, sin, causal=True, k_rotated=False),
                args.warmup, args.steps)
    c2 = {"config": "C2 llama3-8b fwd B=4 S=4096 Hq=32 Hkv=8 D=128", "ms": round(c2_s * 1e3, 4),
          "TFLOP/s": round(4.0 * D * P / c2_s / 1e12, 1)}

    # C3 replayed from a HIP graph (the raw forward + backward calls captured
    # once): the same kernels without per-launch host overhead or autograd
    def raw_step():
        o, l = ops.fwd_raw(qn_, kn_, vn_, cos, sin, causal=True, k_rotated=False)
        return ops.bwd_raw(qn_, kn_, vn_, cos, sin, o, l, do, causal=True)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            raw_step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        raw_step()
    c3g_s = wall(graph.replay, args.warmup, args.steps)
    c3_graph = {"config": "C3 step as one HIP graph replay (fwd_raw + bwd_raw)",
                "ms": round(c3g_s * 1e3, 4), "TFLOP/s": round(flops_step / c3g_s / 1e12, 1)}
    del graph

    # C3-doc: the C3 step on packed sequences (documents of 64..2048 tokens, seeded);
    # flops count only same-document causal pairs, so the rate compares with C3's
    g = torch.Generator().manual_seed(7)
    doc_rows, doc_pairs = [], 0
    for _ in range(B):
        lens_, left = [], S
        while left:
            n = min(left, int(torch.randint(64, 2049, (1,), generator=g)))
            lens_.append(n)
            left -= n
        doc_pairs += Hq * sum(n * (n + 1) // 2 for n in lens_)
        doc_rows.append(torch.cat([torch.full((n,), i, dtype=torch.int32)
                                   for i, n in enumerate(lens_)]))
    doc_ids = torch.stack(doc_rows).to(dev)

    def step_doc():
        out = ops.attention(q, k, v, cos, sin, causal=True, doc_ids=doc_ids)
        torch.autograd.grad(out, (q, k, v), do)

    doc_s = wall(step_doc, args.warmup, args.steps)
    c3doc = {"config": "C3-doc C3 with packed documents of 64..2048 tokens (seed 7), "
                       f"{sum(int(r.max()) + 1 for r in doc_rows)} documents",
             "ms": round(doc_s * 1e3, 4),
             "TFLOP/s": round(14.0 * D * doc_pairs / doc_s / 1e12, 1),
             "visible_pair_frac": round(doc_pairs / P, 4),
             "speedup_vs_dense_causal": round(ms_step / (doc_s * 1e3), 2)}

    # C5: llama3-70b shape fwd+bwd, and C5-cap (probabilities of its first 2048 tokens)
    B5, S5, Hq5, Hkv5 = C5["B"], C5["S"], C5["Hq"], C5["Hkv"]
    q5 = seeded((B5, S5, Hq5, D), 0, bf16, dev).requires_grad_(True)
    k5 = seeded((B5, S5, Hkv5, D), 1, bf16, dev).requires_grad_(True)
    v5 = seeded((B5, S5, Hkv5, D), 2, bf16, dev).requires_grad_(True)
    do5 = seeded((B5, S5, Hq5, D), 3, bf16, dev)
    cos5, sin5 = precompute_rope_frequencies(D, S5, C5["theta"])
    cos5, sin5 = cos5.to(dev), sin5.to(dev)

    def step5():
        out5 = ops.attention(q5, k5, v5, cos5, sin5, causal=True)
        torch.autograd.grad(out5, (q5, k5, v5), do5)

    c5_s = wall(step5, 2, max(5, args.steps // 2))
    P5 = pairs(B5, Hq5, S5)
    c5 = {"config": "C5 llama3-70b fwd+bwd B=1 S=16384 Hq=64 Hkv=8 D=128",
          "ms": round(c5_s * 1e3, 3), "TFLOP/s": round(14.0 * D * P5 / c5_s / 1e12, 1),
          "frac_of_peak": round(14.0 * D * P5 / c5_s / 1e12 / PEAK_BF16_TFLOPS, 4)}
    Sc = C5["cap_tokens"]
    qc, kc_, vc_ = (t.detach()[:, :Sc].contiguous() for t in (q5, k5, v5))
    cap_s = wall(lambda: ops.capture_raw(qc, kc_, vc_, cos5[:Sc], sin5[:Sc], causal=True,
                                         k_rotated=False), 2, args.steps)
    cap_bytes = 4 * Hq5 * Sc * Sc + Sc * (Hq5 + 2 * Hkv5) * D * 2 + Sc * Hq5 * D * 2
    c5cap = {"config": "C5-cap first 2048 tokens of C5, P [1,64,2048,2048] fp32",
             "us": round(cap_s * 1e6, 1), "bytes": cap_bytes,
             "GB/s": round(cap_bytes / cap_s / 1e9, 1),
             "frac_of_hbm_peak": round(cap_bytes / cap_s / 1e9 / PEAK_HBM_GBPS, 4),
             "capture_kernel_traffic": traffic.get("capture_probs@C5-cap")}
    del q5, k5, v5, do5, qc, kc_, vc_

    # decode (C4)
    g = torch.Generator().manual_seed(4)
    Bd, Hqd, Hkvd, Dd = C4["B"], C4["Hq"], C4["Hkv"], C4["D"]
    lens = torch.randint(C4["lo"], C4["hi"] + 1, (Bd,), generator=g, dtype=torch.int32)
    Smax = C4["hi"] + 1
    qn = seeded((Bd, 1, Hqd, Dd), 0, bf16, dev)
    kn = seeded((Bd, 1, Hkvd, Dd), 1, bf16, dev)
    vn = seeded((Bd, 1, Hkvd, Dd), 2, bf16, dev)
    kc = torch.randn(Bd, Hkvd, Smax, Dd, device=dev, dtype=bf16)
    vc = torch.randn(Bd, Hkvd, Smax, Dd, device=dev, dtype=bf16)
    dcos, dsin = precompute_rope_frequencies(Dd, Smax, C4["theta"])
    dcos, dsin = dcos.to(dev), dsin.to(dev)
    lens_d = lens.to(dev)
    dec_bytes = sum(4 * (int(L) + 1) * Hkvd * Dd for L in lens) + 4 * Bd * Hqd * Dd \
        + 4 * Bd * Hkvd * Dd

    def dstep():
        ops.decode_raw(qn, kn, vn, kc, vc, lens_d, dcos, dsin, rope_row_offset=0, max_len=Smax)

    for _ in range(args.warmup):
        dstep()
    torch.cuda.synchronize()
    n_dec = max(args.steps, 50)
    t0 = time.perf_counter()
    for _ in range(n_dec):
        dstep()
    torch.cuda.synchronize()
    dec_us = (time.perf_counter() - t0) / n_dec * 1e6
    with _lib.KernelTimer() as kt2:
        for _ in range(n_dec):
            dstep()
        torch.cuda.synchronize()
    dstats = {n: {"avg_us": t / c * 1e3, "launches": c} for n, (t, c) in kt2.stats.items()}
    split_us = dstats.get("decode_split", {}).get("avg_us")

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import cpu_baseline

        sample = dict(B=1, S=C3["S"], Hq=8, Hkv=2, D=D)
        secs_cpu, reps, used = cpu_baseline.time_fwd_bwd(
            sample["B"], sample["S"], sample["Hq"], sample["Hkv"], sample["D"], C3["theta"],
            bf16, min_seconds=args.cpu_seconds)
        fl = 14.0 * D * pairs(sample["B"], sample["Hq"], sample["S"])
        cpu = {"value": round(fl / secs_cpu / 1e12, 4), "unit": "TFLOP/s",
               "cores": torch.get_num_threads(), "kind": "port",
               "sample": (f"reference PyTorch path (apply_rope -> repeat_interleave -> SDPA "
                          f"is_causal, autograd) fwd+bwd on CPU, {str(used).replace('torch.', '')},"
                          f" B=1 S={sample['S']} Hq=8 Hkv=2 D={D} (1/16 of C3), median of {reps}")}

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
        "c5": c5,
        "c5_cap": c5cap,
        "decode": {"config": "C4 B=32 Hq=32 Hkv=8 D=128 L~U[1024,8192] seed 4",
                   "bytes": dec_bytes, "us_per_step": round(dec_us, 1),
                   "GB/s": round(dec_bytes / (dec_us * 1e-6) / 1e9, 1),
                   "frac_of_hbm_peak": round(dec_bytes / (dec_us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4),
                   "kernels_us": {n: round(s["avg_us"], 1) for n, s in dstats.items()},
                   "split_kernel_GB/s": round(dec_bytes / (split_us * 1e-6) / 1e9, 1)
                   if split_us else None,
                   "split_kernel_traffic": traffic.get("decode_split@C4")},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
