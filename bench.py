#!/usr/bin/env python3
"""Benchmark of the cached-KV in-context attention on one MI355X.

One step = one cached-KV ICL query of the 45k-train + 5k-test, 8-estimator workload: 12 sequential
per-block launches of the d=64 attention kernel, each over 8 estimators x 8 heads x 5,000 test
rows attending over 45,000 cached train rows (bf16 in, fp32 softmax/accumulation). The cache
([estimator, block, head, row, d]) and the queries are synthetic N(0,1) (seed 3) and resident in
HBM before the timed region. Prints one JSON line (see the driver contract).

Roofline: algorithmic FLOPs per launch = 4 * Tq * Tkv * d * heads * estimators (QK^T + PV),
achieved = that / average launch duration (HIP events on the launch stream). Traffic comes from
the committed rocprofv3 PMC summary when present. The CPU baseline times the fp32 CPU torch
restatement of the reference attention (oracle.attention.splash_sdpa_torch) on one (estimator,
block) slice of the same workload and scales it to a whole query.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tabiclv2-torchtpu-v5p-benchmark_amd"))

METRIC = "ms per cached-KV ICL query (45k+5k, 8 est.); attn TFLOP/s & % MFMA peak"
PEAK_BF16_TFLOPS = 2516.6
HBM_PEAK_GBS = 8000.0
EST, BLOCKS, HEADS, D = 8, 12, 8, 64
TRAIN, TEST = 45000, 5000
TRAFFIC_FILE = ROOT / "profiles" / "icl_fwd_c4_traffic.json"


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(seed: int = 3) -> dict:
    """fp32 CPU torch attention (oracle restatement of the reference path) on one (estimator,
    block) slice: 8 heads x 5,000 queries over 45,000 keys, scaled x96 to a whole query."""
    import torch

    from oracle.attention import splash_sdpa_torch

    threads = min(os.cpu_count() or 1, 64)
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, HEADS, TEST, D, generator=g)
    k = torch.randn(1, HEADS, TRAIN, D, generator=g)
    v = torch.randn(1, HEADS, TRAIN, D, generator=g)

    def run():
        for h in range(HEADS):
            for r0 in range(0, TEST, 1000):
                splash_sdpa_torch(q[:, h:h + 1, r0:r0 + 1000], k[:, h:h + 1], v[:, h:h + 1])

    t0 = time.perf_counter()
    run()  # warm-up (also sizes the sample)
    first = time.perf_counter() - t0
    reps = 1 if first > 8.0 else 3
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    per_slice = statistics.median(times)
    return {"value": round(per_slice * EST * BLOCKS * 1000.0, 1), "unit": "ms", "cores": threads,
            "kind": "port",
            "sample": f"1 estimator x 1 block (8 heads x {TEST} q x {TRAIN} keys, fp32 torch on {_cpu_model()}), "
                      f"median of {reps}, scaled x{EST * BLOCKS}"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the workload shards by estimator with no exchange; see DESIGN.md)", file=sys.stderr)
        return 2

    import torch

    import tabicl_mi355_icl as icl

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev).manual_seed(3)
    cache = icl.IclKVCache(EST, BLOCKS, HEADS, TRAIN, D, torch.bfloat16, dev)
    # fit-time build: per block, project-like K/V [est, head, rows, d] then append (timed apart)
    t_build = 0.0
    for b in range(BLOCKS):
        kb = torch.randn(EST, HEADS, TRAIN, D, generator=gen, device=dev, dtype=torch.bfloat16)
        vb = torch.randn(EST, HEADS, TRAIN, D, generator=gen, device=dev, dtype=torch.bfloat16)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        cache.append(b, kb, vb, row0=0)
        torch.cuda.synchronize()
        t_build += time.perf_counter() - t0
        del kb, vb
    q = torch.randn(EST, BLOCKS, HEADS, TEST, D, generator=gen, device=dev, dtype=torch.bfloat16)
    valid = torch.tensor([TRAIN], dtype=torch.int32, device=dev)
    out = torch.empty(EST, BLOCKS, HEADS, TEST, D, device=dev, dtype=torch.bfloat16)
    kv = [cache.block_kv(b) for b in range(BLOCKS)]

    def step(events=None):
        for b in range(BLOCKS):
            if events is not None:
                events[b][0].record()
            icl.ICL_FWD_OUT(q[:, b], kv[b][0], kv[b][1], valid, D ** -0.5, out[:, b])
            if events is not None:
                events[b][1].record()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(BLOCKS)]
          for _ in range(args.steps)]
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record()
    for s in range(args.steps):
        step(ev[s])
    t_end.record()
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)
    ms_per_step = total_ms / args.steps
    launch_ms = [a.elapsed_time(b) for row in ev for (a, b) in row]
    avg_launch_ms = sum(launch_ms) / len(launch_ms)

    flops_launch = 4.0 * TEST * TRAIN * D * HEADS * EST
    flops_step = flops_launch * BLOCKS
    tflops = flops_step / (ms_per_step * 1e-3) / 1e12
    kernel_tflops = flops_launch / (avg_launch_ms * 1e-3) / 1e12
    bytes_launch = 2.0 * (2 * TRAIN * D + 2 * TEST * D) * HEADS * EST  # K,V visible + Q + O (bf16)
    traffic = None
    if TRAFFIC_FILE.exists():
        try:
            traffic = json.loads(TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    rec = {
        "metric": METRIC,
        "value": round(ms_per_step, 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) cache and queries (seed 3), resident in HBM",
        "config": {"workload": "C4 cached-KV ICL query: 12 blocks x 8 est x 8 heads x 5000 q over 45000 cached "
                               "keys, d=64", "estimators": EST, "blocks": BLOCKS, "heads": HEADS, "head_dim": D,
                   "train_rows": TRAIN, "test_rows": TEST, "parallelism": "single GPU"},
        "attn_tflops": round(tflops, 1),
        "pct_mfma_peak": round(100.0 * tflops / PEAK_BF16_TFLOPS, 2),
        "avg_launch_ms": round(avg_launch_ms, 4),
        "cache_build_ms": round(t_build * 1000.0, 2),
        "cache_gib": round(cache.nbytes() / 2 ** 30, 2),
        "roofline": {"bound": "mfma", "achieved": round(kernel_tflops, 1), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(kernel_tflops / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                     "algorithmic_bytes": bytes_launch,
                     "hbm_gbs_algorithmic": round(bytes_launch / (avg_launch_ms * 1e-3) / 1e9, 1)},
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        rec["cpu_baseline"] = cpu_baseline()
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
