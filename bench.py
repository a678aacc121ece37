"""Benchmark of the paged MHA operator on one MI355X.

Headline workload: Q4096 / KV2048, B2 H8 D128 BF16,
page 128, non-causal, full cache, shuffled block table, inputs resident in
HBM. One step = one call of the launch callable (output allocation and every
kernel included, compile and H2D excluded), as the reference times it
(benchmarks/mha/bench_mha_mfu.py:221-247). Alongside: Q1 decode at KV32768
in us/call and HBM GB/s.

Prints one JSON line. `python bench.py --gpus N` with N > 1 exits: the build
runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
METRIC = "MFU% + TFLOP/s (Q4096) and µs/call + HBM GB/s (Q1 decode), 1 MI355X"


def parse():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--samples", type=int, default=51, help="single-call event samples per workload")
    ap.add_argument("--cpu-threads", type=int, default=0, help="0 = all host cores")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    return ap.parse_args()


def timed_steps(call, steps, warmup):
    """Total ms of exactly `steps` calls, bracketed by device synchronisation."""
    import torch
    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        call()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end)


def call_samples(call, samples):
    """Per-call event durations (ms) on the launching stream, reference style."""
    import torch
    out = []
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(samples):
        start.record()
        call()
        end.record()
        end.synchronize()
        out.append(start.elapsed_time(end))
    return out


def cpu_reference_timed(inputs, page, threads, reps):
    import torch
    from oracle import mha_oracle as O
    torch.set_num_threads(threads)
    times, out = [], None
    for _ in range(reps):
        t0 = time.perf_counter()
        out = O.chunked_reference(*inputs, page, False, 128)
        times.append(time.perf_counter() - t0)
    return statistics.median(times), out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU; --gpus {args.gpus} is not supported by this build "
              "(paged MHA work items are independent; see DESIGN.md for how it would shard)",
              file=sys.stderr)
        return 2
    import torch
    from fgw_amd.operators.mha.current import build_kernel
    from oracle import mha_oracle as O

    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    cores = args.cpu_threads or os.cpu_count() or 1

    # ---- headline: Q4096 / KV2048 prefill ------------------------------
    b, sq, h, d, page, kv = 2, 4096, 8, 128, 128, 2048
    host = O.bench_inputs(b, sq, h, d, page, kv, torch.bfloat16)
    inputs = [x.to(dev) for x in host]
    kern = build_kernel(b, sq, h, d, host[1].shape[0], kv // page, page, False, "bfloat16", 0,
                        full_kv_cache=True)
    flops = O.useful_flops([kv] * b, sq, h, d, False)
    got = kern(*inputs)
    torch.cuda.synchronize()

    cpu = None
    expected = None
    if not args.no_cpu_baseline:
        cpu_s, expected = cpu_reference_timed(host, page, cores, 3)
        cpu = {"value": flops / cpu_s / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
               "sample": f"full Q4096/KV2048 B2H8 D128 workload, oracle chunked_reference "
                         f"(torch fp32, chunk 128) at torch.set_num_threads({cores}), median of 3",
               "seconds_per_call": cpu_s}
        # Four threads: the reference harness's CPU cap (resource_guard.py:14-20).
        cpu4_s, _ = cpu_reference_timed(host, page, 4, 1)
        cpu["value_4_threads"] = flops / cpu4_s / 1e12
    else:
        expected = O.chunked_reference(*host, page, False, 128)
    rtol, atol = O.TOLERANCES[torch.bfloat16]
    torch.testing.assert_close(got.cpu(), expected, rtol=rtol, atol=atol)

    call = lambda: kern(*inputs)  # noqa: E731
    total_ms = timed_steps(call, args.steps, args.warmup)
    ms = total_ms / args.steps
    samples = call_samples(call, args.samples)
    kernel_ms = statistics.mean(samples)
    tflops = flops / (ms * 1e-3) / 1e12
    achieved = flops / (kernel_ms * 1e-3) / 1e12

    # ---- decode: Q1 / KV32768 -------------------------------------------
    db, dsq, dkv = 2, 1, 32768
    dhost = O.bench_inputs(db, dsq, h, d, page, dkv, torch.bfloat16)
    dinputs = [x.to(dev) for x in dhost]
    dkern = build_kernel(db, dsq, h, d, dhost[1].shape[0], dkv // page, page, False, "bfloat16", 0,
                         full_kv_cache=True)
    dgot = dkern(*dinputs)
    torch.cuda.synchronize()
    dexp = O.chunked_reference(*dhost, page, False, 128)
    torch.testing.assert_close(dgot.cpu(), dexp, rtol=rtol, atol=atol)
    dbytes = O.algorithmic_bytes([dkv] * db, dsq, h, d, dkv // page)
    dcall = lambda: dkern(*dinputs)  # noqa: E731
    timed_steps(dcall, 20, 20)
    dsamples = call_samples(dcall, args.samples)
    d_us = statistics.median(dsamples) * 1e3
    decode = {"workload": "Q1/KV32768 B2H8 D128 BF16 page128", "us_per_call": d_us,
              "gbs": dbytes / (d_us * 1e-6) / 1e9, "bytes": dbytes,
              "num_splits": dkern.num_splits, "grid": dkern.compute_grid}
    if dkern.execution_mode == "split_and_merge":
        pcall = lambda: dkern.partial_kernel(*dinputs)  # noqa: E731
        timed_steps(pcall, 20, 20)
        p_ms = statistics.mean(call_samples(pcall, args.samples))
        p_achieved = dbytes / (p_ms * 1e-3) / 1e9
        decode["roofline"] = {"bound": "hbm", "kernel": "fwd_kernel (partial)",
                              "achieved": p_achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                              "frac": p_achieved / PEAK_HBM_GBS, "traffic": None}
    if not args.no_cpu_baseline:
        t0 = time.perf_counter()
        O.chunked_reference(*dhost, page, False, 128)
        c_s = time.perf_counter() - t0
        decode["cpu_baseline"] = {"value": dbytes / c_s / 1e9, "unit": "GB/s", "cores": cores,
                                  "kind": "port", "sample": "full Q1/KV32768 workload, 1 run"}

    line = {
        "metric": METRIC, "value": tflops, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "Q4096/KV2048 B2H8 D128 BF16 page128 non-causal full cache",
                   "batch": b, "q_len": sq, "kv_len": kv, "heads": h, "head_dim": d,
                   "page_size": page, "num_splits": kern.num_splits, "grid": kern.compute_grid,
                   "layout": kern.layout},
        "mfu_percent": 100.0 * tflops / PEAK_BF16_TFLOPS,
        "median_call_us": statistics.median(samples) * 1e3,
        "roofline": {"bound": "mfma", "kernel": "fwd_kernel (direct)", "achieved": achieved,
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": achieved / PEAK_BF16_TFLOPS,
                     "traffic": None},
        "cpu_baseline": cpu,
        "decode": decode,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
