"""Benchmark of the paged MHA operator on one MI355X.

Headline workload (benchmark config 3): Q4096 / KV2048, B2 H8 D128 BF16,
page 128, non-causal, full cache, shuffled block table, inputs resident in
HBM. One step = one call of the launch callable (output allocation and every
kernel included, compile and H2D excluded). `value` and `ms_per_step` are the
reference's statistic (benchmarks/mha/bench_mha_mfu.py:221-240): the median
of single calls, each bracketed by its own pair of events on the current
stream and synchronised. Alongside, each figure also back-to-back (one event
pair around K calls). Companions: Q32768 at the same B/H/KV (config 3) and
Q1 decode at KV32768 (config 4) in us/call and HBM GB/s.

`roofline.kernel_us` is the kernel's average launch duration, from the
back-to-back region (one kernel per direct call; it includes the dispatch gap
between launches). `traffic` (HBM bytes per launch) comes from the rocprofv3
FETCH_SIZE / WRITE_SIZE summary under profiles/, scaled by the same counters
read for a plain copy of known size (`--copy-probe` is that copy).

Every workload is prepared (inputs, plans, one call each) before the timed
GPU work, which then runs back to back: the vendor GEMM reference, the
headline, Q32768, decode; the oracle checks and the CPU baselines follow.

The CPU baselines time the oracle's torch-fp32 attention (the reference's CPU
path restated) on this host's cores at 4 threads and at every CPU of the
process's affinity set.

Prints one JSON line. `python bench.py --gpus N` with N > 1 exits: the build
runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import re
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
# Kernel of a direct (single-split) call per layout, as rocprofv3 names it.
PREFILL_KERNELS = {"prefill": "prefill_kernel (direct, prefill layout)",
                   "query": "fwd_kernel (direct, query layout)",
                   "key": "fwd_kernel (direct, key layout)"}
METRIC = "MFU% + TFLOP/s (Q4096) and µs/call + HBM GB/s (Q1 decode), 1 MI355X"
TRAFFIC_SUMMARY = ROOT / "profiles" / "hbm_traffic_q4096_kv2048_and_q1_kv32768.md"
COPY_PROBE_BYTES = 1 << 30


def parse():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="CPU baseline's full thread count; 0 = every CPU of the process's "
                         "affinity set")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="wall-clock bound of the CPU baseline sample at full thread count")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a plain 1 GiB device copy (counter calibration) and exit")
    ap.add_argument("--suite", default="headline",
                    choices=("headline", "decode-scan", "decode-batch", "grid", "prefill",
                             "static", "static-scan", "power", "scans"),
                    help="headline: the one-line bench contract (default). decode-scan: "
                         "config 4 split scan; decode-batch: Q1 decode split scan over larger "
                         "batches and head counts (split cost model calibration); grid: "
                         "config 2 short-Q grid; "
                         "prefill: Q4096 and Q32768; static: B1H1 static-plan path against "
                         "the automatic split path; static-scan: the same over a Q x KV grid "
                         "(calibration of the static builders' fallback); power: MFMA rate "
                         "on N(0,1) against "
                         "constant inputs (library GEMM and the headline kernel); scans: the "
                         "first four scan suites")
    ap.add_argument("--out", default=None, help="scan suites: JSONL file for the records "
                    "(a markdown summary is written beside it)")
    ap.add_argument("--grid-splits", action="store_true",
                    help="grid suite: every admissible split count 1..128 besides split 1 and "
                         "auto (calibration data for the split cost model)")
    ap.add_argument("--scan-samples", type=int, default=21)
    ap.add_argument("--scan-warmup", type=int, default=5)
    return ap.parse_args()


def timed_region(call, steps, warmup):
    """Run `warmup` untimed calls, then exactly `steps` calls between two device
    synchronisations. Each call is bracketed by its own events on the current
    stream. Returns (total ms, per-call ms list)."""
    import torch
    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(2 * steps)]
    for i in range(steps):
        marks[2 * i].record()
        call()
        marks[2 * i + 1].record()
    torch.cuda.synchronize()
    total = marks[0].elapsed_time(marks[-1])
    per_call = [marks[2 * i].elapsed_time(marks[2 * i + 1]) for i in range(steps)]
    return total, per_call


def region_ms(call, steps, warmup):
    """Run `warmup` untimed calls, then exactly `steps` back-to-back calls between
    two device synchronisations, bracketed by one pair of events on the current
    stream (the launching stream). Returns the region's total ms. With one
    kernel per call, total / steps is the kernel's average launch duration plus
    the dispatch gap between launches, without per-launch event packets."""
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


def single_calls(call, samples):
    """Isolated single-call event durations (ms), the reference's statistic."""
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


def cpu_timed(inputs, page, threads, budget_s, min_reps=3):
    """Median wall-clock seconds of the oracle's chunked CPU attention, repeated
    until `budget_s` seconds have passed (at least `min_reps` runs)."""
    import torch
    from oracle import mha_oracle as O
    torch.set_num_threads(threads)
    times, out, spent = [], None, 0.0
    while len(times) < min_reps or spent < budget_s:
        t0 = time.perf_counter()
        out = O.chunked_reference(*inputs, page, False, 128)
        times.append(time.perf_counter() - t0)
        spent += times[-1]
    return statistics.median(times), len(times), out


def traffic_from_profile(kernel_key):
    """HBM bytes per launch recorded in the committed rocprofv3 summary (or None)."""
    if not TRAFFIC_SUMMARY.exists():
        return None
    pat = re.compile(rf"^traffic_bytes\[{re.escape(kernel_key)}\]:\s*(\d+)\s*$", re.M)
    m = pat.search(TRAFFIC_SUMMARY.read_text())
    return int(m.group(1)) if m else None


def copy_probe():
    import torch
    n = COPY_PROBE_BYTES // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": COPY_PROBE_BYTES, "launches": 5}), flush=True)
    return 0


# ---------------------------------------------------------------------------
# Scan suites (benchmark configs 2-4): one record per configuration, each
# checked against the oracle before it is timed, as the reference benches do
# (benchmarks/mha/bench_mha_mfu.py:207-220; bench_v7_split_scan.py:88-120;
# bench_split_breakdown.py:79-96 for the partial / merge components).
# ---------------------------------------------------------------------------
def _time_call(call, samples, warmup):
    """(median single-call us, back-to-back us per call) of `call`; the
    back-to-back figure comes from one event pair around all the calls."""
    back_ms = region_ms(call, samples, warmup)
    single = statistics.median(single_calls(call, samples)) * 1e3
    return single, back_ms / samples * 1e3


def _components(kern, dinputs, samples, warmup):
    """GPU us per launch of the partial kernel and of the merge on fixed
    partials, from graph replays (the components' Python call paths would
    otherwise bound small launches by host time)."""
    import torch
    parts, lse = kern.partial_kernel(*dinputs)
    torch.cuda.synchronize()
    p_us = graph_us(lambda: kern.partial_kernel(*dinputs)[0])
    m_us = graph_us(lambda: kern.merge_kernel(parts, lse))
    return p_us, m_us


def _checked(kern, dinputs, expected, dtype, label):
    import torch
    from oracle import mha_oracle as O
    got = kern(*dinputs)
    torch.cuda.synchronize()
    rtol, atol = O.TOLERANCES[dtype]
    torch.testing.assert_close(got.cpu(), expected, rtol=rtol, atol=atol,
                               msg=lambda m: f"{label}: {m}")


def suite_decode_scan(args, emit):
    """Config 4: B2 H8 D128 page 128, Q in {1, 16} x KV in {512 .. 32768}, FP16 and
    BF16, splits 1..128 and auto; plus the imbalanced B4 variant."""
    import torch
    from fgw_amd.operators.mha.current import build_kernel
    from oracle import mha_oracle as O
    dev = torch.device("cuda", 0)
    b, h, d, page = 2, 8, 128, 128
    for dtype, name in ((torch.bfloat16, "bf16"), (torch.float16, "fp16")):
        for sq in (1, 16):
            for kv in (512, 2048, 8192, 32768):
                host = O.bench_inputs(b, sq, h, d, page, kv, dtype)
                dinputs = [x.to(dev) for x in host]
                expected = O.chunked_reference(*host, page, False, 128)
                nbytes = O.algorithmic_bytes([kv] * b, sq, h, d, kv // page)
                for req in (None, 1, 2, 4, 8, 16, 32, 64, 128):
                    if req is not None and req > kv // 32:
                        continue
                    kern = build_kernel(b, sq, h, d, host[1].shape[0], kv // page, page, False,
                                        name.replace("bf16", "bfloat16").replace("fp16", "float16"),
                                        0, num_splits=req, full_kv_cache=True)
                    label = f"decode {name} q{sq} kv{kv} splits={req}"
                    _checked(kern, dinputs, expected, dtype, label)
                    call = lambda: kern(*dinputs)  # noqa: E731
                    single, back = _time_call(call, args.scan_samples, args.scan_warmup)
                    rec = {"suite": "decode-scan", "dtype": name, "batch": b, "heads": h,
                           "head_dim": d, "q_len": sq, "kv_len": kv, "requested_splits": req,
                           "num_splits": kern.num_splits, "grid": kern.compute_grid,
                           "split_policy": kern.split_policy, "us_per_call": single,
                           "us_back_to_back": back, "hbm_gbs": nbytes / (single * 1e-6) / 1e9}
                    if kern.execution_mode == "split_and_merge":
                        rec["partial_us"], rec["merge_us"] = _components(
                            kern, dinputs, args.scan_samples, args.scan_warmup)
                    emit(rec)
        # Imbalanced variant: B4, lengths uniform in [KV/8, KV] (seeded), width KV/page.
        for sq, kv in ((sq, kv) for sq in (1, 16) for kv in (512, 2048, 8192, 32768)):
            lengths = O.imbalanced_lengths(kv)
            q, k, v, table, _ = O.bench_inputs(4, sq, h, d, page, kv, dtype)
            host = (q, k, v, table, lengths)
            dinputs = [x.to(dev) for x in host]
            expected = O.chunked_reference(*host, page, False, 128)
            nbytes = O.algorithmic_bytes(lengths.tolist(), sq, h, d, kv // page)
            for req in (None, 1, 4, 16):
                if req is not None and req > kv // 32:
                    continue
                # The automatic split with the host-known lengths, as mha_paged_decode
                # plans it (cost model, length-balanced splits).
                kern = build_kernel(4, sq, h, d, k.shape[0], kv // page, page, False,
                                    "bfloat16" if name == "bf16" else "float16", 0,
                                    num_splits=req,
                                    cache_lengths=tuple(lengths.tolist()) if req is None else None)
                _checked(kern, dinputs, expected, dtype, f"imbalanced {name} q{sq} splits={req}")
                single, back = _time_call(lambda: kern(*dinputs), args.scan_samples,
                                          args.scan_warmup)
                emit({"suite": "decode-imbalanced", "dtype": name, "batch": 4, "heads": h,
                      "head_dim": d, "q_len": sq, "kv_len": kv, "lengths": lengths.tolist(),
                      "requested_splits": req, "num_splits": kern.num_splits,
                      "split_keys": kern.split_keys,
                      "grid": kern.compute_grid, "us_per_call": single, "us_back_to_back": back,
                      "hbm_gbs": nbytes / (single * 1e-6) / 1e9})


def suite_decode_batch(args, emit):
    """Q1 decode (D128 BF16, page 128, full cache) over larger batches and head
    counts than config 4 (32 to 512 (b, h) tasks, 134-537 MB of K/V), splits
    1..64 and auto: calibration data for the split cost model beyond B2 H8."""
    import torch
    from fgw_amd.operators.mha.current import build_kernel
    from oracle import mha_oracle as O
    dev = torch.device("cuda", 0)
    d, page = 128, 128
    for b, h, kv in ((4, 8, 32768), (8, 8, 16384), (8, 8, 4096), (4, 32, 8192), (16, 8, 8192),
                     (8, 32, 4096), (32, 8, 2048), (16, 32, 2048), (64, 8, 1024)):
        host = O.bench_inputs(b, 1, h, d, page, kv, torch.bfloat16)
        dinputs = [x.to(dev) for x in host]
        expected = O.chunked_reference(*host, page, False, 128)
        nbytes = O.algorithmic_bytes([kv] * b, 1, h, d, kv // page)
        for req in (None, 1, 2, 4, 8, 16, 32, 64):
            if req is not None and req > kv // 32:
                continue
            kern = build_kernel(b, 1, h, d, host[1].shape[0], kv // page, page, False, "bfloat16",
                                0, num_splits=req, full_kv_cache=True)
            _checked(kern, dinputs, expected, torch.bfloat16, f"decode-batch B{b} H{h} kv{kv} "
                                                              f"splits={req}")
            single, back = _time_call(lambda: kern(*dinputs), args.scan_samples,
                                      args.scan_warmup)
            emit({"suite": "decode-batch", "dtype": "bf16", "batch": b, "heads": h,
                  "head_dim": d, "q_len": 1, "kv_len": kv, "requested_splits": req,
                  "num_splits": kern.num_splits, "grid": kern.compute_grid,
                  "split_policy": kern.split_policy, "us_per_call": single,
                  "us_back_to_back": back, "hbm_gbs": nbytes / (single * 1e-6) / 1e9})
        del dinputs
        torch.cuda.empty_cache()


def suite_grid(args, emit):
    """Config 2: B1 H1 D128 BF16 page 128, Q in {1 .. 512} x KV in {128 .. 16384};
    each spec as one direct kernel (split 1) and with the automatic split, and with
    --grid-splits at every split count 2..128 the planner admits."""
    import torch
    from fgw_amd.operators.mha.current import build_kernel
    from oracle import mha_oracle as O
    dev = torch.device("cuda", 0)
    for sq in (1, 2, 4, 8, 16, 32, 64, 128, 256, 512):
        for kv in (128, 256, 512, 1024, 2048, 4096, 8192, 16384):
            host = O.bench_inputs(1, sq, 1, 128, 128, kv, torch.bfloat16)
            dinputs = [x.to(dev) for x in host]
            expected = O.chunked_reference(*host, 128, False, 128)
            flops = O.useful_flops([kv], sq, 1, 128, False)
            reqs = (1, None) + ((2, 4, 8, 16, 32, 64, 128) if args.grid_splits else ())
            for req in reqs:
                try:
                    kern = build_kernel(1, sq, 1, 128, host[1].shape[0], kv // 128, 128, False,
                                        "bfloat16", 0, num_splits=req, full_kv_cache=True)
                except ValueError:  # more splits than key blocks
                    continue
                _checked(kern, dinputs, expected, torch.bfloat16, f"grid q{sq} kv{kv} {req}")
                single, back = _time_call(lambda: kern(*dinputs), args.scan_samples,
                                          args.scan_warmup)
                emit({"suite": "grid", "dtype": "bf16", "q_len": sq, "kv_len": kv,
                      "requested_splits": req, "num_splits": kern.num_splits,
                      "layout": kern.layout, "grid": kern.compute_grid, "us_per_call": single,
                      "us_back_to_back": back, "tflops": flops / (single * 1e-6) / 1e12})


def suite_prefill(args, emit):
    """Config 3: B2 H8 D128 BF16 page 128, KV 2048, Q 4096 (headline) and Q 32768."""
    import torch
    from fgw_amd.operators.mha.current import build_kernel
    from oracle import mha_oracle as O
    dev = torch.device("cuda", 0)
    for sq in (4096, 32768):
        host = O.bench_inputs(2, sq, 8, 128, 128, 2048, torch.bfloat16)
        dinputs = [x.to(dev) for x in host]
        # Q32768: the first and last 256 query rows of both requests against the
        # oracle (non-causal rows are independent; the whole oracle would take
        # minutes of host time).
        rows = list(range(sq)) if sq <= 4096 else list(range(256)) + list(range(sq - 256, sq))
        expected = O.chunked_reference(host[0][:, rows], *host[1:], 128, False, 128)
        for layout in ("query", "prefill"):
            kern = build_kernel(2, sq, 8, 128, host[1].shape[0], 16, 128, False, "bfloat16", 0,
                                full_kv_cache=True, layout=layout)
            got = kern(*dinputs)
            torch.cuda.synchronize()
            rtol, atol = O.TOLERANCES[torch.bfloat16]
            torch.testing.assert_close(got[:, rows].cpu(), expected, rtol=rtol, atol=atol,
                                       msg=lambda m: f"prefill q{sq} {layout}: {m}")
            flops = O.useful_flops([2048] * 2, sq, 8, 128, False)
            single, back = _time_call(lambda: kern(*dinputs), args.scan_samples, args.scan_warmup)
            emit({"suite": "prefill", "dtype": "bf16", "q_len": sq, "kv_len": 2048,
                  "layout": kern.layout, "grid": kern.compute_grid, "us_per_call": single,
                  "us_back_to_back": back, "tflops_single": flops / (single * 1e-6) / 1e12,
                  "tflops_back_to_back": flops / (back * 1e-6) / 1e12,
                  "mfu_percent": 100.0 * flops / (back * 1e-6) / 1e12 / PEAK_BF16_TFLOPS})


def graph_us(call, calls=20, reps=5):
    """GPU time per call: `calls` calls captured in one HIP graph, replayed
    `reps` times (best replay). Host launch work is not in the figure. The
    first replay's output must equal the eager output bit for bit."""
    import torch
    eager = call()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = [call() for _ in range(calls)]
    best = float("inf")
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for r in range(reps):
        a.record()
        graph.replay()
        b.record()
        b.synchronize()
        best = min(best, a.elapsed_time(b) * 1e3 / calls)
        if r == 0 and not torch.equal(outs[-1], eager):
            raise AssertionError("graph replay output differs from the eager call")
    return best


STATIC_SHAPES = ((128, 512), (512, 2048), (1024, 4096), (3712, 4096), (4096, 2048), (8192, 8192),
                 (16384, 1024), (64, 32768), (5000, 2048), (2048, 16384))


STATIC_SCAN_Q = (64, 128, 256, 512, 1024, 2048, 3712, 4096, 5000, 8192, 16384)
STATIC_SCAN_KV = (512, 1024, 2048, 4096, 8192, 16384, 32768)


def suite_static(args, emit, shapes=None, suite="static"):
    """B1H1 D128 BF16 full page-128 KV: the static-plan path (choose_stream_plan,
    the reference's fused B1H1 entry, its own plan whatever the fallback would
    choose) against the automatic split path, GPU time per call from graph
    replays; both checked against the oracle (sampled rows from Q 4096)."""
    import torch
    from fgw_amd.operators.mha import static_schedule as S
    from fgw_amd.operators.mha.current import build_kernel
    from fgw_amd.operators.mha.kernels.mha_static_host_hip import build_fused_kernel
    from oracle import mha_oracle as O
    dev = torch.device("cuda", 0)
    for sq, kv in shapes or STATIC_SHAPES:
        host = O.bench_inputs(1, sq, 1, 128, 128, kv, torch.bfloat16)
        dinputs = [x.to(dev) for x in host]
        rows = list(range(sq)) if sq <= 4096 else list(range(256)) + list(range(sq - 256, sq))
        expected = O.chunked_reference(host[0][:, rows], *host[1:], 128, False, 128)
        auto = build_kernel(1, sq, 1, 128, host[1].shape[0], kv // 128, 128, False, "bfloat16", 0,
                            full_kv_cache=True)
        static = build_fused_kernel(sq, kv, host[1].shape[0], 0, fallback=False)
        for kern, name in ((auto, "auto"), (static, "static")):
            got = kern(*dinputs)
            torch.cuda.synchronize()
            rtol, atol = O.TOLERANCES[torch.bfloat16]
            torch.testing.assert_close(got[:, rows].cpu(), expected, rtol=rtol, atol=atol,
                                       msg=lambda m: f"{suite} {name} q{sq} kv{kv}: {m}")
        t_auto = graph_us(lambda: auto(*dinputs))
        t_static = graph_us(lambda: static(*dinputs))
        d = static.plan.describe()
        emit({"suite": suite, "q_len": sq, "kv_len": kv, "auto_us": t_auto,
              "auto_splits": auto.num_splits, "auto_layout": auto.layout,
              "auto_grid": auto.compute_grid, "auto_work": auto.compute_work,
              "static_us": t_static,
              "static_strategy": d["strategy"], "static_programs": d["programs"],
              "static_merged_tiles": d["merge_q_tiles"],
              "static_estimate_us": S.estimate_cost(static.plan)["total_us"],
              "speedup": t_auto / t_static})


def suite_static_scan(args, emit):
    """suite_static over STATIC_SCAN_Q x STATIC_SCAN_KV."""
    suite_static(args, emit, [(q, kv) for q in STATIC_SCAN_Q for kv in STATIC_SCAN_KV],
                 "static-scan")


def suite_power(args, emit):
    """Data dependence of the MFMA rate (power-limited shader clock): a library
    bf16 GEMM (torch.matmul, 8192^3) and the headline prefill kernel, each on
    N(0,1) inputs and on constant inputs (every element 1/8 in bf16), timed
    back to back with one event pair."""
    import torch
    from fgw_amd.operators.mha.current import build_kernel
    from oracle import mha_oracle as O
    dev = torch.device("cuda", 0)
    n = 8192
    gen = torch.Generator(device=dev).manual_seed(7)
    for data in ("normal", "constant"):
        if data == "normal":
            a = torch.randn(n, n, device=dev, generator=gen).to(torch.bfloat16)
            bm = torch.randn(n, n, device=dev, generator=gen).to(torch.bfloat16)
        else:
            a = torch.full((n, n), 0.125, device=dev, dtype=torch.bfloat16)
            bm = torch.full((n, n), 0.125, device=dev, dtype=torch.bfloat16)
        steps = 20
        ms = region_ms(lambda: torch.matmul(a, bm), steps, 5)
        emit({"suite": "power", "workload": "torch.matmul bf16 8192^3", "data": data,
              "us_per_call": ms / steps * 1e3, "tflops": 2 * n ** 3 / (ms / steps * 1e-3) / 1e12})
        del a, bm
    b, sq, h, d, page, kv = 2, 4096, 8, 128, 128, 2048
    host = O.bench_inputs(b, sq, h, d, page, kv, torch.bfloat16)
    kern = build_kernel(b, sq, h, d, host[1].shape[0], kv // page, page, False, "bfloat16", 0,
                        full_kv_cache=True)
    flops = O.useful_flops([kv] * b, sq, h, d, False)
    for data in ("normal", "constant"):
        dinputs = [x.to(dev) for x in host]
        if data == "constant":
            for x in dinputs[:3]:
                x.fill_(0.125)
        steps = 100
        ms = region_ms(lambda: kern(*dinputs), steps, 20)
        emit({"suite": "power", "workload": "prefill Q4096/KV2048 B2H8 D128 BF16", "data": data,
              "us_per_call": ms / steps * 1e3, "tflops": flops / (ms / steps * 1e-3) / 1e12})


def run_scans(args):
    import torch
    torch.cuda.set_device(0)
    suites = {"decode-scan": [suite_decode_scan], "decode-batch": [suite_decode_batch],
              "grid": [suite_grid],
              "prefill": [suite_prefill], "static": [suite_static],
              "static-scan": [suite_static_scan], "power": [suite_power],
              "scans": [suite_prefill, suite_decode_scan, suite_grid, suite_static]}[args.suite]
    out = open(args.out, "w") if args.out else None
    records = []

    def emit(rec):
        records.append(rec)
        line = json.dumps(rec)
        print(line, flush=True)
        if out:
            out.write(line + "\n")
            out.flush()

    from fgw_amd.operators.mha.kernels.mha_paged_decode_hip import _device_info
    info = _device_info(0)
    emit({"suite": "device", "name": torch.cuda.get_device_properties(0).gcnArchName,
          "num_cus": info.num_cus, "wg_per_cu": list(info.wg_per_cu),
          "wg_per_cu_key_single": info.wg_per_cu_key_single})
    for fn in suites:
        fn(args, emit)
    if out:
        out.close()
        pathlib.Path(args.out).with_suffix(".md").write_text(scan_markdown(records))
    return 0


def scan_markdown(records):
    """Summary tables of the scan records (the figures quoted in the docs)."""
    lines = []
    pw = [r for r in records if r["suite"] == "power"]
    if pw:
        lines += ["## MFMA rate against input data (back-to-back, one event pair)", "",
                  "| workload | data | us/call | TFLOP/s |", "|---|---|---|---|"]
        lines += [f"| {r['workload']} | {r['data']} | {r['us_per_call']:.1f} | {r['tflops']:.0f} |"
                  for r in pw]
        lines.append("")
    st = [r for r in records if r["suite"] == "static"]
    if st:
        lines += ["## Static plan vs automatic split (B1H1 D128 BF16, full page-128 KV, "
                  "GPU us/call from graph replays)", "",
                  "| Q | KV | auto us (splits) | static us | plan (programs, merged tiles) | "
                  "model us | speedup |", "|---|---|---|---|---|---|---|"]
        lines += [f"| {r['q_len']} | {r['kv_len']} | {r['auto_us']:.1f} (s{r['auto_splits']}) | "
                  f"{r['static_us']:.1f} | {r['static_strategy']} ({r['static_programs']}, "
                  f"{r['static_merged_tiles']}) | {r['static_estimate_us']:.1f} | "
                  f"{r['speedup']:.2f} |" for r in st]
        lines.append("")
    pre = [r for r in records if r["suite"] == "prefill"]
    if pre:
        lines += ["## Prefill (B2 H8 D128 BF16 page 128, KV 2048)", "",
                  "| Q | layout | grid | us/call (single) | us (back-to-back) | TFLOP/s | MFU % |",
                  "|---|---|---|---|---|---|---|"]
        lines += [f"| {r['q_len']} | {r['layout']} | {r['grid']} | {r['us_per_call']:.1f} | "
                  f"{r['us_back_to_back']:.1f} | {r['tflops_back_to_back']:.0f} | "
                  f"{r['mfu_percent']:.1f} |" for r in pre]
        lines.append("")
    dec = [r for r in records if r["suite"] == "decode-scan"]
    if dec:
        lines += ["## Decode split scan (B2 H8 D128 page 128)", "",
                  "| dtype | Q | KV | splits | us/call (single) | us (back-to-back) | partial us "
                  "(graph) | merge us (graph) | GB/s (single) |", "|---|---|---|---|---|---|---|---|---|"]
        for r in dec:
            sp = f"auto->{r['num_splits']}" if r["requested_splits"] is None else str(r["num_splits"])
            lines.append(f"| {r['dtype']} | {r['q_len']} | {r['kv_len']} | {sp} | "
                         f"{r['us_per_call']:.1f} | {r['us_back_to_back']:.1f} | "
                         f"{r.get('partial_us', float('nan')):.1f} | "
                         f"{r.get('merge_us', float('nan')):.1f} | {r['hbm_gbs']:.0f} |")
        lines.append("")
    bat = [r for r in records if r["suite"] == "decode-batch"]
    if bat:
        lines += ["## Decode over larger batches (Q1 D128 BF16 page 128, full cache)", "",
                  "| B | H | KV | splits | grid | us/call (single) | us (back-to-back) | "
                  "GB/s (single) |", "|---|---|---|---|---|---|---|---|"]
        for r in bat:
            sp = f"auto->{r['num_splits']}" if r["requested_splits"] is None else str(r["num_splits"])
            lines.append(f"| {r['batch']} | {r['heads']} | {r['kv_len']} | {sp} | {r['grid']} | "
                         f"{r['us_per_call']:.1f} | {r['us_back_to_back']:.1f} | "
                         f"{r['hbm_gbs']:.0f} |")
        lines.append("")
    imb = [r for r in records if r["suite"] == "decode-imbalanced"]
    if imb:
        lines += ["## Imbalanced decode (B4 H8 D128, lengths uniform in [KV/8, KV], KV 8192)", "",
                  "| dtype | Q | lengths | splits | us/call | GB/s |", "|---|---|---|---|---|---|"]
        for r in imb:
            sp = f"auto->{r['num_splits']}" if r["requested_splits"] is None else str(r["num_splits"])
            lines.append(f"| {r['dtype']} | {r['q_len']} | {r['lengths']} | {sp} | "
                         f"{r['us_per_call']:.1f} | {r['hbm_gbs']:.0f} |")
        lines.append("")
    grid = [r for r in records if r["suite"] == "grid"]
    if grid:
        kvs = sorted({r["kv_len"] for r in grid})
        for req, title in ((1, "split 1 (direct)"), (None, "automatic split")):
            lines += [f"## Short-Q grid, B1 H1 D128 BF16, us/call, {title}", "",
                      "| Q \\ KV | " + " | ".join(map(str, kvs)) + " |",
                      "|---" * (len(kvs) + 1) + "|"]
            for sq in sorted({r["q_len"] for r in grid}):
                row = {r["kv_len"]: r for r in grid if r["q_len"] == sq and r["requested_splits"] == req}
                cells = []
                for kv in kvs:
                    r = row.get(kv)
                    cells.append("" if r is None else (f"{r['us_per_call']:.1f}" + (
                        f" (s{r['num_splits']})" if req is None else "")))
                lines.append(f"| {sq} | " + " | ".join(cells) + " |")
            lines.append("")
    return "\n".join(lines) + "\n"


def cpu_model() -> str:
    try:
        for line in pathlib.Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def gpu_figures(call, steps, warmup, samples):
    """(single-call median ms, single-call list, back-to-back ms per call)."""
    import torch
    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    single = single_calls(call, samples)
    back = region_ms(call, steps, 0) / steps
    return statistics.median(single), single, back


def vendor_gemm_tflops(dev, n=8192, steps=10):
    """Same-box reference for the MFMA roofline: TFLOP/s of a library bf16 GEMM
    (torch.matmul, hipBLASLt) on N(0,1) inputs, back to back. The matrix cores'
    switching activity sets the power-limited clock, so random data reach less
    than the nominal dense peak even in the vendor GEMM."""
    import torch
    gen = torch.Generator(device=dev).manual_seed(7)
    a = torch.randn(n, n, device=dev, generator=gen).to(torch.bfloat16)
    b = torch.randn(n, n, device=dev, generator=gen).to(torch.bfloat16)
    ms = region_ms(lambda: torch.matmul(a, b), steps, 3)
    del a, b
    torch.cuda.empty_cache()
    return 2 * n ** 3 / (ms / steps * 1e-3) / 1e12


def prefill_record(kern, inputs, flops, qkv_bytes, steps, warmup, samples):
    """Figures of one direct prefill workload; the timed single calls are the step."""
    med, single, back = gpu_figures(lambda: kern(*inputs), steps, warmup, samples)
    kernel_ms = back  # direct mode: one kernel per call
    achieved = flops / (kernel_ms * 1e-3) / 1e12
    return {
        "us_per_call": med * 1e3, "us_per_call_min": min(single) * 1e3,
        "tflops": flops / (med * 1e-3) / 1e12, "mfu_percent": 100.0 * flops / (med * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
        "us_back_to_back": back * 1e3,
        "tflops_back_to_back": flops / (back * 1e-3) / 1e12,
        "grid": kern.compute_grid, "layout": kern.layout, "num_splits": kern.num_splits,
        "roofline": {"bound": "mfma", "kernel": PREFILL_KERNELS[kern.layout],
                     "achieved": achieved, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_BF16_TFLOPS, "kernel_us": kernel_ms * 1e3,
                     "kernel_us_source": "average launch duration: one event pair around the "
                                         "back-to-back region of the calls (one kernel each) on "
                                         "the launch stream / calls; includes the dispatch gap "
                                         "between launches",
                     "algorithmic_flops": flops, "algorithmic_bytes": qkv_bytes},
    }


def cpu_baselines(host, dhosts, page, flops, threads_full, budget_s):
    """The oracle's chunked torch-fp32 attention on the host cores: the headline
    prefill, config 1 and Q1 decode at KV 512 / 2048 / 8192 / 32768, each at 4
    threads (the reference harness cap) and at the full thread count."""
    import torch
    from oracle import mha_oracle as O
    out = {"cpu_model": cpu_model(), "cores_full": threads_full, "cores_cap": 4}
    pre = {}
    for threads, budget in ((threads_full, budget_s), (4, budget_s / 2)):
        sec, reps, expected = cpu_timed(host, page, threads, budget)
        pre[threads] = (sec, reps)
    out["prefill"] = {str(t): {"seconds_per_call": s_, "runs": r, "tflops": flops / s_ / 1e12}
                      for t, (s_, r) in pre.items()}
    dec = {}
    for label, (dh, nbytes) in dhosts.items():
        row = {}
        for threads in (4, threads_full):
            sec, reps, _ = cpu_timed(dh, page, threads, budget_s / 8, min_reps=3)
            row[str(threads)] = {"us_per_call": sec * 1e6, "runs": reps, "gbs": nbytes / sec / 1e9}
        dec[label] = row
    out["decode"] = dec
    torch.set_num_threads(threads_full)
    return out, expected


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU; --gpus {args.gpus} is not supported by this build "
              "(every GPU box here has one GPU; work items are independent and would shard "
              "by (batch, head) with no exchange)", file=sys.stderr)
        return 2
    import torch
    torch.cuda.set_device(0)
    if args.copy_probe:
        return copy_probe()
    if args.suite != "headline":
        return run_scans(args)
    from fgw_amd.operators.mha.current import build_kernel
    from oracle import mha_oracle as O

    dev = torch.device("cuda", 0)
    # The CPU baseline's full leg runs on every CPU this process may use (its
    # affinity set: on the GPU boxes a share of the host, whatever
    # os.cpu_count() reports for the whole machine); both counts are recorded.
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None
    cores = args.cpu_threads or affinity or os.cpu_count() or torch.get_num_threads()
    rtol, atol = O.TOLERANCES[torch.bfloat16]
    b, h, d, page, kv = 2, 8, 128, 128, 2048

    # Order. Every workload is set up first (host inputs, device copies, plans
    # and one call each, whose outputs the oracle checks at the end); then the
    # timed GPU work runs back to back, vendor GEMM reference first, and the
    # CPU baselines (tens of seconds of host work) last. A timed region that
    # starts after seconds of host-only work (input generation) finds the card
    # in its power controller's transient: per-call times of the headline rise
    # from ~69 to ~80 us over its first ~100 calls before they settle near
    # 67 us, and a Q32768 measured that way read 577-586 us single-call
    # against 512-514 us when it follows the headline directly.
    # ---- setup ------------------------------------------------------------
    sq = 4096
    host = O.bench_inputs(b, sq, h, d, page, kv, torch.bfloat16)
    inputs = [x.to(dev) for x in host]
    kern = build_kernel(b, sq, h, d, host[1].shape[0], kv // page, page, False, "bfloat16", 0,
                        full_kv_cache=True)
    flops = O.useful_flops([kv] * b, sq, h, d, False)
    got = kern(*inputs)
    big_sq = 32768
    bhost = O.bench_inputs(b, big_sq, h, d, page, kv, torch.bfloat16)
    binputs = [x.to(dev) for x in bhost]
    bkern = build_kernel(b, big_sq, h, d, bhost[1].shape[0], kv // page, page, False, "bfloat16",
                         0, full_kv_cache=True)
    bflops = O.useful_flops([kv] * b, big_sq, h, d, False)
    bgot = bkern(*binputs)
    db, dsq, dkv = 2, 1, 32768
    dhost = O.bench_inputs(db, dsq, h, d, page, dkv, torch.bfloat16)
    dinputs = [x.to(dev) for x in dhost]
    dkern = build_kernel(db, dsq, h, d, dhost[1].shape[0], dkv // page, page, False, "bfloat16", 0,
                         full_kv_cache=True)
    dgot = dkern(*dinputs)
    torch.cuda.synchronize()

    # ---- vendor GEMM reference (the MFMA rate of this box) -------------------
    gemm = vendor_gemm_tflops(dev)

    # ---- headline: Q4096 / KV2048 prefill (the step) ---------------------
    head = prefill_record(kern, inputs, flops, O.algorithmic_bytes([kv] * b, sq, h, d, kv // page),
                          args.steps, args.warmup, args.steps)
    head["roofline"]["traffic"] = traffic_from_profile("prefill_direct")
    head["roofline"]["traffic_source"] = str(TRAFFIC_SUMMARY.relative_to(ROOT))
    head["roofline"]["vendor_gemm_tflops"] = gemm
    head["roofline"]["frac_of_vendor_gemm"] = head["roofline"]["achieved"] / gemm
    head["roofline"]["vendor_gemm"] = ("torch.matmul bf16 8192^3 (hipBLASLt), N(0,1) inputs, "
                                       "back to back on the same box, measured right before "
                                       "the headline")

    # ---- companion: Q32768 / KV2048 prefill ------------------------------
    big_steps = max(10, args.steps // 3)
    big = prefill_record(bkern, binputs, bflops,
                         O.algorithmic_bytes([kv] * b, big_sq, h, d, kv // page),
                         big_steps, max(2, args.warmup // 5), big_steps)
    big["workload"] = "Q32768/KV2048 B2H8 D128 BF16 page128 non-causal full cache"
    big["roofline"]["frac_of_vendor_gemm"] = big["roofline"]["achieved"] / gemm
    big["roofline"]["traffic"] = traffic_from_profile("prefill_direct_q32768")
    big["roofline"]["traffic_source"] = str(TRAFFIC_SUMMARY.relative_to(ROOT))
    big["steps"] = big_steps

    # ---- decode: Q1 / KV32768 -------------------------------------------
    dbytes = O.algorithmic_bytes([dkv] * db, dsq, h, d, dkv // page)
    d_med, d_single, d_back = gpu_figures(lambda: dkern(*dinputs), args.steps, args.warmup,
                                          args.steps)
    decode = {"workload": "Q1/KV32768 B2H8 D128 BF16 page128", "us_per_call": d_med * 1e3,
              "us_per_call_min": min(d_single) * 1e3, "gbs": dbytes / (d_med * 1e-3) / 1e9,
              "us_back_to_back": d_back * 1e3, "bytes": dbytes, "num_splits": dkern.num_splits,
              "stages": dkern.stages,
              "split_policy": dkern.split_policy, "grid": dkern.compute_grid,
              "execution_mode": dkern.execution_mode,
              "roofline_call": {"bound": "hbm", "kernel": "whole call (every kernel, single-call "
                                "median)", "achieved": dbytes / (d_med * 1e-3) / 1e9,
                                "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                "frac": dbytes / (d_med * 1e-3) / 1e9 / PEAK_HBM_GBS}}
    if dkern.execution_mode == "split_and_merge":
        pcall = lambda: dkern.partial_kernel(*dinputs)  # noqa: E731
        p_ms = region_ms(pcall, args.steps, args.warmup) / args.steps
        p_achieved = dbytes / (p_ms * 1e-3) / 1e9
        stage_name = "single-stage" if dkern.stages == 1 else "double-stage"
        decode["roofline"] = {"bound": "hbm",
                              "kernel": f"fwd_kernel (partial, key layout, {stage_name}, "
                                        f"{dkern.num_splits} splits)",
                              "achieved": p_achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                              "frac": p_achieved / PEAK_HBM_GBS,
                              "traffic": traffic_from_profile("decode_partial"),
                              "traffic_source": str(TRAFFIC_SUMMARY.relative_to(ROOT)),
                              "kernel_us": p_ms * 1e3,
                              "kernel_us_source": "back-to-back region of partial-only calls / calls"}

    # ---- correctness of every workload, then the CPU baselines ----------
    dsmall = {}
    for dk in (512, 2048, 8192):
        dh = O.bench_inputs(db, dsq, h, d, page, dk, torch.bfloat16)
        dsmall[f"Q1/KV{dk} B2H8"] = (dh, O.algorithmic_bytes([dk] * db, dsq, h, d, dk // page))
    dsmall["Q1/KV32768 B2H8"] = (dhost, dbytes)
    c1 = O.bench_inputs(1, 1, 1, 128, page, 512, torch.bfloat16)
    dsmall["config1 B1H1 Q1/KV512"] = (c1, O.algorithmic_bytes([512], 1, 1, 128, 512 // page))
    cpu = None
    if not args.no_cpu_baseline:
        base, expected = cpu_baselines(host, dsmall, page, flops, cores, args.cpu_seconds)
        full = base["prefill"][str(cores)]
        cpu = {"value": full["tflops"], "unit": "TFLOP/s", "cores": cores, "kind": "port",
               "cpu_model": base["cpu_model"], "os_cpu_count": os.cpu_count(),
               "affinity_cpus": affinity,
               "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
               "sample": f"whole Q4096/KV2048 B2H8 D128 workload, oracle chunked_reference "
                         f"(torch fp32, chunk 128), median of {full['runs']} runs at "
                         f"torch.set_num_threads({cores}) (every CPU of the process's affinity "
                         f"set: {affinity}; os.cpu_count() {os.cpu_count()}); value_4_threads "
                         "at 4 threads (the reference harness cap); decode: Q1 at KV "
                         "512/2048/8192/32768 and config 1, each at 4 and full threads",
               "seconds_per_call": full["seconds_per_call"],
               "value_4_threads": base["prefill"]["4"]["tflops"],
               "decode": base["decode"]}
    else:
        expected = O.chunked_reference(*host, page, False, 128)
    torch.testing.assert_close(got.cpu(), expected, rtol=rtol, atol=atol)
    dexp = O.chunked_reference(*dhost, page, False, 128)
    torch.testing.assert_close(dgot.cpu(), dexp, rtol=rtol, atol=atol)
    # Q32768: every query row of both requests' first 256-row tile and last tile
    # against the oracle (the whole oracle would take minutes on the host).
    rows = list(range(256)) + list(range(big_sq - 256, big_sq))
    bexp = O.chunked_reference(bhost[0][:, rows], *bhost[1:], page, False, 128)
    torch.testing.assert_close(bgot[:, rows].cpu(), bexp, rtol=rtol, atol=atol)

    line = {
        "metric": METRIC, "value": head["tflops"], "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": head["us_per_call"] / 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "statistic": "median of single calls, each between its own event pair and synchronised "
                     "(bench_mha_mfu.py:221-240)",
        "config": {"workload": "Q4096/KV2048 B2H8 D128 BF16 page128 non-causal full cache",
                   "batch": b, "q_len": sq, "kv_len": kv, "heads": h, "head_dim": d,
                   "page_size": page, "num_splits": head["num_splits"], "grid": head["grid"],
                   "layout": head["layout"]},
        "mfu_percent": head["mfu_percent"],
        "us_per_call_min": head["us_per_call_min"],
        "us_back_to_back": head["us_back_to_back"],
        "tflops_back_to_back": head["tflops_back_to_back"],
        "roofline": head["roofline"],
        "cpu_baseline": cpu,
        "q32768": big,
        "decode": decode,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
