"""Fit the MI355X split-count model from bench.py scan records (offline, CPU only).

Counterpart of the reference's fitting tools (tools/mha/fit_split_cost_model.py,
tools/mha/fit_general_split_model.py): the calibration data are the JSONL
records of `bench.py --suite decode-scan|decode-batch|grid --out FILE` (one record per
(shape, split) with its measured single-call latency); the model is the
linear score of split_cost_model.features.

Objective (the reference's, restated): within each case (one shape scanned at
several split counts) the score differences between candidates should match
the latency differences, weighted by 1 / best latency of the case, with
nonnegative weights. Case-constant costs cancel, so the constant feature gets
weight 0 and scores rank candidates rather than predict absolute latency.
Solved here with scipy's nonnegative least squares on the stacked differences,
with the weight of the partial-bytes feature chosen on a grid by the in-sample
selection quality (least squares alone leaves it at zero; see fit()).

    python -m fgw_amd.operators.mha.fit_split_cost_model SCAN.jsonl [SCAN2.jsonl ...]

writes split_cost_model.json beside split_cost_model.py and prints the
in-sample evaluation (selected split's latency / best measured latency), the
same figures for the C planner's own fill rule (fgw_mha_plan with
num_splits = 0, read from the same records: the baseline the model must
beat), and a held-out check: weights fitted without the --holdout suites,
evaluated on them.
"""
from __future__ import annotations

import argparse
import collections
import hashlib
import json
import math
import pathlib
from typing import Dict, List

import numpy as np
from scipy.optimize import nnls

from fgw_amd.operators.mha import split_cost_model as M

SUITES = ("decode-scan", "decode-batch", "decode-imbalanced", "grid")
HOLDOUT = ("decode-batch", "decode-imbalanced")


class _Device:
    def __init__(self, num_cus, wg_per_cu, wg_per_cu_key_single=2):
        self.num_cus = num_cus
        self.wg_per_cu = tuple(wg_per_cu)
        self.wg_per_cu_key_single = wg_per_cu_key_single


def fill_rule_splits(case, device) -> int:
    """The C planner's automatic split count for a case (fgw_mha_plan with
    num_splits = 0, its automatic layout), on the double-stage key kernel the
    scans' explicit records ran on."""
    import ctypes

    from fgw_amd import _lib
    dev = _lib.DeviceInfo(device.num_cus, (ctypes.c_int32 * _lib.NUM_LAYOUTS)(*device.wg_per_cu),
                          1, device.wg_per_cu_key_single)
    width = -(-case["capacity"] // 128)
    shape = _lib.Shape(case["batch"], case["sq"], case["heads"], case["dim"],
                       case["batch"] * width * 128, width, 128, 0, _lib.DTYPE_BFLOAT16)
    stages = 2 if case["sq"] <= 32 and case["dim"] == 128 else 0
    return _lib.plan(shape, _lib.Request(0, -1, -1, 0, stages), dev).num_splits


def load_cases(paths) -> tuple:
    """Cases {key: {"shape": ..., "lat": {splits: us}}} and the scan device."""
    cases: Dict[tuple, dict] = collections.OrderedDict()
    device = None
    for path in paths:
        for line in pathlib.Path(path).read_text().splitlines():
            rec = json.loads(line)
            if rec["suite"] == "device":
                dev = (rec["num_cus"], tuple(rec["wg_per_cu"]), rec.get("wg_per_cu_key_single", 2))
                if device is not None and device != dev:
                    raise ValueError("scan files come from different devices")
                device = dev
                continue
            if rec["suite"] not in SUITES:
                continue
            batch = rec.get("batch", 1)
            heads = rec.get("heads", 1)
            dim = rec.get("head_dim", 128)
            lengths = tuple(rec.get("lengths") or [rec["kv_len"]] * batch)
            key = (rec["suite"], rec["dtype"], batch, heads, dim, rec["q_len"], rec["kv_len"],
                   lengths)
            case = cases.setdefault(key, {"suite": rec["suite"], "batch": batch, "heads": heads,
                                          "dim": dim, "sq": rec["q_len"],
                                          "capacity": rec["kv_len"], "lengths": lengths,
                                          "lat": {}, "auto": {}})
            # Explicit records measure even splits on the layout's default
            # kernel; the automatic record's plan may differ (length-balanced
            # splits, the single-stage kernel), so it stands for its split
            # count only where no explicit record of that count exists.
            lat = case["auto"] if rec.get("requested_splits") is None else case["lat"]
            s = rec["num_splits"]
            lat[s] = min(lat.get(s, math.inf), rec["us_per_call"])
    if device is None:
        raise ValueError("scan records carry no device record")
    for c in cases.values():
        for s, t in c.pop("auto").items():
            c["lat"].setdefault(s, t)
    return [c for c in cases.values() if len(c["lat"]) >= 2], _Device(*device)


def _differences(cases, device):
    rows, target = [], []
    for c in cases:
        best = min(c["lat"].values())
        base_s = min(c["lat"])  # smallest measured split as the reference candidate
        f0 = np.array(M.features(c["batch"], c["sq"], c["heads"], c["dim"], c["lengths"], base_s,
                                 device.num_cus, device.wg_per_cu))
        for s, t in c["lat"].items():
            if s == base_s:
                continue
            f = np.array(M.features(c["batch"], c["sq"], c["heads"], c["dim"], c["lengths"], s,
                                    device.num_cus, device.wg_per_cu))
            rows.append((f - f0) / best)
            target.append((t - c["lat"][base_s]) / best)
    return np.array(rows), np.array(target)


def _nnls(a, y) -> np.ndarray:
    scale = np.linalg.norm(a, axis=0)
    scale[scale == 0] = 1.0
    w, _ = nnls(a / scale, y)
    return w / scale


# Grid of the partial-bytes weight (us per MB of fp32 partials written and read
# back): 0 .. 0.3, i.e. down to ~6.7 TB/s for the round trip.
PARTIAL_MB_GRID = tuple(round(0.01 * i, 2) for i in range(31))


def fit(cases, device, tolerance: float = 0.03, margin: float = 0.5) -> List[float]:
    """Weights of split_cost_model.features. The partial-bytes weight is taken
    from PARTIAL_MB_GRID by the in-sample selection quality (geomean, then worst
    selected/best ratio, then residual); given it, the others are the
    nonnegative least squares solution. Least squares alone leaves that
    weight at 0: the few long-query cases where partial traffic decides the
    choice carry little of the squared error."""
    a, y = _differences(cases, device)
    col = M.FEATURE_NAMES.index("partial_mbytes")
    rest = np.delete(a, col, axis=1)
    best_key, best_w = None, None
    for pm in PARTIAL_MB_GRID:
        w = np.insert(_nnls(rest, y - a[:, col] * pm), col, pm)
        rep = evaluate(w.tolist(), cases, device, tolerance, margin)
        residual = float(np.linalg.norm(a @ w - y))
        key = (round(rep["geomean_relative_to_best"], 6), round(rep["max_relative_to_best"], 6),
               residual)
        if best_key is None or key < best_key:
            best_key, best_w = key, w
    return best_w.tolist()


def evaluate(weights, cases, device, tolerance, margin) -> dict:
    """Selection quality of the model over `cases` (chosen split's measured
    latency / the case's best), and of the C fill rule over the cases whose
    fill-rule split count was measured (fill_rule_unmeasured counts the
    others; the model's figures on exactly those cases are model_on_fill_cases)."""
    model = {"weights": weights, "selection_tolerance": tolerance, "absolute_margin_us": margin}
    ratios, fill, model_on_fill, rows = [], [], [], []
    unmeasured = 0
    for c in cases:
        preds = {s: M.predict(c["batch"], c["sq"], c["heads"], c["dim"], c["lengths"], s,
                              device.num_cus, device.wg_per_cu, model) for s in c["lat"]}
        lo = min(preds.values())
        limit = lo + max(abs(lo) * tolerance, margin)
        chosen = min(s for s, v in preds.items() if v <= limit)
        best_s = min(c["lat"], key=c["lat"].get)
        r = c["lat"][chosen] / c["lat"][best_s]
        ratios.append(r)
        fs = fill_rule_splits(c, device)
        if fs in c["lat"]:
            fill.append(c["lat"][fs] / c["lat"][best_s])
            model_on_fill.append(r)
        else:
            unmeasured += 1
        rows.append({"suite": c["suite"], "batch": c["batch"], "heads": c["heads"], "sq": c["sq"],
                     "kv": c["capacity"], "chosen": chosen, "fill_rule": fs, "best": best_s,
                     "relative_to_best": round(r, 4)})
    geo = lambda xs: math.exp(sum(map(math.log, xs)) / len(xs)) if xs else None  # noqa: E731
    return {"cases": len(ratios), "within_5pct": sum(r <= 1.05 for r in ratios),
            "geomean_relative_to_best": geo(ratios), "max_relative_to_best": max(ratios),
            "fill_rule_cases": len(fill), "fill_rule_unmeasured": unmeasured,
            "fill_rule_geomean_relative_to_best": geo(fill),
            "fill_rule_max_relative_to_best": max(fill) if fill else None,
            "model_on_fill_cases_geomean": geo(model_on_fill),
            "model_on_fill_cases_max": max(model_on_fill) if model_on_fill else None,
            "fill_rule_within_5pct": sum(r <= 1.05 for r in fill), "rows": rows}


def held_out(cases, device, suites, tolerance, margin) -> dict:
    """Weights fitted on the cases outside `suites`, evaluated on those inside."""
    train = [c for c in cases if c["suite"] not in suites]
    test = [c for c in cases if c["suite"] in suites]
    weights = fit(train, device, tolerance, margin)
    rep = evaluate(weights, test, device, tolerance, margin)
    return {"train_suites": sorted({c["suite"] for c in train}), "test_suites": sorted(suites),
            "train_cases": len(train), "weights": weights,
            **{k: v for k, v in rep.items() if k != "rows"}}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("scans", nargs="+", help="bench.py scan JSONL files")
    ap.add_argument("--output", default=str(M.MODEL_PATH))
    ap.add_argument("--tolerance", type=float, default=0.03,
                    help="relative score tolerance: the smallest split within it wins")
    ap.add_argument("--margin-us", type=float, default=0.5)
    ap.add_argument("--holdout", nargs="*", default=list(HOLDOUT),
                    help="suites left out of the held-out fit and evaluated on it")
    args = ap.parse_args(argv)
    cases, device = load_cases(args.scans)
    weights = fit(cases, device, args.tolerance, args.margin_us)
    report = evaluate(weights, cases, device, args.tolerance, args.margin_us)
    holdout = held_out(cases, device, tuple(args.holdout), args.tolerance, args.margin_us)
    lens = [c["capacity"] for c in cases]
    sqs = [c["sq"] for c in cases]
    model = {
        "version": 1,
        "device": {"num_cus": device.num_cus, "wg_per_cu": list(device.wg_per_cu)},
        "feature_names": list(M.FEATURE_NAMES),
        "weights": weights,
        "selection_tolerance": args.tolerance,
        "absolute_margin_us": args.margin_us,
        "scope": {"num_cus": device.num_cus, "min_kv": min(lens), "max_kv": max(lens),
                  "min_sq": min(sqs), "max_sq": max(sqs),
                  "dims": sorted({c["dim"] for c in cases})},
        "training_cases": report["cases"],
        "in_sample": {k: v for k, v in report.items() if k != "rows"},
        "held_out": holdout,
        "sources": [{"name": pathlib.Path(p).name,
                     "sha256": hashlib.sha256(pathlib.Path(p).read_bytes()).hexdigest()}
                    for p in args.scans],
        "fit": "nonnegative least squares on within-case latency differences against the "
               "smallest scanned split, weighted by 1 / best latency of the case; the "
               "partial-bytes weight searched on a grid by in-sample selection quality",
    }
    pathlib.Path(args.output).write_text(json.dumps(model, indent=2) + "\n")
    print(json.dumps({k: v for k, v in model.items() if k not in ("sources",)}, indent=2))
    worst = sorted(report["rows"], key=lambda r: -r["relative_to_best"])[:8]
    print("worst cases:", json.dumps(worst))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
