"""Split-count selector refit for MI355X (256 CUs).

Counterpart of the reference's frozen 28-core selectors
(operators/mha/split_cost_model.py:13-44 and
operators/mha/general_split_cost_model.py:44-91): a linear latency model over
per-candidate features, with weights fitted on MI355X split scans and frozen
in split_cost_model.json. Pure Python, no device calls. Scores rank split
candidates; the smallest split within the selection tolerance of the best
predicted latency wins (less workspace and merge work), as in
general_split_cost_model.py:152-156.

Features of candidate s (layout and keys-per-round as the C planner uses:
Sq <= 32 -> 4 key-parallel waves over 32 query rows, 128 keys per round;
else 4 query-parallel waves over 128 rows, 64 keys per round):
  constant
  wave_rounds      ceil(tasks * s / CUs) x key rounds of the longest split
                   (critical path of one CU: its resident programs share it)
  waves            ceil(tasks * s / resident slots) (items one program runs)
  has_merge        s > 1
  partial_mbytes   s > 1: fp32 partial + LSE bytes written and read back, in MB
  merge_rows       s > 1: output rows merged x s / 1e3
The reference's ragged-batch feature (the longest request's split rounds
beyond the mean, general_split_cost_model.py:128-131) is not used: ragged
batches run length-balanced splits here (balanced_split_keys), and on the
calibration's ragged cases a fit that gives it weight chooses the same split
counts as one without it.
"""
from __future__ import annotations

import json
import math
import pathlib
from functools import lru_cache
from typing import Optional, Sequence

MODEL_PATH = pathlib.Path(__file__).with_name("split_cost_model.json")
SPLITS = (1, 2, 4, 8, 16, 32, 64, 128)
FEATURE_NAMES = ("constant", "wave_rounds", "waves", "has_merge", "partial_mbytes", "merge_rows")


def geometry(sq: int, dim: int = 128):
    """(layout index, rows per tile, keys per round) of the planner's automatic
    layout choice inside the model's scope (fgw_mha_plan: key layout for
    Sq <= 32, else query layout; eligible_config excludes the shapes where the
    planner takes the prefill layout)."""
    return (1, 32, 128) if sq <= 32 else (0, 128, 64)


def occupancy(device) -> tuple:
    """Resident workgroups per CU of the query, key and prefill kernels
    (fgw_mha_device_info.wg_per_cu)."""
    return tuple(device.wg_per_cu)


def features(batch, sq, heads, dim, lengths: Sequence[int], splits, num_cus, wg_per_cu):
    layout, rows, keys_round = geometry(sq, dim)
    tasks = batch * heads * math.ceil(sq / rows)
    slots = max(1, num_cus * max(1, wg_per_cu[layout]))
    items = tasks * splits
    waves = math.ceil(items / slots)
    rounds = [math.ceil(n / keys_round) for n in lengths]
    longest = math.ceil(max(rounds) / splits) if rounds else 0
    multi = int(splits > 1)
    parts_mb = multi * batch * heads * splits * sq * (dim + 1) * 4 * 2 / 1e6
    # Critical path in key rounds per CU: the programs resident on one CU
    # share its memory bandwidth and matrix cores, so a CU takes
    # ceil(items / CUs) items of `longest` rounds whatever its slot count.
    cu_rounds = math.ceil(items / num_cus) * longest
    return [1.0, cu_rounds * dim / 128.0, float(waves), float(multi), parts_mb,
            multi * batch * heads * sq * splits / 1e3]


@lru_cache(maxsize=2)
def load_model(path: str = str(MODEL_PATH)) -> Optional[dict]:
    """The frozen MI355X model, or None when no calibration has been committed."""
    p = pathlib.Path(path)
    if not p.exists():
        return None
    model = json.loads(p.read_text(encoding="utf-8"))
    if model.get("feature_names") != list(FEATURE_NAMES) or len(model["weights"]) != len(FEATURE_NAMES):
        raise ValueError("split cost model feature mismatch")
    if any(not math.isfinite(w) or w < 0 for w in model["weights"]):
        raise ValueError("split cost model requires finite nonnegative weights")
    return model


def planner_takes_prefill(batch, sq, heads, dim, num_cus, wg_per_cu, kv_tokens) -> bool:
    """True where fgw_mha_plan's automatic layout is the prefill layout (256-row
    tiles, fmha_api.hip auto_prefill): head-dim tile 64 or 128, Sq > 128, and
    its tiles alone fill the device, Sq >= 1024, or B * H * Sq * kv_tokens (the
    table capacity) reaches 2^24. geometry() does not describe that kernel, so
    the model is not used there."""
    dpad = 32
    while dpad < dim:
        dpad *= 2
    if dpad not in (64, 128) or sq <= 128:
        return False
    wg = max(1, wg_per_cu[2]) if wg_per_cu is not None else 1
    return (sq >= 1024 or batch * heads * math.ceil(sq / 256) >= num_cus * wg
            or batch * heads * sq * kv_tokens >= 1 << 24)


def single_stage_splits(batch, sq, heads, dim, capacity_tokens, splits, num_cus,
                        wg_per_cu_key_single) -> int:
    """fgw_mha_plan's single_stage_splits (fmha_api.hip) restated: a short
    decode plan (Sq <= 16, key layout, head-dim tile 128) of >= 16 even
    splits that gives each CU at most one work item moves to the single-stage
    key kernel with 4x the splits (Sq <= 4, >= 512 keys each), else 2x
    (>= 256 keys); returns that split count, or 0 to keep the plan."""
    dpad = 32
    while dpad < dim:
        dpad *= 2
    if (dpad != 128 or sq > 16 or splits < 16 or wg_per_cu_key_single < 2
            or batch * heads * splits > num_cus):
        return 0
    if sq <= 4 and 4 * splits <= SPLITS[-1] and capacity_tokens // (4 * splits) >= 512:
        return 4 * splits
    if 2 * splits <= SPLITS[-1] and capacity_tokens // (2 * splits) >= 256:
        return 2 * splits
    return 0


def planner_fill_preferred(batch, sq, heads, kv_tokens) -> bool:
    """Query-layout shapes (Sq > 32) of at least 2^22 query-key pairs
    (B * H * Sq * table capacity), where fgw_mha_plan's own fill rule (four key
    rounds per split there) measured closer to the best split count than the
    model: 1.009x against 1.041x on geometric mean over 40 multi-head D128
    shapes (the model's query-layout calibration is the single-head B1 H1
    grid)."""
    return sq > 32 and batch * heads * sq * kv_tokens >= 1 << 22


def eligible_config(batch, sq, heads, dim, kv_tokens, *, page_size, causal, full_kv_cache,
                    num_cus, lengths_known=False, wg_per_cu=None) -> bool:
    """Automatic policy guard: the calibrated scope of the frozen model (non-causal,
    the calibrated device, table capacity, query length and head dim, a layout the
    features describe); the cache lengths must be known on the host (a full cache,
    or ragged lengths passed in)."""
    model = load_model()
    if model is None:
        return False
    scope = model["scope"]
    return (not causal and num_cus == scope["num_cus"] and (full_kv_cache or lengths_known)
            and scope["min_kv"] <= kv_tokens <= scope["max_kv"]
            and scope["min_sq"] <= sq <= scope["max_sq"] and dim in scope["dims"]
            and not planner_takes_prefill(batch, sq, heads, dim, num_cus, wg_per_cu, kv_tokens)
            and not planner_fill_preferred(batch, sq, heads, kv_tokens))


def predict(batch, sq, heads, dim, lengths, splits, num_cus, wg_per_cu, model) -> float:
    x = features(batch, sq, heads, dim, lengths, splits, num_cus, wg_per_cu)
    return sum(w * v for w, v in zip(model["weights"], x))


MAX_BALANCED_BATCH = 1024  # FGW_MHA_MAX_BALANCED_BATCH
# split_keys values of balanced plans: 32 * 2^(j / 16), rounded up (steps of
# 4.4%), so that a decode step whose lengths grew by a few tokens usually
# reuses its plan. 32 .. 2^30.
_KEY_GRID = tuple(sorted({math.ceil(32 * 2 ** (j / 16)) for j in range(0, 16 * 25 + 1)}))


# Key rounds (the key layout's 4 waves x 32 keys) a balanced plan must take off
# the longest work item to pay for its per-call work: the lengths round trip
# and prefix sums before the first DMA, and more workspace slots (measured:
# one round saved is a wash, three save ~3.5 us at B4 H8 KV 32768).
KEYS_PER_ROUND = 128
MIN_ROUNDS_SAVED = 2


def balanced_split_keys(lengths, splits, capacity_tokens):
    """(workspace splits, split_keys) of a length-balanced plan with the work
    items of `splits` even splits per request, or None where it would not
    shorten the longest work item by MIN_ROUNDS_SAVED key rounds (uniform
    lengths, one split, a large batch, short caches).

    Request b then takes clamp(ceil(len_b / split_keys), 1, workspace splits)
    splits. split_keys is the smallest value of _KEY_GRID with
    sum_b max(1, ceil(len_b / split_keys)) <= B * splits; the workspace split
    count is the next power of two of the largest request's count, at most
    128 and at most the table's 32-token tiles (the planner's limits).
    """
    batch = len(lengths)
    if splits < 2 or batch < 2 or batch > MAX_BALANCED_BATCH or len(set(lengths)) < 2:
        return None
    longest = max(lengths)
    if longest <= 0:
        return None
    budget = batch * splits
    items = lambda k: sum(max(1, -(-n // k)) for n in lengths)  # noqa: E731
    keys = next((k for k in _KEY_GRID if items(k) <= budget), None)
    rounds = lambda n: -(-n // KEYS_PER_ROUND)  # noqa: E731
    if keys is None or rounds(-(-longest // splits)) - rounds(keys) < MIN_ROUNDS_SAVED:
        return None  # the longest work item would not get shorter enough
    cap = min(128, max(1, -(-capacity_tokens // 32)))
    need = -(-longest // keys)
    slots = 1
    while slots < need:
        slots *= 2
    slots = min(slots, cap)
    return (slots, keys) if slots >= 2 else None


def select_splits(batch, sq, heads, dim, capacity_tokens, lengths, device, model=None) -> int:
    """Split count with the lowest predicted latency (ties -> fewer splits)."""
    model = model or load_model()
    if model is None:
        raise ValueError("No MI355X split cost model calibration is available; use split_policy='legacy'")
    if len(lengths) != batch or any(n < 0 or n > capacity_tokens for n in lengths):
        raise ValueError("cache_lengths must match batch and page-table capacity")
    wg = occupancy(device)
    max_split = max(1, math.ceil(capacity_tokens / 32))
    costs = {s: predict(batch, sq, heads, dim, lengths, s, device.num_cus, wg, model)
             for s in SPLITS if s <= max_split}
    best = min(costs.values())
    limit = best + max(abs(best) * model["selection_tolerance"], model.get("absolute_margin_us", 0.0))
    return min(s for s, c in costs.items() if c <= limit)
