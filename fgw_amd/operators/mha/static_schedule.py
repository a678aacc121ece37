"""Host static KV-block schedules for the B1H1 long-query path.

Same plans as the reference planner (operators/mha/static_schedule.py:47-262):
the (128-row Q tile, 128-key KV block) units of one head are assigned to
programs as contiguous segments (Q tile, first KV block, KV blocks, slot);
a Q tile cut across programs gets one partial slot per piece and a merge
group (Q tile, first slot, slots); slot -1 marks a whole tile written
directly. Plans are pure host data with no device timing or search.

Policies, as in the reference:
  make_plan         balanced contiguous ranges of units over `cores` programs
  make_q_plan       whole consecutive Q tiles per program, never a partial
  make_tail_plan    whole tiles in full waves, only the final wave's tiles split
  make_stream_plan  whole-tile-first assignment against a remaining-work target
  choose_plan / choose_stream_plan  the cheapest by estimate_cost

MI355X differences: a program is one resident workgroup of the query-layout
kernel, so `cores` ranges over 1..MAX_CORES (the reference: 1..28 Cube
cores); the choosers scan the program counts of CANDIDATE_CORES (every count
up to 32, then multiples of 16) instead of every count; estimate_cost has the
terms of this build's kernels (below), fitted on MI355X, not the Ascend ones.
"""
from __future__ import annotations

import json
import math
import pathlib
from dataclasses import dataclass
from functools import lru_cache

BLOCK = 128          # rows per Q tile and keys per KV block
MAX_CORES = 1024     # programs a plan may use
NUM_CUS = 256        # MI355X compute units
DEFAULT_CORES = 512  # 256 CUs x 2 resident query-layout workgroups
CANDIDATE_CORES = tuple(range(1, 33)) + tuple(range(48, MAX_CORES + 1, 16))

# Stage costs in microseconds (B1H1, BF16, D128), fitted by nonnegative least
# squares to the GPU time of 50 plans (10 shapes Q 64..16384 x KV 512..32768,
# five policies; median error 3%, worst 28%):
#   local = max over programs (blocks * b + segments * segment_us), with
#           b = block_us while every program has a CU to itself and
#           shared_block_us once programs outnumber the CUs (two per CU)
#   merge = merge_launch_us + max_parts * parts_us + groups * merge_tile_us
# (a merge thread walks its group's slots in turn; groups run in parallel).
# The per-segment cost was not separable from these plans (one or two
# segments per program) and is left at zero. A constant of ~7.4 us common to
# every plan is left out, as in the reference model.
COST_MODEL = dict(block_us=3.19, shared_block_us=5.38, segment_us=0.0, merge_launch_us=5.74,
                  parts_us=0.119, merge_tile_us=0.126)


@dataclass(frozen=True)
class Plan:
    q: int
    kv: int
    programs: tuple      # per program: ((tile, first block, blocks, slot), ...)
    merges: tuple        # ((tile, first slot, slots), ...)
    partial_count: int
    strategy: str = "balanced"

    @property
    def max_segments(self):
        return max(len(p) for p in self.programs)

    @property
    def max_parts(self):
        return max((n for _, _, n in self.merges), default=0)

    def describe(self):
        loads = [sum(seg[2] for seg in p) for p in self.programs]
        tiles = -(-self.q // BLOCK)
        return dict(strategy=self.strategy, Q=self.q, KV=self.kv, programs=len(loads),
                    q_tiles=tiles, min_kv_blocks=min(loads), max_kv_blocks=max(loads),
                    segments=sum(len(p) for p in self.programs), max_segments=self.max_segments,
                    partial_count=self.partial_count, merge_q_tiles=len(self.merges),
                    direct_q_tiles=tiles - len(self.merges), max_parts=self.max_parts,
                    partial_bytes=self.partial_count * BLOCK * 128 * 4,
                    lse_bytes=self.partial_count * BLOCK * 4)


def _check_args(q, kv, cores):
    if type(q) is not int or type(kv) is not int or q <= 0 or kv <= 0 or kv % BLOCK:
        raise ValueError("positive integer Q and positive 128-aligned KV required")
    if type(cores) is not int or not 1 <= cores <= MAX_CORES:
        raise ValueError(f"cores must be 1..{MAX_CORES}")
    tiles, blocks = -(-q // BLOCK), kv // BLOCK
    if tiles * blocks > 2**31 - 1:
        raise ValueError("int32 scheduling range exceeded")
    return tiles, blocks


def _with_slots(q, kv, programs, strategy):
    """Give every piece of a tile owned by more than one program a slot, in
    tile order and, within a tile, in the order the programs list them."""
    pieces = {}
    for pid, segs in enumerate(programs):
        for idx, seg in enumerate(segs):
            pieces.setdefault(seg[0], []).append((pid, idx))
    merges, slot = [], 0
    out = [list(map(list, segs)) for segs in programs]
    for tile in sorted(pieces):
        owners = pieces[tile]
        if len(owners) < 2:
            continue
        merges.append((tile, slot, len(owners)))
        for pid, idx in owners:
            out[pid][idx][3] = slot
            slot += 1
    plan = Plan(q, kv, tuple(tuple(tuple(seg) for seg in segs) for segs in out),
                tuple(merges), slot, strategy)
    validate_plan(plan)
    return plan


@lru_cache(maxsize=128)
def make_plan(q, kv, cores=DEFAULT_CORES):
    """Balanced plan: program p takes units [p T / P + min(p, T % P), ...) of
    the tile-major unit order, cut into per-tile segments."""
    tiles, blocks = _check_args(q, kv, cores)
    total = tiles * blocks
    n = min(cores, total)
    base, extra = divmod(total, n)
    programs = []
    for pid in range(n):
        lo = pid * base + min(pid, extra)
        hi = lo + base + (1 if pid < extra else 0)
        segs = []
        while lo < hi:
            tile, first = divmod(lo, blocks)
            end = min(hi, (tile + 1) * blocks)
            segs.append((tile, first, end - lo, -1))
            lo = end
        programs.append(segs)
    return _with_slots(q, kv, programs, "balanced")


@lru_cache(maxsize=128)
def make_q_plan(q, kv, cores=DEFAULT_CORES):
    """Whole consecutive Q tiles per program; no partial state."""
    tiles, blocks = _check_args(q, kv, cores)
    n = min(cores, tiles)
    base, extra = divmod(tiles, n)
    programs, tile = [], 0
    for pid in range(n):
        count = base + (1 if pid < extra else 0)
        programs.append(tuple((t, 0, blocks, -1) for t in range(tile, tile + count)))
        tile += count
    plan = Plan(q, kv, tuple(programs), (), 0, "q_only")
    validate_plan(plan)
    return plan


@lru_cache(maxsize=128)
def make_tail_plan(q, kv, cores=DEFAULT_CORES, pieces=None):
    """Whole tiles in the full waves; each tile of the final wave is cut into
    `pieces` (default: its share of the programs) KV pieces handed out round
    robin after the full waves. Falls back to the whole-tile plan when there
    is no full wave, no final wave or a single KV block."""
    tiles, blocks = _check_args(q, kv, cores)
    if pieces is not None and (type(pieces) is not int or pieces < 2):
        raise ValueError("pieces must be None or an integer >=2")
    full, tail = divmod(tiles, cores)
    if full == 0 or tail == 0 or blocks < 2:
        return make_q_plan(q, kv, cores)
    programs = [[(t, 0, blocks, -1) for t in range(pid * full, (pid + 1) * full)]
                for pid in range(cores)]
    merges, slot, nxt = [], 0, 0
    for i in range(tail):
        tile = full * cores + i
        n = min(blocks, pieces if pieces is not None else cores // tail + (1 if i < cores % tail else 0))
        if n == 1:
            programs[nxt % cores].append((tile, 0, blocks, -1))
            nxt += 1
            continue
        merges.append((tile, slot, n))
        base, extra = divmod(blocks, n)
        first = 0
        for part in range(n):
            size = base + (1 if part < extra else 0)
            programs[nxt % cores].append((tile, first, size, slot))
            first += size
            nxt += 1
            slot += 1
    if not merges:
        return make_q_plan(q, kv, cores)
    plan = Plan(q, kv, tuple(tuple(p) for p in programs), tuple(merges), slot, "tail")
    validate_plan(plan)
    return plan


@lru_cache(maxsize=128)
def make_stream_plan(q, kv, cores=DEFAULT_CORES):
    """Walk the tile-major units; each program takes whole remaining tiles
    while they fit its target (remaining units / remaining programs, half a
    block of slack) and cuts the tile that would overshoot it."""
    tiles, blocks = _check_args(q, kv, cores)
    total = tiles * blocks
    n = min(cores, total)
    programs, cursor = [], 0
    for pid in range(n):
        if cursor == total:
            break
        target = (total - cursor) / (n - pid)
        taken, segs = 0, []
        while cursor < total:
            tile, first = divmod(cursor, blocks)
            left = blocks - first
            if taken + left <= target + 0.5 or pid == n - 1:
                take = left
            else:
                take = min(left, max(0, int(target + 0.5 - taken)))
                if not segs:
                    take = max(1, take)
                if take == 0:
                    break
            segs.append((tile, first, take, -1))
            cursor += take
            taken += take
            if taken >= target - 0.5:
                break
        programs.append(segs)
    plan = _with_slots(q, kv, programs, "stream")
    if not plan.merges:
        # Without a cut tile the whole-tile layout of the same programs.
        return make_q_plan(q, kv, len(programs))
    return plan


def validate_plan(plan):
    """Every (tile, block) unit owned exactly once; whole tiles direct; cut
    tiles in one merge group with consecutive slots."""
    tiles, blocks = -(-plan.q // BLOCK), plan.kv // BLOCK
    spans, direct, slots_of, loads = {}, set(), {}, []
    for segs in plan.programs:
        if not segs:
            raise AssertionError("empty program")
        loads.append(sum(seg[2] for seg in segs))
        for tile, first, count, slot in segs:
            if not (0 <= tile < tiles and 0 <= first < blocks and 0 < count <= blocks - first):
                raise AssertionError(f"segment out of range: {(tile, first, count, slot)}")
            spans.setdefault(tile, []).append((first, first + count))
            if slot < 0:
                if first != 0 or count != blocks or tile in direct:
                    raise AssertionError(f"direct segment must cover its whole tile: {tile}")
                direct.add(tile)
            else:
                slots_of.setdefault(tile, []).append(slot)
    if set(spans) != set(range(tiles)):
        raise AssertionError("every Q tile must be covered")
    for tile, ranges in spans.items():
        cursor = 0
        for first, end in sorted(ranges):
            if first != cursor:
                raise AssertionError(f"tile {tile}: KV blocks covered twice or not at all")
            cursor = end
        if cursor != blocks:
            raise AssertionError(f"tile {tile}: KV blocks not covered to the end")
    if max(loads) - min(loads) > (1 if plan.strategy == "balanced" else blocks):
        raise AssertionError("program loads differ by more than the strategy allows")
    all_slots = sorted(s for v in slots_of.values() for s in v)
    if all_slots != list(range(plan.partial_count)):
        raise AssertionError("partial slots must be 0 .. partial_count - 1")
    if set(slots_of) & direct or len(slots_of) + len(direct) != tiles:
        raise AssertionError("a tile is either direct or merged")
    if len(plan.merges) > len(plan.programs) - 1 and plan.merges:
        raise AssertionError("more merge groups than program boundaries")
    groups = {tile: (first, n) for tile, first, n in plan.merges}
    if len(groups) != len(plan.merges) or set(groups) != set(slots_of):
        raise AssertionError("one merge group per cut tile")
    for tile, (first, n) in groups.items():
        if n < 2 or sorted(slots_of[tile]) != list(range(first, first + n)):
            raise AssertionError(f"tile {tile}: merge group slots must be consecutive")
    return True


def estimate_cost(plan):
    """Critical program work plus the merge, in microseconds (see COST_MODEL)."""
    c = COST_MODEL
    b = c["block_us"] if len(plan.programs) <= NUM_CUS else c["shared_block_us"]
    local = max(sum(seg[2] for seg in segs) * b + len(segs) * c["segment_us"]
                for segs in plan.programs)
    merge = 0.0
    if plan.merges:
        merge = (c["merge_launch_us"] + plan.max_parts * c["parts_us"]
                 + len(plan.merges) * c["merge_tile_us"])
    return dict(local_us=local, merge_us=merge, total_us=local + merge)


def _candidates(limit):
    return [c for c in CANDIDATE_CORES if c <= limit]


@lru_cache(maxsize=128)
def choose_plan(q, kv, cores=DEFAULT_CORES):
    """Cheapest of the whole-tile plan and balanced plans of up to `cores` programs."""
    _check_args(q, kv, cores)
    plans = [make_q_plan(q, kv, cores)] + [make_plan(q, kv, c) for c in _candidates(cores)]
    return min(plans, key=lambda p: (estimate_cost(p)["total_us"], p.partial_count,
                                     -len(p.programs)))


@lru_cache(maxsize=128)
def choose_stream_plan(q, kv, cores=DEFAULT_CORES):
    """Split plan (stream or tail, up to `cores` programs) only when it beats
    the whole-tile plan by more than one block's cost."""
    _check_args(q, kv, cores)
    direct = make_q_plan(q, kv, cores)
    plans = [make_stream_plan(q, kv, c) for c in _candidates(cores)]
    plans += [make_tail_plan(q, kv, c) for c in _candidates(cores)]
    split = min(plans, key=lambda p: (estimate_cost(p)["total_us"], p.partial_count))
    if estimate_cost(direct)["total_us"] - estimate_cost(split)["total_us"] > COST_MODEL["block_us"]:
        return split
    return direct


# Fallback of the static builder (build_fused_kernel): the automatic split path
# is faster at most B1H1 shapes on MI355X, and the two estimates (estimate_cost
# above and any comparable model of the automatic plans) miss by 10% on median,
# more than the paths usually differ, so the choice is read from measurements:
# `python bench.py --suite static-scan` timed both paths (GPU time per call
# from graph replays, checked against the oracle) over Q 64..16384 x KV
# 512..32768 (calibration/mi355x_static_scan.jsonl); the static plan is kept
# where the nearest measured shape (in log2 Q, log2 KV) ran it at least
# STATIC_MIN_SPEEDUP times as fast as the automatic path.
STATIC_CALIBRATION = pathlib.Path(__file__).with_name("calibration") / "mi355x_static_scan.jsonl"
STATIC_MIN_SPEEDUP = 1.02


@lru_cache(maxsize=1)
def static_calibration() -> tuple:
    """((Q, KV, automatic us, static us), ...) of the committed static-scan records."""
    out = []
    for line in STATIC_CALIBRATION.read_text().splitlines():
        rec = json.loads(line)
        if rec.get("suite") == "static-scan":
            out.append((rec["q_len"], rec["kv_len"], rec["auto_us"], rec["static_us"]))
    if not out:
        raise ValueError(f"{STATIC_CALIBRATION} holds no static-scan records")
    return tuple(out)


def static_preferred(q: int, kv: int) -> bool:
    """True where the static plan measured at least STATIC_MIN_SPEEDUP times
    as fast as the automatic split at the nearest calibrated shape."""
    _check_args(q, kv, 1)
    lq, lk = math.log2(q), math.log2(kv)
    nq, nk, auto_us, static_us = min(
        static_calibration(), key=lambda r: ((math.log2(r[0]) - lq) ** 2 + (math.log2(r[1]) - lk) ** 2,
                                             r[0], r[1]))
    return auto_us >= STATIC_MIN_SPEEDUP * static_us
