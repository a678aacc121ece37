"""Automatic plans of the planner's larger-shape rules against the CPU oracle
(MI355X only): the prefill layout for Q > 128 from 2^24 query-key pairs, its
split fill of at least 8 keys per query-tile task, the query layout's fill of
four key rounds from 2^22 pairs, and the move of short-decode plans of 16 or
more splits to the single-stage key kernel. Each case checks the plan the
rule predicts (split_cost_model restates the planner) and the output at the
reference tolerances, with ragged lengths and NaN in every unread pool row.
"""
import pytest
import torch

from oracle import mha_oracle as O
from tests.test_gpu_parity import check_output

pytestmark = pytest.mark.gpu

PAGE = 128


def run(b, sq, h, d, kv, causal, dtype, lengths=None):
    from fgw_amd.operators.mha.current import build_kernel
    width = kv // PAGE
    case = (f"auto_B{b}_Q{sq}_H{h}_D{d}_KV{kv}", b, sq, h, d, PAGE, width)
    q, k, v, table = O.make_inputs(case, 77, dtype)
    lt = torch.tensor(lengths or [kv] * b, dtype=torch.int32)
    k, v = O.poison_unread(k, v, table, lt, PAGE)
    full = lengths is None
    kern = build_kernel(b, sq, h, d, k.shape[0], width, PAGE, causal,
                        "float16" if dtype == torch.float16 else "bfloat16", 0,
                        full_kv_cache=full, cache_lengths=None if full else tuple(lengths))
    label = (f"B{b} Q{sq} H{h} D{d} KV{kv} causal={causal} {dtype}: layout={kern.layout} "
             f"splits={kern.num_splits} stages={kern.stages} grid={kern.compute_grid}")
    print(label, flush=True)
    got = kern(*(x.cuda() for x in (q, k, v, table, lt)))
    torch.cuda.synchronize()
    expected = O.chunked_reference(q, k, v, table, lt, PAGE, causal, 128)
    check_output(got, expected, q, lt, causal, label)
    return kern


@pytest.mark.parametrize("b,sq,h,d,kv,causal,splits", [
    (4, 384, 8, 128, 8192, False, 4),   # 2^26.6 pairs, 32 tasks: 256 keys per split at least
    (4, 384, 8, 128, 8192, True, 4),
    (2, 160, 16, 64, 8192, False, 8),   # Sq just above one query-layout tile
    (8, 320, 8, 128, 1024, False, 1),   # 128 tasks: 1024 keys per split, KV 1024 stays whole
])
def test_prefill_layout_from_2_24_pairs(b, sq, h, d, kv, causal, splits):
    kern = run(b, sq, h, d, kv, causal, torch.bfloat16)
    assert (kern.layout, kern.num_splits) == ("prefill", splits)


def test_query_layout_below_the_pairs_rule():
    # 2^23 pairs at Q512: the query layout, four key rounds (256 keys) per split.
    kern = run(1, 512, 4, 128, 4096, False, torch.float16)
    assert kern.layout == "query"
    assert 4096 // kern.num_splits >= 256


def test_query_fill_of_four_rounds():
    # 2^23 pairs, head dim 64 (outside the cost model): 16 tasks x 16 splits of 256
    # keys, not 32 splits of 128.
    kern = run(2, 96, 8, 64, 4096, False, torch.bfloat16)
    assert (kern.layout, kern.num_splits) == ("query", 16)


@pytest.mark.parametrize("b,sq,h,kv,dtype,splits", [
    (2, 1, 8, 32768, torch.float16, 64),    # 16 splits -> 64 single-stage (512 keys each)
    (1, 4, 16, 16384, torch.bfloat16, 32),  # Sq 4: 16 -> 32 (512 keys each)
    (2, 1, 8, 8192, torch.bfloat16, 32),    # 16 -> 32 (256 keys each)
])
def test_short_decode_moves_to_the_single_stage_kernel(b, sq, h, kv, dtype, splits):
    # The cost model picks 16 double-stage splits for each of these shapes.
    kern = run(b, sq, h, 128, kv, False, dtype)
    assert (kern.layout, kern.stages, kern.num_splits) == ("key", 1, splits)


def test_ragged_decode_keeps_the_balanced_double_stage_plan():
    # Host-known ragged lengths: the length-balanced plan of the cost model, which the
    # single-stage move leaves alone.
    kern = run(4, 1, 8, 128, 32768, False, torch.bfloat16,
               lengths=[int(x) for x in O.imbalanced_lengths(32768)])
    assert kern.stages == 2 and kern.split_keys > 0
