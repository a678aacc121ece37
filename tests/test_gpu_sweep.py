"""Seeded random sweep of the main entry against the CPU oracle (MI355X only).

Each case draws B, H, D (16..256 in steps of 16), page size, table width, Q
length, ragged lengths, causal, dtype, split request and layout from a fixed
seed, poisons every unread pool row with NaN and checks the output against
the oracle at the reference tolerances, with exactly-zero rows where no key
is visible. Key-layout plans at head-dim tile 128 also run on the
single-stage key kernel, which must give the same bits. The draws stay small
enough for the oracle to finish in seconds.
"""
import random

import pytest
import torch

from oracle import mha_oracle as O

pytestmark = pytest.mark.gpu
CASES = 160


def draw(i):
    r = random.Random(9000 + i)
    b, h = r.choice([1, 2, 3]), r.choice([1, 2, 4, 8])
    d = 16 * r.randint(1, 16)
    page = r.choice([16, 32, 48, 64, 128, 256])
    width = r.randint(1, max(1, 2048 // page))
    sq = r.choice([1, 2, 7, 16, 33, 64, 129, 200, 256, 300])
    causal = r.random() < 0.4
    dtype = r.choice([torch.float16, torch.bfloat16])
    layout = r.choice([None, None, "query", "key", "prefill"])
    if layout == "prefill" and not 32 < d <= 128:
        layout = "query"
    splits = r.choice([None, None, 1, 2, 4, 8])
    capacity = width * page
    lengths = [r.choice([0, 1, capacity, r.randint(0, capacity)]) for _ in range(b)]
    return b, h, d, page, width, sq, causal, dtype, layout, splits, lengths


@pytest.mark.parametrize("i", range(CASES))
def test_random_case(i):
    from fgw_amd.operators.mha.current import build_kernel
    b, h, d, page, width, sq, causal, dtype, layout, splits, lengths = draw(i)
    if splits is not None and splits > (width * page + 31) // 32:
        splits = None
    case = (f"sweep{i}", b, sq, h, d, page, width)
    q, k, v, table = O.make_inputs(case, i, dtype)
    lt = torch.tensor(lengths, dtype=torch.int32)
    k, v = O.poison_unread(k, v, table, lt, page)
    label = (f"sweep {i}: B{b} H{h} D{d} page{page} W{width} Sq{sq} causal={causal} {dtype} "
             f"layout={layout} splits={splits} lengths={lengths}")
    print(label, flush=True)
    kern = build_kernel(b, sq, h, d, k.shape[0], width, page, causal,
                        "float16" if dtype == torch.float16 else "bfloat16", 0,
                        num_splits=splits, layout=layout, cache_lengths=tuple(lengths))
    dev = [x.cuda() for x in (q, k, v, table, lt)]
    got = kern(*dev)
    if kern.layout == "key" and kern.dim_padded == 128:
        # The single-stage key kernel computes the same bits.
        single = build_kernel(b, sq, h, d, k.shape[0], width, page, causal,
                              "float16" if dtype == torch.float16 else "bfloat16", 0,
                              num_splits=kern.num_splits, layout="key", stages=1)
        assert single.stages == 1 and torch.equal(single(*dev), got), label
    torch.cuda.synchronize()
    expected = O.reference(q, k, v, table, lt, page, causal)
    got = got.cpu()
    assert torch.isfinite(got).all(), label
    rtol, atol = O.TOLERANCES[dtype]
    torch.testing.assert_close(got, expected, rtol=rtol, atol=atol, msg=lambda m: f"{label}: {m}")
    visible = lt[:, None].expand(b, sq)
    if causal:
        visible = (visible - sq + torch.arange(sq)[None, :] + 1).clamp_min(0)
    assert torch.count_nonzero(got[visible == 0]).item() == 0, label


BALANCED_CASES = 48


def draw_balanced(i):
    """A key-layout plan with length-balanced splits: ragged lengths (some 0,
    some full), B up to 9, explicit split_keys anywhere in 1 .. capacity."""
    r = random.Random(7000 + i)
    b, h = r.randint(1, 9), r.choice([1, 2, 4, 8])
    d = 16 * r.randint(1, 16)
    page = r.choice([16, 32, 64, 128])
    width = r.randint(2, max(2, 2048 // page))
    capacity = width * page
    sq = r.choice([1, 2, 7, 16, 32])
    causal = r.random() < 0.3
    dtype = r.choice([torch.float16, torch.bfloat16])
    splits = r.choice([s for s in (2, 4, 8, 16, 32) if s <= (capacity + 31) // 32] or [2])
    split_keys = r.choice([1, 31, 100, r.randint(1, capacity), capacity])
    lengths = [r.choice([0, 1, capacity, r.randint(0, capacity)]) for _ in range(b)]
    return b, h, d, page, width, sq, causal, dtype, splits, split_keys, lengths


@pytest.mark.parametrize("i", range(BALANCED_CASES))
def test_random_balanced_case(i):
    from fgw_amd.operators.mha.current import build_kernel
    b, h, d, page, width, sq, causal, dtype, splits, split_keys, lengths = draw_balanced(i)
    case = (f"balanced{i}", b, sq, h, d, page, width)
    q, k, v, table = O.make_inputs(case, i, dtype)
    lt = torch.tensor(lengths, dtype=torch.int32)
    k, v = O.poison_unread(k, v, table, lt, page)
    label = (f"balanced sweep {i}: B{b} H{h} D{d} page{page} W{width} Sq{sq} causal={causal} "
             f"{dtype} splits={splits} split_keys={split_keys} lengths={lengths}")
    print(label, flush=True)
    kern = build_kernel(b, sq, h, d, k.shape[0], width, page, causal,
                        "float16" if dtype == torch.float16 else "bfloat16", 0,
                        num_splits=splits, layout="key", split_keys=split_keys)
    assert kern.split_balance == "length", label
    dev = [x.cuda() for x in (q, k, v, table, lt)]
    got = kern(*dev)
    parts, lse = kern.partial_kernel(*dev)
    merged = kern.merge_kernel(parts, lse, dev[4])
    if kern.dim_padded == 128:
        single = build_kernel(b, sq, h, d, k.shape[0], width, page, causal,
                              "float16" if dtype == torch.float16 else "bfloat16", 0,
                              num_splits=splits, layout="key", split_keys=split_keys, stages=1)
        assert single.stages == 1 and torch.equal(single(*dev), got), label
    torch.cuda.synchronize()
    assert torch.equal(merged, got), label
    expected = O.reference(q, k, v, table, lt, page, causal)
    got = got.cpu()
    assert torch.isfinite(got).all(), label
    rtol, atol = O.TOLERANCES[dtype]
    torch.testing.assert_close(got, expected, rtol=rtol, atol=atol, msg=lambda m: f"{label}: {m}")
    visible = lt[:, None].expand(b, sq)
    if causal:
        visible = (visible - sq + torch.arange(sq)[None, :] + 1).clamp_min(0)
    assert torch.count_nonzero(got[visible == 0]).item() == 0, label
