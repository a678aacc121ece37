"""Pins of the CPU oracle (oracle/mha_oracle.py) -- CPU only.

Each oracle function is checked against something that does not restate it:
the reference's recorded harness vectors, a float64 brute force written with
plain Python loops, closed forms, the reference's own merge vectors and
published counts. Planted mistakes in copies of the oracle must fail the
same checks.
"""
import json
import math
import pathlib
import random

import numpy as np
import pytest
import torch

from oracle import mha_oracle as O
from tests import mha_cases

GOLDEN = pathlib.Path(__file__).with_name("golden") / "accuracy_report_vectors.json"


# ---------------------------------------------------------------- input recipes
def test_lengths_and_pool_rows_match_reference_reports():
    vectors = json.loads(GOLDEN.read_text())["vectors"]
    assert len(vectors) >= 200
    for vec in vectors:
        case = (vec["case"], vec["B"], vec["Sq"], vec["H"], vec["D"], vec["page_size"],
                vec["table_width"])
        assert O.lengths_for(case, vec["pattern"], vec["seed"]) == vec["lengths"], vec
        pool_pages = max(case[6] + 3, case[1] * case[6] + 1)
        assert pool_pages * case[5] == vec["pool_rows"], vec


def test_make_inputs_recipe_properties():
    for name in ("tiny", "many_queries", "general_d48_page48", "split_d16_q1"):
        case = mha_cases.ALL_CASES[name]
        _, b, sq, h, d, p, w = case
        q, k, v, table = O.make_inputs(case, 7, torch.bfloat16)
        pool_pages = max(w + 3, b * w + 1)
        assert q.shape == (b, sq, h, d) and k.shape == (pool_pages * p, h, d) == v.shape
        assert table.dtype == torch.int32 and table.shape == (b, w)
        assert int(table.max()) < pool_pages - 1  # the last pool page is never referenced
        if b > 1:
            assert (table[1:, 0] == table[0, 0]).all()
        if w > 1:
            assert table[-1, -1] == table[-1, 0]
        q2, _, _, table2 = O.make_inputs(case, 7, torch.bfloat16)
        assert torch.equal(q, q2) and torch.equal(table, table2)  # seeded


def test_poison_unread_marks_exactly_the_dead_rows():
    case = mha_cases.ALL_CASES["many_queries"]
    q, k, v, table = O.make_inputs(case, 42, torch.float16)
    lengths = torch.tensor(O.lengths_for(case, "mixed", 42), dtype=torch.int32)
    kp, vp = O.poison_unread(k, v, table, lengths, case[5])
    live = set()
    for b in range(table.shape[0]):
        for pos in range(int(lengths[b])):
            live.add(int(table[b, pos // case[5]]) * case[5] + pos % case[5])
    for row in range(k.shape[0]):
        assert bool(torch.isnan(kp[row]).all()) == (row not in live)
        assert bool(torch.isnan(vp[row]).all()) == (row not in live)


# ------------------------------------------------------------- float64 brute force
def brute_force(q, k, v, table, lengths, page, causal):
    """Softmax attention in float64 with explicit Python loops."""
    q64, k64, v64 = (x.double().numpy() for x in (q, k, v))
    b_, sq, h_, d = q64.shape
    out = np.zeros((b_, sq, h_, d))
    for b in range(b_):
        n = int(lengths[b])
        rows = [int(table[b, pos // page]) * page + pos % page for pos in range(n)]
        for qi in range(sq):
            end = max(n - sq + qi + 1, 0) if causal else n
            for hh in range(h_):
                if end == 0:
                    continue
                scores = [sum(q64[b, qi, hh, x] * k64[r, hh, x] for x in range(d)) / math.sqrt(d)
                          for r in rows[:end]]
                peak = max(scores)
                w = [math.exp(s - peak) for s in scores]
                tot = sum(w)
                for x in range(d):
                    out[b, qi, hh, x] = sum(wi * v64[r, hh, x] for wi, r in zip(w, rows[:end])) / tot
    return torch.from_numpy(out)


def tiny_problem(seed, b=3, sq=4, h=2, d=16, page=3, width=4, lengths=(0, 2, 11), dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    pages = b * width + 2
    table = torch.randperm(pages, generator=g)[: b * width].reshape(b, width).to(torch.int32)
    table[-1, -1] = table[-1, 0]
    q = torch.randn(b, sq, h, d, generator=g).to(dtype)
    k = torch.randn(pages * page, h, d, generator=g).to(dtype)
    v = torch.randn(pages * page, h, d, generator=g).to(dtype)
    return q, k, v, table, torch.tensor(lengths, dtype=torch.int32), page


@pytest.mark.parametrize("seed", [1, 2, 3])
@pytest.mark.parametrize("causal", [False, True])
def test_reference_matches_float64_brute_force(seed, causal):
    q, k, v, table, lengths, page = tiny_problem(seed)
    expected = brute_force(q, k, v, table, lengths, page, causal)
    for fn in (O.reference, lambda *a: O.chunked_reference(*a, chunk=3)):
        got = fn(q, k, v, table, lengths, page, causal)
        torch.testing.assert_close(got.double(), expected, rtol=1e-5, atol=1e-6)


def test_reference_closed_forms():
    q, k, v, table, lengths, page = tiny_problem(5, lengths=(1, 0, 7))
    out = O.reference(q, k, v, table, lengths, page, False)
    row0 = int(table[0, 0]) * page
    torch.testing.assert_close(out[0, :, :, :], v[row0].expand_as(out[0]), rtol=0, atol=1e-6)
    assert torch.count_nonzero(out[1]) == 0
    # Equal keys give equal weights: the output is the mean of the visible V rows.
    k2 = k.clone()
    k2[:] = k[0]
    out = O.reference(q, k2, v, table, lengths, page, False)
    rows = O.physical_rows(table, 2, 7, page)
    torch.testing.assert_close(out[2, 0], v[rows].mean(0), rtol=1e-5, atol=1e-6)
    # Causal, Sq > len: rows with no visible key are exactly zero.
    out = O.reference(q, k, v, table, lengths, page, True)
    assert torch.count_nonzero(out[0, :3]) == 0 and torch.count_nonzero(out[0, 3]) > 0


def test_chunked_reference_equals_reference_at_bf16():
    case = mha_cases.ALL_CASES["cube_q129"]
    q, k, v, table = O.make_inputs(case, 7, torch.bfloat16)
    for causal in (False, True):
        lengths = torch.tensor(O.lengths_for(case, "mixed", 7), dtype=torch.int32)
        a = O.reference(q, k, v, table, lengths, case[5], causal)
        b = O.chunked_reference(q, k, v, table, lengths, case[5], causal, 32)
        torch.testing.assert_close(a, b, rtol=1e-2, atol=4e-3)


# Planted mistakes: each must be caught by the brute-force pin.
def _wrong_scale(q, k, v, table, lengths, page, causal):
    return O.reference(q * math.sqrt(q.shape[-1]) ** 0.5, k, v, table, lengths, page, causal)


def _wrong_causal(q, k, v, table, lengths, page, causal):
    return O.reference(q, k, v, table, lengths + 1, page, causal)


def _wrong_page(q, k, v, table, lengths, page, causal):
    return O.reference(q, k, v, table.flip(1).contiguous(), lengths, page, causal)


def _wrong_operand(q, k, v, table, lengths, page, causal):
    return O.reference(q, v, k, table, lengths, page, causal)


@pytest.mark.parametrize("mutant", [_wrong_scale, _wrong_causal, _wrong_page, _wrong_operand])
def test_planted_mistakes_fail_the_pin(mutant):
    q, k, v, table, lengths, page = tiny_problem(9, lengths=(5, 9, 11))
    expected = brute_force(q, k, v, table, lengths, page, True)
    got = mutant(q, k, v, table, lengths.clone(), page, True)
    assert not torch.allclose(got.double(), expected, rtol=1e-3, atol=1e-4)


# ------------------------------------------------------------------- split merge
def test_merge_matches_reference_raw_partition_vectors():
    # Vectors of tests/mha/test_raw_partial_state.py:8-10 (2-D keys/values).
    keys = [(1., 2.), (-3., 4.), (5., -6.), (2., -1.), (-4., -2.), (3., 5.)]
    values = [(2., -1.), (4., 3.), (-2., 5.), (7., -3.), (1., 6.), (-5., 8.)]
    for query in ((1., -2.), (-3., 4.), (100., -100.)):
        scores = [sum(a * b for a, b in zip(query, key)) / math.sqrt(2) for key in keys]
        peak = max(scores)
        w = [math.exp(x - peak) for x in scores]
        dense = [sum(wi * val[d] for wi, val in zip(w, values)) / sum(w) for d in range(2)]
        parts, lse = [], []
        for begin, end in ((0, 2), (2, 5), (5, 6), (6, 6)):
            if begin == end:
                parts.append([0.0, 0.0])
                lse.append(-1e30)
                continue
            m = max(scores[begin:end])
            ww = [math.exp(x - m) for x in scores[begin:end]]
            parts.append([sum(a * val[d] for a, val in zip(ww, values[begin:end])) / sum(ww)
                          for d in range(2)])
            lse.append(m + math.log(sum(ww)))
        p = torch.tensor(parts, dtype=torch.float64).reshape(1, 1, 4, 1, 2)
        s = torch.tensor(lse, dtype=torch.float64).reshape(1, 1, 4, 1)
        got = O.merge_partials(p, s, torch.float64)
        torch.testing.assert_close(got.reshape(2).double(), torch.tensor(dense, dtype=torch.float64),
                                   rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("splits", [1, 2, 3, 8])
@pytest.mark.parametrize("causal", [False, True])
def test_partial_states_merge_to_dense(splits, causal):
    q, k, v, table, lengths, page = tiny_problem(11, sq=5, lengths=(0, 4, 12))
    parts, lse = O.partial_states(q, k, v, table, lengths, page, causal, splits, block_keys=2,
                                  rows_per_tile=2)
    got = O.merge_partials(parts, lse, torch.float32)
    expected = brute_force(q, k, v, table, lengths, page, causal)
    torch.testing.assert_close(got.double(), expected, rtol=1e-5, atol=1e-6)
    empty = lse <= -1e29
    assert torch.count_nonzero(parts[empty.unsqueeze(-1).expand_as(parts)]) == 0


# ------------------------------------------------------------ counts and helpers
def test_useful_flops_and_bytes_known_answers():
    assert O.useful_flops([2048, 2048], 4096, 8, 128, False) == 68_719_476_736
    assert O.useful_flops([2048, 2048], 32768, 8, 128, False) == 549_755_813_888
    assert O.algorithmic_bytes([32768, 32768], 1, 8, 128, 256) == 268_445_704
    # Causal square attention counts S(S+1)/2 pairs (MFU.md section 4).
    assert O.useful_flops([100], 100, 1, 16, True) == 4 * 16 * 100 * 101 // 2


def test_page_division_is_exact():
    rng = random.Random(3)
    for page in list(range(1, 300)) + [1000, 4096, 65535, 2**20 + 7]:
        magic, shift = O.page_divisor(page)
        assert 0 <= magic < 2**32
        ns = list(range(0, 3000)) + [rng.randrange(0, 2**31) for _ in range(300)] + [2**31 - 1]
        for n in ns:
            assert O.page_div(n, magic, shift) == n // page, (page, n)


def test_gather_packed_matches_explicit_rows():
    q, k, v, table, lengths, page = tiny_problem(4, lengths=(3, 0, 10))
    ok, ov = O.gather_packed(k, v, table, lengths, page, out_len=12)
    for b in range(3):
        for pos in range(12):
            if pos < int(lengths[b]):
                row = int(table[b, pos // page]) * page + pos % page
                assert torch.equal(ok[b, pos], k[row]) and torch.equal(ov[b, pos], v[row])
            else:
                assert torch.count_nonzero(ok[b, pos]) == 0


def test_packed_offsets_closed_form():
    offsets, rows, table = O.packed_offsets([0, 1, 128, 129, 300], 128, 3)
    assert offsets == [0, 0, 128, 256, 512, 896] and rows == 896
    assert table.tolist() == [[0, 1, 2], [0, 1, 2], [1, 2, 3], [2, 3, 4], [4, 5, 6]]
    offsets, rows, _ = O.packed_offsets([0, 0], 16, 2)
    assert offsets == [0, 0, 0] and rows == 16  # rows never below one page


def test_pack_pages_matches_row_by_row_resolution():
    q, k, v, table, lengths, page = tiny_problem(4, lengths=(3, 0, 10))
    ok, ov, offsets = O.pack_pages(k, v, table, lengths, page)
    assert offsets == [0, 3, 3, 15] and ok.shape == (15,) + tuple(k.shape[1:])  # page 3
    for b in range(3):
        n = int(lengths[b])
        live = O.physical_rows(table, b, n, page)
        for pos in range(offsets[b + 1] - offsets[b]):
            # live rows through the attention's own resolution, page tails
            # through the page id of the last live page
            row = int(live[pos]) if pos < n else int(table[b, pos // page]) * page + pos % page
            assert torch.equal(ok[offsets[b] + pos], k[row])
            assert torch.equal(ov[offsets[b] + pos], v[row])


def test_bench_inputs_recipe_properties():
    q, k, v, table, lengths = O.bench_inputs(2, 3, 4, 16, 8, 40, torch.bfloat16)
    assert q.shape == (2, 3, 4, 16) and k.shape == (2 * 5 * 8, 4, 16) == v.shape
    assert table.dtype == torch.int32 and lengths.tolist() == [40, 40]
    # The table is a shuffle of all pool pages: every page is read exactly once.
    assert sorted(table.flatten().tolist()) == list(range(10))
    again = O.bench_inputs(2, 3, 4, 16, 8, 40, torch.bfloat16)
    assert all(torch.equal(a, b) for a, b in zip((q, k, v, table), again[:4]))
    other = O.bench_inputs(2, 3, 4, 16, 8, 40, torch.bfloat16, seed=8)
    assert not torch.equal(table, other[3]) or not torch.equal(q, other[0])


def test_bench_inputs_recipe_values():
    """Literal values of the benchmark recipe at seed 7 (B2, Q4096, H8, D128,
    page 128, KV 2048): the shuffled table and the first draws of q, k and v.
    They fail an unshuffled (identity) table, a different seed and a changed
    draw order (table, then q, k, v; bench_mha_mfu.py:181-187). The
    reference records none of these values, so they pin the recipe against
    changes of this restatement, not against a reference run."""
    q, k, v, table, lengths = O.bench_inputs(2, 4096, 8, 128, 128, 2048, torch.bfloat16)
    assert table.tolist() == [[15, 11, 3, 6, 19, 20, 21, 1, 12, 16, 30, 24, 5, 22, 9, 29],
                              [26, 7, 27, 10, 8, 18, 2, 23, 28, 13, 31, 0, 4, 14, 25, 17]]
    assert not torch.equal(table.flatten(), torch.arange(32, dtype=torch.int32))
    assert q[0, 0, 0, :4].float().tolist() == [0.50390625, -0.08349609375, -0.0234375,
                                               0.1748046875]
    assert k[0, 0, :4].float().tolist() == [0.59375, 1.2578125, 0.75, -0.88671875]
    assert v[-1, -1, -4:].float().tolist() == [1.7578125, -1.6875, 0.4296875, -0.404296875]


def test_imbalanced_lengths_recipe():
    """Config 4's imbalanced variant, randint(KV // 8, KV + 1, (4,)) from
    Generator().manual_seed(7), at every KV of the config: literal values, and
    every length inside [KV / 8, KV]."""
    expected = {512: [415, 147, 348, 469], 2048: [1194, 1931, 345, 1618],
                8192: [4635, 4285, 4326, 1917], 32768: [13321, 16319, 6592, 12115]}
    for kv, want in expected.items():
        got = O.imbalanced_lengths(kv)
        assert got.dtype == torch.int32 and got.tolist() == want
        assert all(kv // 8 <= n <= kv for n in want)
    assert O.imbalanced_lengths(8192, seed=8).tolist() != expected[8192]


def test_rounded_reference_pins():
    """rounded_reference (the reference kernel's rounding points): with
    float32 inputs the cast of P is exact and it equals reference; a two-key
    row follows the closed form (v0 + p v1) / (1 + p) with p cast to bfloat16
    in the numerator only."""
    case = ("pin", 2, 3, 2, 32, 16, 3)
    q, k, v, table = O.make_inputs(case, 11, torch.float32)
    lengths = torch.tensor([37, 5], dtype=torch.int32)
    for causal in (False, True):
        torch.testing.assert_close(O.rounded_reference(q, k, v, table, lengths, 16, causal),
                                   O.reference(q, k, v, table, lengths, 16, causal),
                                   rtol=1e-5, atol=1e-6)
    d = 16
    q1 = torch.zeros(1, 1, 1, d, dtype=torch.bfloat16)
    q1[0, 0, 0, 0] = 1.0
    k1 = torch.zeros(2, 1, d, dtype=torch.bfloat16)
    k1[1, 0, 0] = -3.0  # score difference 3 / sqrt(16) = 0.75
    v1 = torch.zeros(2, 1, d, dtype=torch.bfloat16)
    v1[0, 0, 0], v1[1, 0, 0] = 1.0, 8.0
    table1 = torch.tensor([[0]], dtype=torch.int32)
    got = O.rounded_reference(q1, k1, v1, table1, torch.tensor([2], dtype=torch.int32), 2, False)
    p = math.exp(-0.75)
    p16 = float(torch.tensor(p).to(torch.bfloat16))
    assert p16 != p
    want = float(torch.tensor((1.0 + 8.0 * p16) / (1.0 + p)).to(torch.bfloat16))
    assert float(got[0, 0, 0, 0]) == want


@pytest.mark.parametrize("name,seed,causal,pattern,ratio", [
    ("cube_direct_q129", 42, True, "mixed", 0.733),
    ("cube_direct_q1024", 7, True, "mixed", 0.710),
    ("cube_q257", 2026, True, "full", 0.676),
    ("dim128", 2026, False, "mixed", 0.639),
])
def test_rounding_points_set_the_worst_accuracy_checks(name, seed, causal, pattern, ratio):
    """The accuracy suite's worst BF16 checks: the reference kernel's rounding
    points alone (rounded_reference) reach these error / tolerance ratios
    against the fp32 reference; the HIP kernel's ratios on the same checks are
    the same (tests/test_accuracy_vs_reference.py). dim128 is the reference's
    own recorded worst check (0.639, mha_cube_general_accuracy.json); the
    causal CUBE checks are outside its reports."""
    case = mha_cases.ALL_CASES[name]
    q, k, v, table = O.make_inputs(case, seed, torch.bfloat16)
    lengths = torch.tensor(O.lengths_for(case, pattern, seed), dtype=torch.int32)
    exp = O.chunked_reference(q, k, v, table, lengths, case[5], causal, 128)
    got = O.rounded_reference(q, k, v, table, lengths, case[5], causal)
    rtol, atol = O.TOLERANCES[torch.bfloat16]
    r = ((got.float() - exp.float()).abs() / (atol + rtol * exp.float().abs())).max().item()
    assert r == pytest.approx(ratio, abs=0.001)
