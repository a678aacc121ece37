"""GPU parity of the HIP kernels against the CPU oracle (MI355X only).

Every case follows the reference accuracy harness
(tests/mha/test_mha_paged_accuracy.py:213-273): seeded inputs with a shared
and a repeated page, NaN in every unread pool row, the reference tolerances
(BF16 rtol 1e-2 / atol 4e-3, FP16 2e-3 / 2e-3) and exactly-zero rows where no
key is visible. The K/V gather is checked bit-exactly.
"""
import ctypes
import sys

import pytest
import torch

from oracle import mha_oracle as O
from tests import mha_cases as C

pytestmark = pytest.mark.gpu
DTYPES = (torch.float16, torch.bfloat16)
# BASELINE bar next to the reference's: max-abs 2e-2 (BF16) / 5e-3 (FP16), rtol 1e-2.
BASELINE_ATOL = {torch.bfloat16: 2e-2, torch.float16: 5e-3}


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    from fgw_amd import _lib
    _lib.load()
    name = torch.cuda.get_device_properties(0).gcnArchName
    assert name.startswith("gfx950"), name
    torch.cuda.set_device(0)


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def check_output(got, expected, q, lengths, causal, label):
    """Reference harness assertions; returns the worst error/tolerance ratio."""
    dtype = q.dtype
    assert got.shape == q.shape and got.dtype == dtype and got.is_contiguous(), label
    got = got.cpu()
    assert torch.isfinite(got).all(), f"{label}: non-finite output"
    rtol, atol = O.TOLERANCES[dtype]
    err = (got.float() - expected.float()).abs()
    ratio = (err / (atol + rtol * expected.float().abs())).max().item()
    torch.testing.assert_close(got, expected, rtol=rtol, atol=atol, msg=lambda m: f"{label}: {m}")
    assert err.max().item() <= BASELINE_ATOL[dtype] + 1e-2 * expected.float().abs().max().item()
    b, sq = q.shape[:2]
    visible = lengths[:, None].expand(b, sq)
    if causal:
        visible = (visible - sq + torch.arange(sq)[None, :] + 1).clamp_min(0)
    assert torch.count_nonzero(got[visible == 0]).item() == 0, f"{label}: empty rows must be zero"
    return ratio


def run_case(case, seed, dtype, causal, pattern, **kwargs):
    from fgw_amd.operators.mha.current import mha_paged_decode
    _, b, sq, h, d, p, w = case
    q, k, v, table = O.make_inputs(case, seed, dtype)
    lengths = torch.tensor(O.lengths_for(case, pattern, seed), dtype=torch.int32)
    k, v = O.poison_unread(k, v, table, lengths, p)
    dev = [x.cuda() for x in (q, k, v, table, lengths)]
    got = mha_paged_decode(*dev, page_size=p, is_causal=causal, **kwargs)
    torch.cuda.synchronize()
    if sq > 256:
        expected = O.chunked_reference(q, k, v, table, lengths, p, causal, 128)
    else:
        expected = O.reference(q, k, v, table, lengths, p, causal)
    label = f"{case[0]} seed={seed} {dtype} causal={causal} {pattern} {kwargs}"
    return check_output(got, expected, q, lengths, causal, label)


SUITE = C.EXTENDED + C.CUBE + C.GENERAL + C.SPLIT


@pytest.mark.parametrize("case", SUITE, ids=[c[0] for c in SUITE])
def test_accuracy_suite(case):
    seeds = C.SEEDS if case[2] * case[1] <= 512 else (7,)
    worst = 0.0
    for seed in seeds:
        for dtype in DTYPES:
            for causal in (False, True):
                for pattern in C.PATTERNS:
                    worst = max(worst, run_case(case, seed, dtype, causal, pattern))
    log(f"{case[0]}: worst error/tolerance {worst:.3f}")


@pytest.mark.parametrize("splits", [1, 2, 4, 8, 16, 32])
def test_forced_splits(splits):
    for name in ("split_d16_q1", "split_d48_q17", "split_d128_q33", "split_d256_q129"):
        case = C.ALL_CASES[name]
        for dtype in DTYPES:
            for causal in (False, True):
                run_case(case, 7, dtype, causal, "mixed", num_splits=splits)
                run_case(case, 7, dtype, causal, "full", num_splits=splits)


def test_cost_model_policy_on_causal_ragged_calls():
    """split_policy='cost_model' with causal, ragged lengths plans with the
    host lengths (v7_experimental.py:885-886) and matches the oracle."""
    for name in ("split_d16_q1", "split_d128_q33", "split_d48_q17", "cube_decode2048"):
        case = C.ALL_CASES[name]
        for dtype in DTYPES:
            run_case(case, 7, dtype, True, "mixed", split_policy="cost_model")
            run_case(case, 11, dtype, False, "mixed", split_policy="cost_model")


def test_gather_bit_exact():
    from fgw_amd import _lib
    lib = _lib.load()
    for name in ("tiny", "general_d48_page48", "many_queries", "page256", "split_d16_q1",
                 "non_power_two_dim"):
        case = C.ALL_CASES[name]
        _, b, sq, h, d, p, w = case
        for pattern in C.PATTERNS:
            q, k, v, table = O.make_inputs(case, 42, torch.bfloat16)
            lengths = torch.tensor(O.lengths_for(case, pattern, 42), dtype=torch.int32)
            k, v = O.poison_unread(k, v, table, lengths, p)
            out_len = p * w
            ok = torch.full((b, out_len, h, d), float("nan"), dtype=k.dtype, device="cuda")
            ov = torch.full_like(ok, float("nan"))
            dk, dv, dt, dl = (x.cuda() for x in (k, v, table, lengths))
            shape = _lib.Shape(b, sq, h, d, k.shape[0], w, p, 0, _lib.DTYPE_BFLOAT16)
            t = _lib.Tensors(None, dk.data_ptr(), dv.data_ptr(), dt.data_ptr(), dl.data_ptr(),
                             None, None, None)
            stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            _lib.check(lib.fgw_mha_gather_kv(ctypes.byref(shape), ctypes.byref(t), ok.data_ptr(),
                                             ov.data_ptr(), out_len, stream))
            torch.cuda.synchronize()
            ek, ev = O.gather_packed(k, v, table, lengths, p, out_len)
            torch.testing.assert_close(ok.cpu(), ek, rtol=0, atol=0, equal_nan=False)
            torch.testing.assert_close(ov.cpu(), ev, rtol=0, atol=0, equal_nan=False)


def test_layouts_and_persistent_grids_agree():
    from fgw_amd.operators.mha.current import build_kernel
    case = ("q40", 2, 40, 4, 128, 64, 20)
    for causal in (False, True):
        q, k, v, table = O.make_inputs(case, 7, torch.bfloat16)
        lengths = torch.tensor([1000, 37], dtype=torch.int32)
        k, v = O.poison_unread(k, v, table, lengths, 64)
        dev = [x.cuda() for x in (q, k, v, table, lengths)]
        expected = O.reference(q, k, v, table, lengths, 64, causal)
        outs = []
        for layout in ("query", "key", "prefill"):
            for persistent in (None, 1, 7, "device"):
                kern = build_kernel(2, 40, 4, 128, k.shape[0], 20, 64, causal, "bfloat16", 0,
                                    num_splits=2, persistent_programs=persistent, layout=layout)
                got = kern(*dev)
                torch.cuda.synchronize()
                check_output(got, expected, q, lengths, causal, f"{layout} {persistent}")
                outs.append((layout, persistent, got.cpu()))
        # Work placement never changes the arithmetic of a work item.
        for layout, persistent, got in outs:
            ref = next(o for lay, _, o in outs if lay == layout)
            diff = (got.float() - ref.float()).abs()
            assert torch.equal(got, ref), (
                f"causal={causal} {layout} persistent={persistent}: {int((diff > 0).sum())} "
                f"values differ, max {diff.max().item():.3g}")


def test_partial_and_merge_components():
    from fgw_amd.operators.mha.current import build_kernel
    case = ("comp", 2, 20, 4, 96, 32, 40)
    q, k, v, table = O.make_inputs(case, 2026, torch.bfloat16)
    lengths = torch.tensor([1200, 333], dtype=torch.int32)
    dev = [x.cuda() for x in (q, k, v, table, lengths)]
    for causal in (False, True):
        kern = build_kernel(2, 20, 4, 96, k.shape[0], 40, 32, causal, "bfloat16", 0, num_splits=8)
        assert kern.execution_mode == "split_and_merge" and kern.layout == "key"
        parts, lse = kern.partial_kernel(*dev)
        torch.cuda.synchronize()
        eparts, else_ = O.partial_states(q, k, v, table, lengths, 32, causal, 8, block_keys=32,
                                         rows_per_tile=kern.block_q)
        empty = else_ <= -1e29
        assert torch.equal(lse.cpu() <= -1e29, empty)
        torch.testing.assert_close(lse.cpu()[~empty], else_[~empty], rtol=0, atol=2e-3)
        torch.testing.assert_close(parts.cpu(), eparts, rtol=1e-2, atol=4e-3)
        # Merge of the oracle's exact partials against the oracle merge.
        out = kern.merge_kernel(eparts.cuda().contiguous(), else_.cuda().contiguous())
        torch.cuda.synchronize()
        torch.testing.assert_close(out.cpu().float(),
                                   O.merge_partials(eparts, else_, torch.bfloat16).float(),
                                   rtol=8e-3, atol=1e-5)
        full = kern(*dev)
        expected = O.reference(q, k, v, table, lengths, 32, causal)
        check_output(full, expected, q, lengths, causal, f"components causal={causal}")


def test_wide_merge_many_splits():
    """Merges of more than 16 splits (the splits spread over one workgroup per
    row) against the oracle merge: head dims whose column count does not divide
    the workgroup (48), several chunks per thread (D 256, 128 splits), empty
    splits and one all-empty row (exact zero)."""
    from fgw_amd.operators.mha.current import build_kernel
    gen = torch.Generator().manual_seed(11)
    cases = ((2, 3, 2, 128, 64, torch.bfloat16), (1, 1, 3, 48, 128, torch.float16),
             (2, 2, 1, 256, 32, torch.bfloat16), (1, 5, 2, 16, 32, torch.float16),
             (2, 1, 8, 128, 32, torch.bfloat16), (1, 2, 1, 256, 128, torch.bfloat16))
    for (b, sq, h, d, splits, dtype) in cases:
        page, kv = 32, splits * 64
        name = "bfloat16" if dtype == torch.bfloat16 else "float16"
        kern = build_kernel(b, sq, h, d, b * kv, kv // page, page, False, name, 0,
                            num_splits=splits)
        assert kern.num_splits == splits and kern.execution_mode == "split_and_merge"
        parts = torch.randn(b, h, splits, sq, d, generator=gen)
        lse = torch.randn(b, h, splits, sq, generator=gen) * 4.0
        lse[torch.rand(lse.shape, generator=gen) < 0.3] = -1e30
        lse[0, 0, :, 0] = -1e30
        out = kern.merge_kernel(parts.cuda(), lse.cuda())
        torch.cuda.synchronize()
        label = f"wide merge B{b} Q{sq} H{h} D{d} splits={splits} {name}"
        assert torch.equal(out[0, 0, 0].cpu(), torch.zeros(d, dtype=dtype)), label
        torch.testing.assert_close(out.cpu().float(), O.merge_partials(parts, lse, dtype).float(),
                                   rtol=8e-3, atol=1e-5, msg=label)


def test_length_balanced_splits():
    """Ragged decode batches with length-balanced splits (request b:
    clamp(ceil(len_b / split_keys), 1, S) slots): the automatic split picks
    them for config 4's imbalanced B4 at KV 32768; explicit plans cover the
    rest. Outputs against the oracle with NaN in every unread pool row; the
    partial and merge components (the merge given the lengths) equal the
    fused call bit for bit; with uniform lengths a balanced plan equals the
    even plan bit for bit."""
    from fgw_amd.operators.mha.current import build_kernel, mha_paged_decode
    cases = (("imbalanced_kv32768", 4, 1, 8, 128, 128, 256, [13321, 16319, 6592, 12115],
              torch.bfloat16, None),
             ("imbalanced_q16", 4, 16, 8, 128, 128, 64, [4635, 4285, 4326, 1917], torch.float16,
              (16, 491)),
             ("empty_and_short", 5, 1, 2, 128, 64, 64, [0, 4096, 17, 1000, 2500], torch.bfloat16,
              (16, 470)),
             ("page32_q7", 3, 7, 4, 128, 32, 64, [2048, 100, 1500], torch.bfloat16, (32, 83)))
    for (name, b, sq, h, d, page, width, lens, dtype, explicit) in cases:
        case = (name, b, sq, h, d, page, width)
        q, k, v, table = O.make_inputs(case, 5, dtype)
        lengths = torch.tensor(lens, dtype=torch.int32)
        k, v = O.poison_unread(k, v, table, lengths, page)
        dev = [x.cuda() for x in (q, k, v, table, lengths)]
        dname = "bfloat16" if dtype == torch.bfloat16 else "float16"
        if explicit is None:
            got = mha_paged_decode(*dev, page_size=page)
            kern = build_kernel(b, sq, h, d, k.shape[0], width, page, False, dname, 0,
                                cache_lengths=tuple(lens))
        else:
            kern = build_kernel(b, sq, h, d, k.shape[0], width, page, False, dname, 0,
                                num_splits=explicit[0], layout="key", split_keys=explicit[1])
            got = kern(*dev)
        torch.cuda.synchronize()
        expected = O.reference(q, k, v, table, lengths, page, False)
        check_output(got, expected, q, lengths, False, f"balanced {name}")
        assert kern.split_balance == "length" and kern.split_keys > 0, (name, kern.num_splits)
        fused = kern(*dev)
        parts, lse = kern.partial_kernel(*dev)
        merged = kern.merge_kernel(parts, lse, dev[4])
        torch.cuda.synchronize()
        assert torch.equal(fused, got) and torch.equal(merged, fused), name
        with pytest.raises(ValueError, match="length-balanced"):
            kern.merge_kernel(parts, lse)
        log(f"{name}: splits {kern.num_splits} split_keys {kern.split_keys}")
    # Uniform lengths: every request takes all slots, the even partition.
    from fgw_amd import _lib
    from fgw_amd.operators.mha.kernels import mha_paged_decode_hip as HIP
    q, k, v, table, lengths = O.bench_inputs(2, 1, 8, 128, 128, 8192, torch.bfloat16)
    dev = [x.cuda() for x in (q, k, v, table, lengths)]
    even = build_kernel(2, 1, 8, 128, k.shape[0], 64, 128, False, "bfloat16", 0, num_splits=16)
    meta = (("persistent_programs", HIP.PERSISTENT_DEVICE), ("requested_split_policy", "auto"),
            ("split_policy", "explicit"))
    balanced = HIP._planned(2, 1, 8, 128, k.shape[0], 64, 128, False, "bfloat16", 0, 16, -1,
                            None, meta, 512)
    assert balanced.split_keys == 512 and even.split_keys == 0
    assert torch.equal(balanced(*dev), even(*dev))


def test_key_layout_stage_variants():
    """The key layout's single-stage kernel (two workgroups per CU) and its
    double-stage kernel (head-dim tile 128) give the same bits for every plan,
    and the oracle's output: even and length-balanced splits, direct plans,
    several work items per program (64 splits of B2 H8: 1024 items on 512
    single-stage programs), ragged, empty and causal rows, FP16 and BF16, head
    dims 96 and 128."""
    from fgw_amd.operators.mha.current import build_kernel
    cases = (
        # name, B, Sq, H, D, page, width, dtype, lengths, causal, split_keys
        ("decode_kv8192", 2, 1, 8, 128, 128, 64, torch.bfloat16, "full", False, None),
        ("q5_ragged_causal", 3, 5, 2, 128, 16, 64, torch.float16, [1000, 0, 4], True, None),
        ("q32_d96", 2, 32, 3, 96, 32, 24, torch.bfloat16, [768, 31], False, None),
        ("balanced", 4, 1, 8, 128, 128, 64, torch.bfloat16, [4635, 0, 8192, 1917], False, 491),
    )
    for (name, b, sq, h, d, page, width, dtype, lens, causal, split_keys) in cases:
        case = (name, b, sq, h, d, page, width)
        q, k, v, table = O.make_inputs(case, 9, dtype)
        lens = O.lengths_for(case, lens, 9) if isinstance(lens, str) else lens
        lengths = torch.tensor(lens, dtype=torch.int32)
        k, v = O.poison_unread(k, v, table, lengths, page)
        dev = [x.cuda() for x in (q, k, v, table, lengths)]
        dname = "bfloat16" if dtype == torch.bfloat16 else "float16"
        expected = O.reference(q, k, v, table, lengths, page, causal)
        for splits in ((16,) if split_keys else (1, 4, 16, 64)):
            outs = {}
            if splits * 32 > width * page:
                continue
            for stages in (1, 2):
                kern = build_kernel(b, sq, h, d, k.shape[0], width, page, causal, dname, 0,
                                    num_splits=splits, layout="key", split_keys=split_keys,
                                    stages=stages)
                assert kern.stages == stages and kern.layout == "key", (name, stages)
                if name == "decode_kv8192" and splits == 64:
                    assert kern.compute_grid == (512 if stages == 1 else 256), kern.compute_grid
                outs[stages] = kern(*dev)
                if stages == 1 and splits > 1:  # the component calls run the same kernel
                    parts, lse = kern.partial_kernel(*dev)
                    merged = kern.merge_kernel(parts, lse, dev[4] if split_keys else None)
                    assert torch.equal(merged, outs[1]), f"{name} splits={splits} components"
            torch.cuda.synchronize()
            label = f"stages {name} splits={splits}"
            log(label)
            check_output(outs[1], expected, q, lengths, causal, label)
            assert torch.equal(outs[1], outs[2]), f"{label}: the two kernels differ in bits"


def test_headline_shapes():
    from fgw_amd.operators.mha.current import build_kernel
    for (b, sq, h, d, p, kv) in ((1, 1, 1, 128, 128, 512), (2, 4096, 8, 128, 128, 2048),
                                  (2, 1, 8, 128, 128, 32768), (2, 16, 8, 128, 128, 32768)):
        q, k, v, table, lengths = O.bench_inputs(b, sq, h, d, p, kv, torch.bfloat16)
        kern = build_kernel(b, sq, h, d, k.shape[0], kv // p, p, False, "bfloat16", 0,
                            full_kv_cache=True)
        got = kern(*(x.cuda() for x in (q, k, v, table, lengths)))
        torch.cuda.synchronize()
        expected = O.chunked_reference(q, k, v, table, lengths, p, False, 128)
        r = check_output(got, expected, q, lengths, False, f"B{b} Q{sq} H{h} KV{kv}")
        log(f"B{b} Q{sq} H{h} KV{kv}: splits={kern.num_splits} grid={kern.compute_grid} ratio={r:.3f}")



@pytest.mark.parametrize("page", [16, 64, 128])
def test_prefill_layout_long_ragged_cache(page):
    """The prefill layout over caches longer than its 64-block offset windows
    (window refresh), ragged lengths, page sizes that split blocks or not, and
    splits whose block ranges do not align with the windows."""
    from fgw_amd.operators.mha.current import build_kernel
    width = (8192 + page - 1) // page
    case = (f"long_p{page}", 2, 300, 4, 128, page, width)
    q, k, v, table = O.make_inputs(case, 2026, torch.bfloat16)
    lengths = torch.tensor([5000, 8192], dtype=torch.int32)
    k, v = O.poison_unread(k, v, table, lengths, page)
    dev = [x.cuda() for x in (q, k, v, table, lengths)]
    for causal in (False, True):
        expected = O.chunked_reference(q, k, v, table, lengths, page, causal, 128)
        for splits in (1, 3):
            kern = build_kernel(2, 300, 4, 128, k.shape[0], width, page, causal, "bfloat16", 0,
                                num_splits=None if splits == 1 else 4, layout="prefill",
                                persistent_programs=None if splits == 1 else 5)
            got = kern(*dev)
            torch.cuda.synchronize()
            check_output(got, expected, q, lengths, causal,
                         f"prefill long page={page} causal={causal} splits={kern.num_splits}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("dim", [64, 128])
def test_prefill_layout_every_block_count(dim, dtype):
    """The prefill layout's main loops run four 64-key blocks per iteration
    and the rest through a general body: requests of 0 to 11 blocks (a partial
    last block included) take every path, from no block at all through each
    remainder of the unrolled loop, against the oracle; split 2 halves them.
    Persistent grids of 1 and 3 programs run the items back to back, so that
    every program prefetches its next item's Q rows from each of those paths
    and stores a whole-tile item's output rows once the next item's first
    block has landed (296 rows: a second tile of 40 rows, whose waves hold
    32, 8 or no rows; causal: the tiles in reverse order, with rows that see
    no key): bit-identical to one program per item."""
    from fgw_amd.operators.mha.current import build_kernel
    page = 64
    lens = [0, 1, 64, 65, 130, 192, 256, 300, 384, 448, 512, 600, 640, 704]
    width = (max(lens) + page - 1) // page
    name = "bfloat16" if dtype == torch.bfloat16 else "float16"
    for sq, causal in ((256, False), (296, False), (296, True)):
        case = (f"blocks_d{dim}_q{sq}", len(lens), sq, 1, dim, page, width)
        q, k, v, table = O.make_inputs(case, 3, dtype)
        lengths = torch.tensor(lens, dtype=torch.int32)
        k, v = O.poison_unread(k, v, table, lengths, page)
        dev = [x.cuda() for x in (q, k, v, table, lengths)]
        expected = O.reference(q, k, v, table, lengths, page, causal)
        for splits in (None, 2):
            first = None
            for persistent in (None, 1, 3):
                kern = build_kernel(len(lens), sq, 1, dim, k.shape[0], width, page, causal, name,
                                    0, num_splits=splits, layout="prefill",
                                    persistent_programs=persistent)
                assert kern.layout == "prefill"
                got = kern(*dev)
                torch.cuda.synchronize()
                label = (f"prefill blocks {name} d={dim} sq={sq} causal={causal} "
                         f"splits={kern.num_splits} grid={kern.compute_grid}")
                check_output(got, expected, q, lengths, causal, label)
                if first is None:
                    first = got
                else:
                    assert torch.equal(got, first), f"{label}: the grid changed the output"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("dim,page", [(64, 32), (96, 16), (128, 128)])
def test_prefill_layout_dtypes_and_dims(dtype, dim, page):
    """The prefill layout for both input dtypes, both head-dim tiles (64, 128)
    and a padded head dim (96: every block on the per-key path), a partial
    last query tile, ragged lengths, causal and split."""
    from fgw_amd.operators.mha.current import build_kernel
    width = (1500 + page - 1) // page
    case = (f"prefill_d{dim}_p{page}", 2, 520, 2, dim, page, width)
    q, k, v, table = O.make_inputs(case, 11, dtype)
    lengths = torch.tensor([1500, 611], dtype=torch.int32)
    k, v = O.poison_unread(k, v, table, lengths, page)
    dev = [x.cuda() for x in (q, k, v, table, lengths)]
    for causal in (False, True):
        expected = O.reference(q, k, v, table, lengths, page, causal)
        for splits in (None, 2):
            kern = build_kernel(2, 520, 2, dim, k.shape[0], width, page, causal,
                                "float16" if dtype == torch.float16 else "bfloat16", 0,
                                num_splits=splits, layout="prefill")
            assert kern.layout == "prefill"
            got = kern(*dev)
            torch.cuda.synchronize()
            check_output(got, expected, q, lengths, causal,
                         f"prefill d={dim} page={page} causal={causal} splits={kern.num_splits}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rise", [48.0, 96.0])
def test_rising_scores_move_the_exponent_reference(dtype, rise):
    """Scores that rise along the keys make every 64-key block raise the row
    maximum by about 10 (rise 48: p up to ~2^10 against the previous exponent
    reference, under the sum bound) or about 20 log2 units (rise 96: the
    rescale path -- row maximum, O/l rescale, P recomputed -- runs on every
    block), in every layout."""
    from fgw_amd.operators.mha.current import build_kernel
    page, width, sq = 64, 24, 300
    case = ("rising", 2, sq, 2, 128, page, width)
    q, k, v, table = O.make_inputs(case, 5, dtype)
    q = (q.float().abs() * 0.5 + 0.25).to(dtype)  # positive queries
    ramp = torch.linspace(0.0, rise, k.shape[0])[:, None, None]
    k = (k.float().abs() * 0.1 + ramp).to(dtype)  # pool row r: scores grow with r
    # Table pages in pool order, so scores rise with the key position too.
    table = torch.arange(2 * width, dtype=torch.int32).reshape(2, width)
    lengths = torch.tensor([1500, 977], dtype=torch.int32)
    dev = [x.cuda() for x in (q, k, v, table, lengths)]
    for causal in (False, True):
        expected = O.reference(q, k, v, table, lengths, page, causal)
        for layout in ("query", "key", "prefill"):
            kern = build_kernel(2, sq, 2, 128, k.shape[0], width, page, causal,
                                "float16" if dtype == torch.float16 else "bfloat16", 0,
                                layout=layout)
            got = kern(*dev)
            torch.cuda.synchronize()
            check_output(got, expected, q, lengths, causal, f"rising {layout} causal={causal}")
