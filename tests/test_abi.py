"""C ABI and host logic, CPU only: the library loads, exports every declared
symbol, and its planner/validation behave as specified (no kernel launches)."""
import ctypes
import pathlib
import re

import pytest
import torch

from fgw_amd import _lib

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "fgw_mha.h"
# MI355X: 256 CUs; resident workgroups per CU of the query, key and prefill
# kernels (head-dim tile 128) and of the key layout's single-stage kernel.
DEVICE = _lib.DeviceInfo(256, (ctypes.c_int32 * _lib.NUM_LAYOUTS)(2, 1, 1), 1, 2)


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIBRARY.exists():
        from fgw_amd import build
        build.build(verbose=False)
    return _lib.load()


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(fgw_mha_\w+)\s*\(", text, flags=re.M)))


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert len(names) == 12, names
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.SIGNATURES)
    assert lib.fgw_mha_abi_version() == _lib.ABI_VERSION


def shape(b=2, sq=1, h=8, d=128, kv=32768, page=128, causal=0, dtype=_lib.DTYPE_BFLOAT16):
    width = (kv + page - 1) // page
    return _lib.Shape(b, sq, h, d, b * width * page, width, page, causal, dtype)


def test_cost_model_guard_matches_the_planner_layout(lib):
    # split_cost_model.planner_takes_prefill restates fgw_mha_plan's automatic
    # prefill-layout rule; the split cost model must never be used for shapes
    # the planner runs on the prefill kernel.
    from fgw_amd.operators.mha import split_cost_model as M
    wg = tuple(DEVICE.wg_per_cu)
    for b in (1, 2, 16):
        for h in (1, 8, 32):
            for sq in (1, 32, 33, 128, 129, 200, 255, 256, 384, 512, 1023, 1024, 4096):
                for d in (32, 64, 96, 128, 192):
                    for kv in (128, 1000, 2048, 8192, 65536):
                        p = _lib.plan(shape(b=b, h=h, sq=sq, d=d, kv=kv), _lib.Request(0, -1, -1), DEVICE)
                        width = (kv + 127) // 128
                        want = M.planner_takes_prefill(b, sq, h, d, DEVICE.num_cus, wg, width * 128)
                        assert (p.layout == 2) == want, (b, h, sq, d, kv)


def test_single_stage_rule_matches_the_planner(lib):
    # split_cost_model.single_stage_splits restates fgw_mha_plan's move of automatic
    # short-decode plans to the single-stage key kernel (the Python host applies it
    # to the cost model's split count).
    from fgw_amd.operators.mha import split_cost_model as M
    moved = 0
    for b in (1, 2, 4, 16):
        for h in (1, 4, 8, 32):
            for sq in (1, 4, 5, 16, 17):
                for d in (64, 128):
                    for kv in (1024, 4096, 8192, 32768, 65536):
                        s = shape(b=b, h=h, sq=sq, d=d, kv=kv)
                        fill = _lib.plan(s, _lib.Request(0, -1, -1, 0, 0 if d != 128 or sq > 32 else 2), DEVICE)
                        auto = _lib.plan(s, _lib.Request(0, -1, -1), DEVICE)
                        up = M.single_stage_splits(b, sq, h, d, kv, fill.num_splits, DEVICE.num_cus,
                                                   DEVICE.wg_per_cu_key_single)
                        want = (up, 1) if up else (fill.num_splits, fill.stages)
                        assert (auto.num_splits, auto.stages) == want, (b, h, sq, d, kv)
                        moved += bool(up)
    assert moved >= 10


def test_plan_headline_shapes(lib):
    # 2 x 8 x 16 prefill tiles of 256 rows fill the 256 CUs: prefill layout.
    prefill = _lib.plan(shape(sq=4096, kv=2048), _lib.Request(0, -1, -1), DEVICE)
    assert (prefill.layout, prefill.rows_per_tile, prefill.q_tiles, prefill.num_splits) == (2, 256, 16, 1)
    assert (prefill.work_items, prefill.grid, prefill.execution_mode) == (256, 256, 0)
    assert prefill.threads == 512
    mid = _lib.plan(shape(sq=128, kv=2048), _lib.Request(0, -1, -1), DEVICE)
    assert (mid.layout, mid.rows_per_tile, mid.threads) == (0, 128, 256)  # short Q: query layout
    # 64 prefill tiles, KV splits fill the device: prefill layout from Q 1024 (head-dim
    # tiles 64 and 128, causal or not), and for Q > 128 from 2^24 query-key pairs
    # (B x H x Sq x capacity); splits of at least 8 keys per task (512 here).
    few = _lib.plan(shape(sq=1024, kv=2048), _lib.Request(0, -1, -1), DEVICE)
    assert (few.layout, few.q_tiles, few.num_splits, few.work_items) == (2, 4, 4, 256)
    assert _lib.plan(shape(sq=512, kv=2048), _lib.Request(0, -1, -1), DEVICE).layout == 2
    assert _lib.plan(shape(sq=512, kv=1024), _lib.Request(0, -1, -1), DEVICE).layout == 0
    assert _lib.plan(shape(sq=129, kv=8192), _lib.Request(0, -1, -1), DEVICE).layout == 2
    assert _lib.plan(shape(sq=128, kv=32768), _lib.Request(0, -1, -1), DEVICE).layout == 0
    # Query layout: 4 key rounds (256 keys) per split from 2^22 pairs, else 2 rounds.
    q96 = _lib.plan(shape(sq=96, d=64, kv=4096), _lib.Request(0, -1, -1), DEVICE)
    assert (q96.layout, q96.num_splits) == (0, 16)  # 16 tasks; 32 splits would be 128 keys
    q64 = _lib.plan(shape(b=1, h=1, sq=64, kv=4096), _lib.Request(0, -1, -1), DEVICE)
    assert (q64.layout, q64.num_splits) == (0, 32)  # 2^18 pairs: 128 keys per split
    # 96 tasks: 768 keys per split at least, so KV 1024 stays unsplit (the fill
    # rule of 256 keys alone took 2 splits).
    tall = _lib.plan(shape(b=1, h=16, sq=1536, kv=1024), _lib.Request(0, -1, -1), DEVICE)
    assert (tall.layout, tall.q_tiles, tall.num_splits) == (2, 6, 1)
    assert _lib.plan(shape(sq=1024, kv=2048, causal=1), _lib.Request(0, -1, -1), DEVICE).layout == 2
    assert _lib.plan(shape(sq=1024, kv=2048, d=64), _lib.Request(0, -1, -1), DEVICE).layout == 2
    wide = _lib.plan(shape(sq=4096, kv=2048, d=256), _lib.Request(0, -1, -1), DEVICE)
    assert (wide.layout, wide.dim_padded) == (0, 256)  # no prefill kernel for D > 128
    narrow = _lib.plan(shape(sq=4096, kv=2048, d=32), _lib.Request(0, -1, -1), DEVICE)
    assert narrow.layout == 0
    # Decode: 16 double-stage splits fill the 256 CUs; the automatic plan moves to the
    # single-stage key kernel with 4x the splits (512 keys each), two programs per CU.
    decode = _lib.plan(shape(sq=1, kv=32768), _lib.Request(0, -1, -1), DEVICE)
    assert (decode.layout, decode.rows_per_tile, decode.num_splits, decode.work_items) == (1, 32, 64, 1024)
    assert (decode.stages, decode.grid) == (1, 512)
    assert decode.parts_floats == 2 * 8 * 64 * 1 * 128 and decode.lse_floats == 2 * 8 * 64
    fill = _lib.plan(shape(sq=1, kv=32768), _lib.Request(0, -1, -1, 0, 2), DEVICE)
    assert (fill.num_splits, fill.stages, fill.grid) == (16, 2, 256)
    big = _lib.plan(shape(sq=32768, kv=2048), _lib.Request(0, -1, -1), DEVICE)
    assert big.layout == 2 and big.work_items == 2 * 8 * 128
    assert big.grid == 256  # persistent cap = 256 CUs x 1 program
    uncapped = _lib.plan(shape(sq=32768, kv=2048), _lib.Request(0, 0, -1), DEVICE)
    assert uncapped.grid == uncapped.work_items
    capped = _lib.plan(shape(sq=32768, kv=2048), _lib.Request(0, 28, -1), DEVICE)
    assert capped.grid == 28
    # causal work items differ in size: the device request leaves one workgroup per item
    causal = _lib.plan(shape(sq=32768, kv=2048, causal=1), _lib.Request(0, -1, -1), DEVICE)
    assert causal.grid == causal.work_items == 2 * 8 * 128
    causal_capped = _lib.plan(shape(sq=32768, kv=2048, causal=1), _lib.Request(0, 28, -1), DEVICE)
    assert causal_capped.grid == 28


def test_plan_split_rules(lib):
    # Auto splits never leave a split with fewer than two rounds of key blocks.
    small = _lib.plan(shape(sq=1, kv=512), _lib.Request(0, -1, -1), DEVICE)
    assert small.num_splits == 2
    tiny = _lib.plan(shape(sq=1, kv=128), _lib.Request(0, -1, -1), DEVICE)
    assert tiny.num_splits == 1 and tiny.execution_mode == 0
    explicit = _lib.plan(shape(sq=16, kv=8192), _lib.Request(16, -1, -1), DEVICE)
    assert explicit.num_splits == 16 and explicit.execution_mode == 1
    forced = _lib.plan(shape(sq=64, kv=8192), _lib.Request(0, -1, _lib.LAYOUT_KEY), DEVICE)
    assert (forced.layout, forced.q_tiles) == (1, 2)
    pre = _lib.plan(shape(sq=64, kv=8192), _lib.Request(0, -1, _lib.LAYOUT_PREFILL), DEVICE)
    assert (pre.layout, pre.q_tiles, pre.rows_per_tile) == (2, 1, 256)
    with pytest.raises(ValueError, match="prefill layout"):
        _lib.plan(shape(sq=512, d=256), _lib.Request(0, -1, _lib.LAYOUT_PREFILL), DEVICE)
    for bad in (3, 256, -2):
        with pytest.raises(ValueError, match="num_splits"):
            _lib.plan(shape(), _lib.Request(bad, -1, -1), DEVICE)
    with pytest.raises(ValueError, match="KV tiles"):
        _lib.plan(shape(kv=128), _lib.Request(8, -1, -1), DEVICE)


def test_plan_length_balanced_splits(lib):
    """split_keys > 0: accepted for the key layout with >= 2 splits and B <= 1024,
    carried into the plan; rejected otherwise."""
    key = _lib.plan(shape(sq=1, kv=8192), _lib.Request(16, -1, _lib.LAYOUT_KEY, 600), DEVICE)
    assert (key.layout, key.num_splits, key.split_keys) == (_lib.LAYOUT_KEY, 16, 600)
    even = _lib.plan(shape(sq=1, kv=8192), _lib.Request(16, -1, _lib.LAYOUT_KEY), DEVICE)
    assert even.split_keys == 0 and even.work_items == key.work_items
    for req, s in ((_lib.Request(16, -1, _lib.LAYOUT_QUERY, 600), shape(sq=1, kv=8192)),
                   (_lib.Request(1, -1, _lib.LAYOUT_KEY, 600), shape(sq=1, kv=8192)),
                   (_lib.Request(16, -1, _lib.LAYOUT_KEY, -1), shape(sq=1, kv=8192))):
        with pytest.raises(ValueError, match="split_keys"):
            _lib.plan(s, req, DEVICE)
    big = shape(sq=1, kv=8192)
    big.batch = 1025
    big.pool_rows = 1025 * 8192
    with pytest.raises(ValueError, match="split_keys"):
        _lib.plan(big, _lib.Request(16, -1, _lib.LAYOUT_KEY, 600), DEVICE)


def test_plan_kernel_stages(lib):
    """Stages: the layout's default kernel unless requested. The key layout at
    head-dim tile 128 has a single-stage kernel (two workgroups per CU) beside
    its double-stage default; other kernels accept only their own count; the
    grid cap follows the selected kernel."""
    plan = lambda s, splits=0, stages=0: _lib.plan(  # noqa: E731
        s, _lib.Request(splits, -1, -1, 0, stages), DEVICE)
    for splits in (8, 16, 64):
        assert (plan(shape(), splits).stages, plan(shape(), splits).grid) == (2, min(16 * splits, 256))
    assert (plan(shape(), 64, 1).stages, plan(shape(), 64, 1).grid) == (1, 512)
    assert (plan(shape(), 8, 1).stages, plan(shape(), 8, 1).grid) == (1, 128)
    assert (plan(shape(), 64, 2).stages, plan(shape(), 64, 2).grid) == (2, 256)
    # A requested stage count keeps the fill's split count; only the automatic plan
    # moves to the single-stage kernel with more splits.
    assert plan(shape(), 0, 1).num_splits == plan(shape(), 0, 2).num_splits == 16
    assert (plan(shape()).num_splits, plan(shape()).stages) == (64, 1)
    # Other kernels have one stage count: accepted when requested, else refused.
    assert plan(shape(d=64)).stages == 2 and plan(shape(d=256)).stages == 1
    assert plan(shape(d=256), 0, 1).stages == 1
    assert plan(shape(sq=128, kv=2048), 0, 2).stages == 2  # query layout
    assert plan(shape(sq=4096, kv=2048)).stages == 4  # prefill rings
    for s, stages in ((shape(d=64), 1), (shape(d=256), 2), (shape(sq=128, kv=2048), 1),
                      (shape(sq=4096, kv=2048), 2), (shape(), 3)):
        with pytest.raises(ValueError, match="stages"):
            plan(s, 0, stages)
    # A plan with a stage count the kernel does not have is refused before any launch.
    bad = _lib.Plan.from_buffer_copy(plan(shape(), 16))
    bad.stages = 3
    s, t = shape(), _lib.Tensors(16, 32, 48, 64, 80, 96, 112, 128)
    rc = lib.fgw_mha_fwd(ctypes.byref(s), ctypes.byref(bad), ctypes.byref(t), None)
    assert rc == _lib.FGW_MHA_EINVAL and b"plan" in lib.fgw_mha_last_error()


@pytest.mark.parametrize("field,value,message", [
    ("dim", 24, "divisible by 16"),
    ("dim", 272, "D must be"),
    ("page_size", 0, "positive page size"),
    ("pool_rows", 1000, "whole pool pages"),
    ("dtype", 7, "FP16/BF16"),
    ("sq", 0, "positive Q extents"),
])
def test_plan_rejects_invalid_shapes(lib, field, value, message):
    s = shape()
    setattr(s, field, value)
    with pytest.raises(ValueError, match=message):
        _lib.plan(s, _lib.Request(0, -1, -1), DEVICE)


def test_fwd_rejects_null_and_misaligned_buffers(lib):
    s = shape(sq=4, kv=512)
    p = _lib.plan(s, _lib.Request(1, -1, -1), DEVICE)
    t = _lib.Tensors()
    rc = lib.fgw_mha_fwd(ctypes.byref(s), ctypes.byref(p), ctypes.byref(t), None)
    assert rc == _lib.FGW_MHA_EINVAL and b"NULL" in lib.fgw_mha_last_error()
    t = _lib.Tensors(16, 32, 48, 64, 80, 97, None, None)
    rc = lib.fgw_mha_fwd(ctypes.byref(s), ctypes.byref(p), ctypes.byref(t), None)
    assert rc == _lib.FGW_MHA_EINVAL and b"aligned" in lib.fgw_mha_last_error()
    p.grid = 0  # a plan that does not match the shape is rejected before any launch
    rc = lib.fgw_mha_fwd(ctypes.byref(s), ctypes.byref(p), ctypes.byref(t), None)
    assert rc == _lib.FGW_MHA_EINVAL and b"plan" in lib.fgw_mha_last_error()


def test_pack_rejects_bad_arguments_before_any_launch(lib):
    s = shape(sq=1, kv=512)
    t = _lib.Tensors()
    rc = lib.fgw_mha_pack_pages(ctypes.byref(s), ctypes.byref(t), 16, 1, 32, 48, None)
    assert rc == _lib.FGW_MHA_EINVAL and b"pack needs" in lib.fgw_mha_last_error()
    t = _lib.Tensors(None, 32, 48, 64, None, None, None, None)
    rc = lib.fgw_mha_pack_pages(ctypes.byref(s), ctypes.byref(t), 16, 1, 32, 49, None)
    assert rc == _lib.FGW_MHA_EINVAL and b"aligned" in lib.fgw_mha_last_error()
    rc = lib.fgw_mha_pack_pages(ctypes.byref(s), ctypes.byref(t), 16, -1, 32, 48, None)
    assert rc == _lib.FGW_MHA_EINVAL and b"total_pages" in lib.fgw_mha_last_error()
    # nothing to pack: no launch, success
    assert lib.fgw_mha_pack_pages(ctypes.byref(s), ctypes.byref(t), 16, 0, 32, 48, None) == 0


def test_public_validation_matches_reference_messages():
    from fgw_amd.operators.mha.current import build_kernel, mha_paged_decode
    q = torch.zeros(1, 1, 2, 16, dtype=torch.bfloat16)
    k = torch.zeros(32, 2, 16, dtype=torch.bfloat16)
    table = torch.zeros(1, 2, dtype=torch.int32)
    lengths = torch.zeros(1, dtype=torch.int32)
    cases = [
        ((q[0], k, k, table, lengths, 16), "expected Q\\[B,Sq,H,D\\]"),
        ((q, k[:, :1], k, table, lengths, 16), "K/V shape mismatch"),
        ((q, k, k, table[:, :0], lengths, 16), "metadata shape mismatch"),
        ((q.half(), k, k, table, lengths, 16), "matching FP16/BF16"),
        ((q, k, k, table.long(), lengths, 16), "int32 metadata"),
        ((q, k, k, table, lengths, 16), "same GPU"),  # CPU tensors
    ]
    for args, message in cases:
        with pytest.raises(ValueError, match=message):
            mha_paged_decode(*args)
    with pytest.raises(TypeError):
        mha_paged_decode(q, k, k, table, lengths, 16, cube_mode="general")
    with pytest.raises(ValueError, match="split_policy"):
        build_kernel(1, 1, 2, 16, 32, 2, 16, False, "bfloat16", 0, split_policy="fastest")
    with pytest.raises(ValueError, match="num_splits"):
        build_kernel(1, 1, 2, 16, 32, 2, 16, False, "bfloat16", 0, num_splits=3)
    with pytest.raises(ValueError, match="D must be"):
        build_kernel(1, 1, 2, 24, 32, 2, 16, False, "bfloat16", 0)


def test_launch_shim_loads_and_checks_its_arguments(lib):
    """The C++ launch callable (fgw_amd._launch) loads on the CPU, refuses
    buffers that are not the C ABI structs, and on a call refuses non-tensors
    and tensors that do not match its plan with the operator's messages,
    before any allocation or launch."""
    launch = _lib.load_launch_module()
    sh = shape(b=1, sq=4, h=2, d=64, kv=256, page=64)
    pl = _lib.plan(sh, _lib.Request(1, -1, -1), DEVICE)
    fwd, err = _lib.entry_address("fgw_mha_fwd"), _lib.entry_address("fgw_mha_last_error")
    with pytest.raises(TypeError, match="C ABI structs"):
        launch.Launcher(bytes(sh)[:-4], bytes(pl), 0, fwd, err)
    with pytest.raises(TypeError, match="function addresses"):
        launch.Launcher(bytes(sh), bytes(pl), 0, 0, err)
    call = launch.Launcher(bytes(sh), bytes(pl), 0, fwd, err)
    q = torch.zeros(1, 4, 2, 64, dtype=torch.bfloat16)
    kv = torch.zeros(sh.pool_rows, 2, 64, dtype=torch.bfloat16)
    table = torch.zeros(1, 4, dtype=torch.int32)
    lengths = torch.zeros(1, dtype=torch.int32)
    with pytest.raises(TypeError, match="expected"):
        call(q, kv, kv, table)
    with pytest.raises(TypeError, match="torch tensors"):
        call(q, kv, kv, table, 3)
    with pytest.raises(ValueError, match="tensor shapes"):
        call(q[:, :3], kv, kv, table, lengths)
    with pytest.raises(ValueError, match="matching FP16/BF16"):
        call(q.half(), kv, kv, table, lengths)
    with pytest.raises(ValueError, match="int32 metadata"):
        call(q, kv, kv, table.long(), lengths)
    with pytest.raises(ValueError, match="same GPU"):  # CPU tensors
        call(q, kv, kv, table, lengths)


def test_plan_tile_balanced_causal_splits(lib):
    # Prefill layout, causal: split_keys gives each 256-row query tile
    # clamp(ceil(visible keys at capacity / split_keys), 1, num_splits) work items.
    s = shape(b=2, h=8, sq=4096, kv=4096, causal=1)
    p = _lib.plan(s, _lib.Request(2, -1, 2, 2176), DEVICE)
    # tiles 0-7 see 256..2048 keys (one slot), tiles 8-15 see 2304..4096 (two)
    assert (p.layout, p.num_splits, p.split_keys, p.work_items) == (2, 2, 2176, 16 * (8 + 16))
    assert p.grid == p.work_items  # causal plans stay uncapped
    capped = _lib.plan(s, _lib.Request(2, 64, 2, 2176), DEVICE)
    assert capped.grid == 64 and capped.work_items == 384
    wide = _lib.plan(s, _lib.Request(32, -1, 2, 256), DEVICE)
    assert wide.work_items == 16 * sum(min(32, -(-256 * (t + 1) // 256)) for t in range(16))
    ragged = _lib.plan(shape(b=1, h=2, sq=300, kv=1000, causal=1), _lib.Request(4, -1, 2, 256),
                       DEVICE)
    # capacity 1024, Sq 300: tile 0 sees up to 980 keys (4 slots), tile 1 all 1024 (4)
    assert ragged.work_items == 2 * (4 + 4)
    for req, shp in ((_lib.Request(2, -1, 2, 256), shape(sq=4096, kv=4096)),  # not causal
                     (_lib.Request(1, -1, 2, 256), s),  # one split
                     (_lib.Request(2, -1, 0, 256), s)):  # query layout
        with pytest.raises(ValueError, match="split_keys"):
            _lib.plan(shp, req, DEVICE)


def test_plan_automatic_tile_balanced_causal_splits(lib):
    # Causal self-attention with at most half the device's programs in query tiles
    # of very different lengths: the planner cuts the long tiles.
    auto = _lib.plan(shape(b=1, h=8, sq=4096, kv=4096, causal=1), _lib.Request(0, -1, -1), DEVICE)
    # 1.5 x 278528 keys / 256 CUs = 1632 -> 1664 keys per item; the longest tile takes 3
    assert (auto.layout, auto.num_splits, auto.split_keys) == (2, 4, 1664)
    assert auto.work_items == 8 * sum(-(-256 * (t + 1) // 1664) for t in range(16))
    # Left alone: a prefix-cached shape (tiles of similar lengths), short tiles, and
    # as many tiles as half the programs and more.
    for s in (shape(b=1, h=8, sq=1024, kv=8192, causal=1), shape(b=1, h=32, sq=1024, kv=1024, causal=1),
              shape(b=1, h=16, sq=4096, kv=4096, causal=1), shape(b=1, h=8, sq=4096, kv=4096)):
        assert _lib.plan(s, _lib.Request(0, -1, -1), DEVICE).split_keys == 0
    # An explicit split count keeps even splits.
    assert _lib.plan(shape(b=1, h=8, sq=4096, kv=4096, causal=1), _lib.Request(2, -1, -1),
                     DEVICE).split_keys == 0


def test_cost_model_plans_receive_host_lengths_causal_or_not():
    """An explicit cost_model call plans with the host lengths whether or not
    it is causal (v7_experimental.py:885-886); 'auto' forwards them only for
    non-causal calls; full caches and explicit split counts never."""
    from fgw_amd.operators.mha.kernels.mha_paged_decode_hip import planning_lengths
    ragged = [100, 3000]
    assert planning_lengths(ragged, False, None, "cost_model", True) == (100, 3000)
    assert planning_lengths(ragged, False, None, "cost_model", False) == (100, 3000)
    assert planning_lengths(ragged, False, None, "auto", False) == (100, 3000)
    assert planning_lengths(ragged, False, None, "auto", True) is None
    assert planning_lengths(ragged, False, None, "legacy", False) is None
    assert planning_lengths(ragged, False, 4, "cost_model", True) is None
    assert planning_lengths([4096, 4096], True, None, "cost_model", False) is None


def test_cost_model_with_an_explicit_layout_keeps_that_layout(lib, monkeypatch):
    """The cost model's move to the single-stage kernel applies to the key
    layout only: with layout='query' or 'prefill' the plan keeps the layout's
    own kernel instead of requesting a stage count the planner refuses."""
    from fgw_amd.operators.mha.kernels import mha_paged_decode_hip as K
    monkeypatch.setattr(K, "_device_info", lambda index: DEVICE)
    kv = 32768
    args = (2, 1, 8, 128, 2 * kv, kv // 128, 128, False, "bfloat16", 0)
    auto = K.build_kernel(*args, split_policy="cost_model", full_kv_cache=True)
    assert auto.layout == "key" and auto.stages == 1
    for layout in ("query", "key"):
        kern = K.build_kernel(*args, split_policy="cost_model", full_kv_cache=True, layout=layout)
        assert kern.layout == layout
        assert kern.stages == (1 if layout == "key" else 2)
    sq = 512  # the prefill layout needs Sq > 128 to be worth asking for; any Sq plans
    pre = K.build_kernel(2, sq, 8, 128, 2 * kv, kv // 128, 128, False, "bfloat16", 0,
                         split_policy="cost_model", full_kv_cache=True, layout="prefill")
    assert pre.layout == "prefill"


def test_plan_fused_merge_counters(lib):
    """arrival_counters: the split plans whose merge fgw_mha_fwd fuses (key
    layout, Sq <= 2, at most 16 splits; at most 8 at head-dim tile 32) carry
    one 128-byte counter line (32 int32) per task; others carry none."""
    def plan(req, **kw):
        return _lib.plan(shape(**kw), req, DEVICE)
    key, line = _lib.LAYOUT_KEY, 32
    assert plan(_lib.Request(16, -1, key)).arrival_counters == 16 * line  # B2 H8 Q1
    assert plan(_lib.Request(8, -1, key), sq=2).arrival_counters == 16 * line
    assert plan(_lib.Request(1, -1, key)).arrival_counters == 0
    assert plan(_lib.Request(32, -1, key)).arrival_counters == 0
    assert plan(_lib.Request(8, -1, key), sq=3).arrival_counters == 0
    assert plan(_lib.Request(8, -1, key), d=32).arrival_counters == 16 * line
    assert plan(_lib.Request(16, -1, key), d=32).arrival_counters == 0
    assert plan(_lib.Request(16, -1, key), d=64).arrival_counters == 16 * line
    assert plan(_lib.Request(4, -1, _lib.LAYOUT_QUERY), sq=2).arrival_counters == 0
    assert plan(_lib.Request(4, -1, _lib.LAYOUT_PREFILL), sq=4096, kv=2048).arrival_counters == 0


def test_fwd_rejects_a_plan_with_other_arrival_counters(lib):
    sh = shape(b=2, sq=1, h=8, d=128, kv=8192)
    p = _lib.plan(sh, _lib.Request(16, -1, _lib.LAYOUT_KEY), DEVICE)
    assert p.arrival_counters == 16 * 32
    p.arrival_counters = 16
    t = _lib.Tensors()
    rc = lib.fgw_mha_fwd(ctypes.byref(sh), ctypes.byref(p), ctypes.byref(t), None)
    assert rc == _lib.FGW_MHA_EINVAL
    assert b"plan does not match" in lib.fgw_mha_last_error()
