"""Static KV-block schedules: the reference's known answers and invariants.

The known answers are those of the reference's CPU tests
(tests/mha/test_static_schedule.py:11-140) at its 28 programs; coverage and
ownership are checked by brute force. The GPU tests run the static-schedule
kernels against the CPU oracle.
"""
import ctypes
from collections import Counter

import pytest
import torch

from fgw_amd.operators.mha import static_schedule as S


def units(plan):
    return Counter((tile, k) for segs in plan.programs for tile, first, count, _ in segs
                   for k in range(first, first + count))


def test_whole_q_plans():  # test_static_schedule.py:12-20
    for q in (1, 17, 129, 3712, 32768):
        plan = S.make_q_plan(q, 512, 28)
        assert not plan.merges and plan.partial_count == 0
        tiles = [tile for segs in plan.programs for tile, _, _, _ in segs]
        assert tiles == list(range((q + 127) // 128))
        assert all(first == 0 and count == 4 and slot == -1
                   for segs in plan.programs for _, first, count, slot in segs)


def test_coverage_and_unique_ownership():  # :113-128
    for q in (1, 17, 128, 129, 257):
        for kv in (128, 256, 512, 1024):
            for cores in (1, 2, 7, 28, 300):
                for plan in (S.make_plan(q, kv, cores), S.make_stream_plan(q, kv, cores),
                             S.make_tail_plan(q, kv, cores)):
                    seen = units(plan)
                    assert set(seen) == {(t, k) for t in range((q + 127) // 128)
                                         for k in range(kv // 128)}
                    assert all(n == 1 for n in seen.values())
                    S.validate_plan(plan)


def test_balanced_target_shapes():  # :130-138
    plan = S.make_plan(8192, 32768, 28)
    assert (plan.partial_count, len(plan.merges)) == (54, 27)
    d = plan.describe()
    assert (d["min_kv_blocks"], d["max_kv_blocks"]) == (585, 586)
    for q in (3584, 7168, 17920, 28672):
        plan = S.make_plan(q, 32768, 28)
        assert (plan.partial_count, len(plan.merges)) == (0, 0)
        assert plan.describe()["min_kv_blocks"] == plan.describe()["max_kv_blocks"]


def test_tail_wave():  # :96-108
    for kv in (4096, 8192):
        plan = S.make_tail_plan(32768, kv, 28)
        assert (len(plan.merges), plan.partial_count) == (4, 28)
        assert {tile for tile, _, _ in plan.merges} == set(range(252, 256))
        d = plan.describe()
        assert d["direct_q_tiles"] == 252 and d["max_kv_blocks"] - d["min_kv_blocks"] <= 1
    for q in (1, 129, 3584, 3712, 4096, 8192, 32768):
        for kv in (128, 256, 512, 4096, 8192):
            for pieces in (None, 2, 4, 7):
                S.validate_plan(S.make_tail_plan(q, kv, 28, pieces))


def test_one_cut_tile_on_two_programs():  # :140-144
    for plan in (S.make_plan(257, 512, 2), S.make_tail_plan(257, 512, 2),
                 S.make_stream_plan(257, 512, 2)):
        assert len(plan.merges) == 1


def test_choosers_give_valid_plans():
    for q in (1, 128, 257, 3712, 8192, 32768):
        for kv in (512, 2048, 32768):
            for plan in (S.choose_plan(q, kv, 64), S.choose_stream_plan(q, kv, 64)):
                S.validate_plan(plan)
                assert len(plan.programs) <= 64
    # the stream chooser splits only when that saves more than one block
    for q, kv in ((128, 512), (16384, 1024), (64, 32768)):
        plan = S.choose_stream_plan(q, kv)
        gain = (S.estimate_cost(S.make_q_plan(q, kv))["total_us"]
                - S.estimate_cost(plan)["total_us"])
        assert (gain > S.COST_MODEL["block_us"]) == bool(plan.merges)


@pytest.mark.parametrize("args,message", [
    ((0, 512), "positive integer Q"), ((128, 100), "128-aligned KV"),
    ((128, 512, 0), "cores must be"), ((128, 512, S.MAX_CORES + 1), "cores must be")])
def test_argument_checks(args, message):
    with pytest.raises(ValueError, match=message):
        S.make_plan(*args)


def test_validate_rejects_broken_plans():
    plan = S.make_plan(257, 512, 2)
    progs = list(plan.programs)
    progs[0] = progs[0][:-1]  # drop a segment: a tile is no longer covered
    with pytest.raises(AssertionError):
        S.validate_plan(S.Plan(plan.q, plan.kv, tuple(progs), plan.merges, plan.partial_count))


# ---- the static-schedule kernel path --------------------------------------

@pytest.mark.parametrize("kwargs,message", [
    (dict(fused_output=True), "fused_output experiment requires rawsimd"),
    (dict(plan_policy="q"), "plan_policy must be"),
    (dict(merge_policy="x"), "merge_policy must be"),
    (dict(merge_programs=30), "merge_programs must be 28 or 56"),
    (dict(merge_policy="grouped", merge_rows=16), "grouped comparison requires original R8"),
    (dict(merge_rows=4), "merge_rows must be 8, 16 or 32"),
    (dict(plan_policy="cost", programs=4), "explicit programs require balanced policy"),
])
def test_static_build_checks(kwargs, message):
    from fgw_amd.operators.mha.kernels.mha_static_host_hip import build_kernel
    with pytest.raises(ValueError, match=message):
        build_kernel(512, 1024, 1024, device_index=0, **kwargs)


def test_static_pool_check():
    from fgw_amd.operators.mha.kernels.mha_static_host_hip import build_kernel
    with pytest.raises(ValueError, match="whole physical pool pages"):
        build_kernel(512, 1024, 1000, programs=4, device_index=0)
    with pytest.raises(ValueError, match="whole physical pool pages"):
        build_kernel(512, 1024, 896, programs=4, device_index=0)


def test_static_abi_rejects_bad_schedules():
    from fgw_amd import _lib
    lib = _lib.load()
    shape = _lib.Shape(1, 512, 1, 128, 1024, 8, 128, 0, _lib.DTYPE_BFLOAT16)
    t = _lib.Tensors(16, 32, 48, 64, 80, 96, 112, 128)
    rc = lib.fgw_mha_static_local(ctypes.byref(shape), ctypes.byref(t), None, None)
    assert rc == _lib.FGW_MHA_EINVAL and b"schedule is NULL" in lib.fgw_mha_last_error()
    sched = _lib.Schedule(16, 32, None, 4, 0, 0, 100)
    rc = lib.fgw_mha_static_local(ctypes.byref(shape), ctypes.byref(t), ctypes.byref(sched), None)
    assert rc == _lib.FGW_MHA_EINVAL and b"block_keys" in lib.fgw_mha_last_error()
    sched = _lib.Schedule(16, 32, None, 4, 1, 2, 128)
    rc = lib.fgw_mha_static_merge(ctypes.byref(shape), ctypes.byref(t), ctypes.byref(sched), None)
    assert rc == _lib.FGW_MHA_EINVAL and b"merges" in lib.fgw_mha_last_error()
    sched = _lib.Schedule(16, 32, None, 0, 0, 0, 128)
    rc = lib.fgw_mha_static_local(ctypes.byref(shape), ctypes.byref(t), ctypes.byref(sched), None)
    assert rc == _lib.FGW_MHA_EINVAL and b"programs" in lib.fgw_mha_last_error()
    sched = _lib.Schedule(16, 32, None, 4, 0, 0, 128)  # no merges: nothing to launch
    assert lib.fgw_mha_static_merge(ctypes.byref(shape), ctypes.byref(t), ctypes.byref(sched),
                                    None) == 0


def _static_inputs(sq, kv, seed):
    g = torch.Generator().manual_seed(seed)
    width = kv // 128
    pages = width + 2
    table = torch.randperm(pages, generator=g)[:width].to(torch.int32)[None]
    q = torch.randn(1, sq, 1, 128, generator=g).bfloat16()
    k = torch.randn(pages * 128, 1, 128, generator=g).bfloat16()
    v = torch.randn(pages * 128, 1, 128, generator=g).bfloat16()
    lengths = torch.tensor([kv], dtype=torch.int32)
    return q, k, v, table, lengths


STATIC_CASES = [
    (1, 512, "balanced", None), (129, 512, "balanced", 2), (257, 1024, "tail", 2),
    (257, 1024, "balanced", 28), (1000, 2048, "cost", None), (3712, 4096, "tail", 28),
    (4096, 2048, "stream", None), (4096, 2048, "balanced", 100), (8192, 1024, "balanced", None),
]


@pytest.mark.gpu
@pytest.mark.parametrize("sq,kv,policy,programs", STATIC_CASES)
def test_static_path_matches_oracle(sq, kv, policy, programs):
    from fgw_amd.operators.mha.kernels.mha_static_host_hip import build_kernel
    from oracle import mha_oracle as O
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    q, k, v, table, lengths = _static_inputs(sq, kv, sq + kv)
    pool = k.shape[0]
    launch = build_kernel(sq, kv, pool, plan_policy=policy, programs=programs, device_index=0)
    print(f"static {policy} programs={programs} sq={sq} kv={kv}: "
          f"{launch.plan.describe()}", flush=True)
    dev = [x.cuda() for x in (q, k, v, table, lengths)]
    launch.validate_inputs(*dev)
    got = launch(*dev)
    torch.cuda.synchronize()
    expected = (O.chunked_reference if sq > 256 else O.reference)(
        q, k, v, table, lengths, 128, False)
    rtol, atol = O.TOLERANCES[torch.bfloat16]
    torch.testing.assert_close(got.cpu(), expected, rtol=rtol, atol=atol)
    # the two phases on their own give the same result
    parts, lse, out = launch.compute(*dev)
    assert (parts is None) == (not launch.plan.merges)
    again = launch.finish(parts, lse, out)
    torch.cuda.synchronize()
    assert torch.equal(again.cpu(), got.cpu())


@pytest.mark.gpu
def test_fused_static_path_matches_oracle():
    from fgw_amd.operators.mha.kernels.mha_static_host_hip import build_fused_kernel
    from oracle import mha_oracle as O
    from fgw_amd.operators.mha.current import build_kernel
    for sq, kv in ((64, 4096), (3712, 2048), (16384, 1024), (1024, 1024)):
        q, k, v, table, lengths = _static_inputs(sq, kv, 7 + sq)
        dev = [x.cuda() for x in (q, k, v, table, lengths)]
        expected = (O.chunked_reference if sq > 256 else O.reference)(
            q, k, v, table, lengths, 128, False)
        rtol, atol = O.TOLERANCES[torch.bfloat16]
        for fallback in (False, True):
            launch = build_fused_kernel(sq, kv, k.shape[0], 0, fallback=fallback)
            want = "static" if not fallback or S.static_preferred(sq, kv) else "automatic"
            assert launch.execution == want, (sq, kv, fallback)
            print(f"fused static sq={sq} kv={kv} fallback={fallback}: {launch.execution} "
                  f"{launch.plan.describe()}", flush=True)
            got = launch(*dev)
            parts, lse, out = launch.compute(*dev)
            again = launch.finish(parts, lse, out)
            torch.cuda.synchronize()
            torch.testing.assert_close(got.cpu(), expected, rtol=rtol, atol=atol)
            assert torch.equal(again, got)
            if launch.execution == "automatic":  # the main entry's own call, same bits
                auto = build_kernel(1, sq, 1, 128, k.shape[0], kv // 128, 128, False, "bfloat16",
                                    0, full_kv_cache=True)
                assert torch.equal(got, auto(*dev))


def test_static_fallback_follows_the_calibration():
    """build_fused_kernel keeps the static plan exactly where the committed
    MI355X static scan measured it >= 1.02x as fast as the automatic split
    (at calibrated shapes; elsewhere the nearest one decides)."""
    records = S.static_calibration()
    assert len(records) >= 70
    for q, kv, auto_us, static_us in records:
        assert S.static_preferred(q, kv) == (auto_us >= S.STATIC_MIN_SPEEDUP * static_us), (q, kv)
    assert S.static_preferred(1024, 1024) and S.static_preferred(16384, 1024)
    assert not S.static_preferred(4096, 2048) and not S.static_preferred(64, 32768)
    assert S.static_preferred(1152, 1152) == S.static_preferred(1024, 1024)  # nearest shape


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
def test_static_c_entries_general_tasks(dtype):
    """The C entries take any B, H, D and dtype: task t = (b H + h) q_tiles + q tile.
    A balanced plan over all tasks (cut tiles included), against the oracle."""
    from fgw_amd import _lib
    from fgw_amd.operators.mha.kernels.mha_paged_decode_hip import _current_stream
    from oracle import mha_oracle as O
    lib = _lib.load()
    b, sq, h, d, page, width = 2, 300, 3, 64, 32, 24
    case = ("static_general", b, sq, h, d, page, width)
    q, k, v, table = O.make_inputs(case, 5, dtype)
    lengths = torch.tensor([width * page, 517], dtype=torch.int32)
    k, v = O.poison_unread(k, v, table, lengths, page)
    q_tiles = (sq + 127) // 128
    tasks = b * h * q_tiles
    plan = S.make_plan(tasks * 128, width * page // 128 * 128, 7)
    segs, offsets = [], [0]
    for program in plan.programs:
        segs.extend(program)
        offsets.append(len(segs))
    dev = torch.device("cuda", 0)
    t_segs = torch.tensor(segs, dtype=torch.int32, device=dev)
    t_off = torch.tensor(offsets, dtype=torch.int32, device=dev)
    t_mer = torch.tensor(list(plan.merges) or [(-1, -1, -1)], dtype=torch.int32, device=dev)
    dq, dk, dv, dt, dl = (x.to(dev) for x in (q, k, v, table, lengths))
    out = torch.empty_like(dq)
    slots = plan.partial_count
    parts = torch.empty(max(1, slots) * 128 * d, dtype=torch.float32, device=dev)
    lse = torch.empty(max(1, slots) * 128, dtype=torch.float32, device=dev)
    shape = _lib.Shape(b, sq, h, d, k.shape[0], width, page, 0,
                       _lib.DTYPE_BFLOAT16 if dtype == torch.bfloat16 else _lib.DTYPE_FLOAT16)
    tens = _lib.Tensors(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dt.data_ptr(), dl.data_ptr(),
                        out.data_ptr(), parts.data_ptr(), lse.data_ptr())
    sched = _lib.Schedule(t_segs.data_ptr(), t_off.data_ptr(), t_mer.data_ptr(),
                          len(plan.programs), len(plan.merges), slots, 128)
    print(f"static C entries: tasks={tasks} {plan.describe()}", flush=True)
    stream = _current_stream(0)
    _lib.check(lib.fgw_mha_static_local(ctypes.byref(shape), ctypes.byref(tens),
                                        ctypes.byref(sched), stream))
    _lib.check(lib.fgw_mha_static_merge(ctypes.byref(shape), ctypes.byref(tens),
                                        ctypes.byref(sched), stream))
    torch.cuda.synchronize()
    assert plan.merges  # the plan cuts tiles across programs
    expected = O.chunked_reference(q, k, v, table, lengths, page, False)
    rtol, atol = O.TOLERANCES[dtype]
    torch.testing.assert_close(out.cpu(), expected, rtol=rtol, atol=atol)
