"""Fused split merge: the last work item of each (b, h, q tile) merges its
splits inside the partial kernel (MI355X only; key layout, Sq <= 2, at most
16 splits, where it measured level with or faster than a second launch).

fgw_mha_fwd with arrival counters launches the partial kernel alone; its
output must equal, bit for bit, the two-launch path (partial_kernel then
merge_kernel, the same arithmetic), on two calls in a row (the counters return
to zero), and match the oracle at the reference tolerances. Cases cover the
double- and single-stage key-layout kernels, 2 to 16 splits,
length-balanced plans, causal and ragged lengths with empty requests, both
dtypes and head dims 32 to 256.
"""
import ctypes

import pytest
import torch

from fgw_amd import _lib
from oracle import mha_oracle as O

pytestmark = pytest.mark.gpu

CASES = [
    # name, B, Sq, H, D, page, KV, dtype, causal, lengths, splits, layout, extra
    ("q1_s16_single_stage", 2, 1, 8, 128, 128, 8192, torch.bfloat16, False, "full", 16, "key",
     {"stages": 1}),
    ("q1_s16_ragged", 3, 1, 4, 128, 64, 4096, torch.float16, False, (4096, 1000, 0), 16, "key",
     {}),
    ("q2_s8_causal", 2, 2, 4, 64, 64, 4096, torch.bfloat16, True, (4000, 37), 8, "key", {}),
    ("q1_s8", 2, 1, 8, 128, 128, 4096, torch.float16, False, (4096, 2000), 8, "key", {}),
    ("q2_s4_d48", 2, 2, 2, 48, 48, 960, torch.float16, False, (960, 500), 4, "key", {}),
    ("q1_s16_d256", 1, 1, 2, 256, 256, 8192, torch.bfloat16, False, "full", 16, "key", {}),
    ("balanced_q1", 4, 1, 8, 128, 128, 8192, torch.bfloat16, False, (8192, 100, 4000, 0), 16,
     "key", {"split_keys": 491}),
    ("q1_d32_s8", 2, 1, 4, 32, 32, 1024, torch.float16, False, (1024, 333), 8, "key", {}),
    ("q2_d32_s2_causal", 2, 2, 2, 32, 32, 4096, torch.bfloat16, True, (4096, 10), 2, "key", {}),
]


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    torch.cuda.set_device(0)


def _inputs(name, b, sq, h, d, page, kv, dtype, lengths):
    width = kv // page
    case = (name, b, sq, h, d, page, width)
    q, k, v, table = O.make_inputs(case, 5, dtype)
    lens = [kv] * b if lengths == "full" else list(lengths)
    lt = torch.tensor(lens, dtype=torch.int32)
    k, v = O.poison_unread(k, v, table, lt, page)
    return (q, k, v, table, lt), width


@pytest.mark.parametrize("name,b,sq,h,d,page,kv,dtype,causal,lengths,splits,layout,extra", CASES,
                         ids=[c[0] for c in CASES])
def test_fused_merge_equals_the_two_launch_path(name, b, sq, h, d, page, kv, dtype, causal,
                                                lengths, splits, layout, extra):
    from fgw_amd.operators.mha.current import build_kernel
    host, width = _inputs(name, b, sq, h, d, page, kv, dtype, lengths)
    dev = [x.cuda() for x in host]
    kern = build_kernel(b, sq, h, d, host[1].shape[0], width, page, causal,
                        "float16" if dtype == torch.float16 else "bfloat16", 0,
                        num_splits=splits, layout=layout, **extra)
    label = f"{name}: splits {kern.num_splits} layout {kern.layout} stages {kern.stages}"
    print(label, flush=True)
    assert kern.execution_mode == "split_and_merge" and kern.merge_fused, label
    first = kern(*dev)
    second = kern(*dev)  # the counters the first call used are back at zero
    parts, lse = kern.partial_kernel(*dev)
    two_launch = kern.merge_kernel(parts, lse, dev[4])
    torch.cuda.synchronize()
    assert torch.equal(first, two_launch), label
    assert torch.equal(second, two_launch), label
    expected = O.reference(*host, page, causal)
    rtol, atol = O.TOLERANCES[dtype]
    torch.testing.assert_close(first.cpu(), expected, rtol=rtol, atol=atol,
                               msg=lambda m: f"{label}: {m}")


@pytest.mark.parametrize("name,b,sq,h,d,page,kv,splits,layout", [
    ("query_layout", 2, 4, 2, 128, 128, 2048, 4, "query"),
    ("q4_more_rows", 2, 4, 4, 128, 128, 2048, 8, "key"),
    ("s32_more_splits", 2, 1, 4, 128, 128, 8192, 32, "key"),
    ("d32_s16_chunk", 2, 1, 4, 32, 32, 2048, 16, "key"),
])
def test_plans_outside_the_fused_rule_merge_in_a_second_launch(name, b, sq, h, d, page, kv, splits,
                                                                 layout):
    """The query layout, Sq > 2, more than 16 splits and the 16-split chunk
    at head-dim tile 32 keep the second launch, and are still correct."""
    from fgw_amd.operators.mha.current import build_kernel
    host, width = _inputs(name, b, sq, h, d, page, kv, torch.bfloat16, "full")
    dev = [x.cuda() for x in host]
    kern = build_kernel(b, sq, h, d, host[1].shape[0], width, page, True, "bfloat16", 0,
                        num_splits=splits, layout=layout)
    assert kern.execution_mode == "split_and_merge" and not kern.merge_fused, name
    got = kern(*dev)
    parts, lse = kern.partial_kernel(*dev)
    assert torch.equal(got, kern.merge_kernel(parts, lse)), name
    rtol, atol = O.TOLERANCES[torch.bfloat16]
    torch.testing.assert_close(got.cpu(), O.reference(*host, page, True), rtol=rtol, atol=atol)


def _c_call(shape, plan, dev, out, ws, arrivals):
    q, k, v, table, lengths = dev
    parts = ws.data_ptr()
    t = _lib.Tensors(q.data_ptr(), k.data_ptr(), v.data_ptr(), table.data_ptr(),
                     lengths.data_ptr(), out.data_ptr(), parts, parts + 4 * plan.parts_floats,
                     None if arrivals is None else arrivals.data_ptr())
    _lib.check(_lib.load().fgw_mha_fwd(ctypes.byref(shape), ctypes.byref(plan), ctypes.byref(t),
                                       torch.cuda.current_stream().cuda_stream))


def test_c_abi_fused_call_leaves_its_counters_at_zero():
    """Through the C ABI: fgw_mha_fwd with caller counters (one launch) twice
    in a row, the second on a smaller batch of the same buffer; the counters
    are zero after each call and the outputs equal the call without counters
    (two launches)."""
    dev_info = _lib.query_device(0)
    for b, sq, h, d, page, kv, splits in ((2, 1, 8, 128, 128, 8192, 16), (1, 2, 4, 64, 64, 2048, 8)):
        host, width = _inputs("c_abi", b, sq, h, d, page, kv, torch.bfloat16, "full")
        dev = [x.cuda() for x in host]
        shape = _lib.Shape(b, sq, h, d, host[1].shape[0], width, page, 0, _lib.DTYPE_BFLOAT16)
        plan = _lib.plan(shape, _lib.Request(splits, -1, _lib.LAYOUT_KEY), dev_info)
        label = f"C ABI B{b} Q{sq} H{h} D{d} KV{kv} splits {plan.num_splits}"
        print(label, flush=True)
        assert plan.arrival_counters == 32 * plan.query_tile_tasks > 0, label
        arrivals = torch.zeros(plan.arrival_counters, dtype=torch.int32, device="cuda")
        ws = torch.empty(plan.parts_floats + plan.lse_floats, dtype=torch.float32, device="cuda")
        fused = torch.empty_like(dev[0])
        plain = torch.empty_like(dev[0])
        _c_call(shape, plan, dev, fused, ws, arrivals)
        torch.cuda.synchronize()
        assert torch.count_nonzero(arrivals).item() == 0, label
        _c_call(shape, plan, dev, plain, ws, None)
        torch.cuda.synchronize()
        assert torch.equal(fused, plain), label


def test_noalloc_graph_replays_with_static_counters():
    """fgw_mha_fwd_noalloc fuses the merge with its static counters and needs
    no allocation, so it can be captured: each replay equals the eager
    workspace call bit for bit (the static counters return to zero every
    replay)."""
    b, sq, h, d, page, kv, splits = 2, 1, 8, 128, 128, 4096, 16
    host, width = _inputs("noalloc_graph", b, sq, h, d, page, kv, torch.bfloat16, "full")
    dq, dk, dv, dt, dl = (x.cuda() for x in host)
    shape = _lib.Shape(b, sq, h, d, host[1].shape[0], width, page, 0, _lib.DTYPE_BFLOAT16)
    plan = _lib.plan(shape, _lib.Request(splits, -1, _lib.LAYOUT_KEY), _lib.query_device(0))
    assert 0 < plan.arrival_counters <= _lib.NOALLOC_ARRIVALS
    out = torch.empty_like(dq)
    t = _lib.Tensors(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dt.data_ptr(), dl.data_ptr(),
                     out.data_ptr(), None, None, None)
    lib = _lib.load()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up outside capture
        _lib.check(lib.fgw_mha_fwd_noalloc(ctypes.byref(shape), ctypes.byref(plan),
                                           ctypes.byref(t), side.cuda_stream))
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _lib.check(lib.fgw_mha_fwd_noalloc(ctypes.byref(shape), ctypes.byref(plan),
                                           ctypes.byref(t),
                                           torch.cuda.current_stream().cuda_stream))
    ws = torch.empty(plan.parts_floats + plan.lse_floats, dtype=torch.float32, device="cuda")
    gen = torch.Generator().manual_seed(23)
    for rep in range(3):
        dq.copy_(torch.randn(dq.shape, generator=gen).to(torch.bfloat16))
        eager = torch.empty_like(dq)
        _c_call(shape, plan, (dq, dk, dv, dt, dl), eager, ws, None)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep} differs from the eager call"
    expected = O.reference(dq.cpu(), *host[1:], page, False)
    rtol, atol = O.TOLERANCES[torch.bfloat16]
    torch.testing.assert_close(out.cpu(), expected, rtol=rtol, atol=atol)
