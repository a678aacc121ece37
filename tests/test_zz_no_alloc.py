"""fgw_mha_fwd_noalloc: the forward without a caller workspace (MI355X only).

Called through the C ABI, twice in a row (the second call smaller than the
first, so it runs over what the first left in the static scratch), and
compared bit for bit with fgw_mha_fwd on a caller-allocated workspace, and
with the oracle at the reference tolerances. A plan whose workspace exceeds
the scratch is rejected before any launch; a direct plan needs no scratch.
"""
import ctypes

import pytest
import torch

from fgw_amd import _lib
from oracle import mha_oracle as O

pytestmark = pytest.mark.gpu


def _plan(b, sq, h, d, page, kv, dtype, splits):
    width = kv // page
    shape = _lib.Shape(b, sq, h, d, b * width * page, width, page, 0,
                       _lib.DTYPE_BFLOAT16 if dtype == torch.bfloat16 else _lib.DTYPE_FLOAT16)
    plan = _lib.plan(shape, _lib.Request(splits, -1, -1), _lib.query_device(0))
    return shape, plan


def _call(entry, shape, plan, inputs, workspace):
    q, k, v, table, lengths = inputs
    out = torch.empty_like(q)
    parts = lse = None
    if workspace is not None:
        parts = workspace.data_ptr()
        lse = parts + 4 * plan.parts_floats
    t = _lib.Tensors(q.data_ptr(), k.data_ptr(), v.data_ptr(), table.data_ptr(),
                     lengths.data_ptr(), out.data_ptr(), parts, lse)
    rc = getattr(_lib.load(), entry)(ctypes.byref(shape), ctypes.byref(plan), ctypes.byref(t),
                                     torch.cuda.current_stream().cuda_stream)
    _lib.check(rc)
    return out


def test_noalloc_matches_the_workspace_entry_on_two_calls():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    torch.cuda.set_device(0)
    # (B, Sq, H, D, page, KV, dtype, splits): the second call is smaller.
    for b, sq, h, d, page, kv, dtype, splits in ((2, 16, 8, 128, 128, 8192, torch.bfloat16, 16),
                                                 (1, 1, 2, 64, 64, 1024, torch.float16, 4)):
        label = f"noalloc B{b} Q{sq} H{h} D{d} page{page} KV{kv} {dtype} splits={splits}"
        print(label, flush=True)
        host = O.bench_inputs(b, sq, h, d, page, kv, dtype)
        inputs = [x.cuda() for x in host]
        shape, plan = _plan(b, sq, h, d, page, kv, dtype, splits)
        assert plan.num_splits == splits and plan.execution_mode == 1, label
        assert 4 * (plan.parts_floats + plan.lse_floats) <= _lib.NOALLOC_SCRATCH_BYTES
        ws = torch.empty(plan.parts_floats + plan.lse_floats, dtype=torch.float32, device="cuda")
        want = _call("fgw_mha_fwd", shape, plan, inputs, ws)
        got = _call("fgw_mha_fwd_noalloc", shape, plan, inputs, None)
        torch.cuda.synchronize()
        assert torch.equal(got, want), label
        expected = O.chunked_reference(*host, page, False, 128)
        rtol, atol = O.TOLERANCES[dtype]
        torch.testing.assert_close(got.cpu(), expected, rtol=rtol, atol=atol,
                                   msg=lambda m: f"{label}: {m}")


def test_noalloc_direct_plan_and_oversize_rejection():
    torch.cuda.set_device(0)
    host = O.bench_inputs(1, 4, 2, 128, 128, 512, torch.bfloat16)
    inputs = [x.cuda() for x in host]
    shape, plan = _plan(1, 4, 2, 128, 128, 512, torch.bfloat16, 1)
    got = _call("fgw_mha_fwd_noalloc", shape, plan, inputs, None)
    want = _call("fgw_mha_fwd", shape, plan, inputs, None)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    # 2 x 8 x 8 splits x 4096 rows x 128 fp32 partials: 256 MiB, over the scratch.
    big_shape, big_plan = _plan(2, 4096, 8, 128, 128, 2048, torch.bfloat16, 8)
    assert 4 * (big_plan.parts_floats + big_plan.lse_floats) > _lib.NOALLOC_SCRATCH_BYTES
    q = torch.empty(2, 4096, 8, 128, dtype=torch.bfloat16, device="cuda")
    kv = torch.empty(big_shape.pool_rows, 8, 128, dtype=torch.bfloat16, device="cuda")
    meta = (torch.zeros(2, 16, dtype=torch.int32, device="cuda"),
            torch.zeros(2, dtype=torch.int32, device="cuda"))
    with pytest.raises(ValueError, match="static scratch"):
        _call("fgw_mha_fwd_noalloc", big_shape, big_plan, (q, kv, kv) + meta, None)
