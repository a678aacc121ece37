"""Runtime-shape family (operators/mha/runtime_lengths.py in the reference).

CPU tests cover the build-time and call-time checks, which run before any
device work; the GPU test runs one family over several query lengths, pool
sizes and table widths against the CPU oracle with the reference tolerances.
"""
import pytest
import torch

from fgw_amd.operators.mha.runtime_lengths import build_runtime_kernel
from oracle import mha_oracle as O


@pytest.mark.parametrize("args,message", [
    ((2, 1, 4), "Runtime candidate requires B1H1"),
    ((1, 8, 4), "Runtime candidate requires B1H1"),
    ((1, 1, 3), "Runtime candidate requires B1H1"),
    ((1, 1, 32), "Runtime candidate requires B1H1"),
])
def test_build_checks(args, message):
    with pytest.raises(ValueError, match=message):
        build_runtime_kernel(*args)


def test_merge_rows_check():
    with pytest.raises(ValueError, match="merge_rows must be 1/2/4/8"):
        build_runtime_kernel(1, 1, 4, merge_rows=3)


def test_family_key():
    call = build_runtime_kernel(1, 1, 4, merge_rows=2, device_index=0)
    assert call.family_key == (1, 1, 4, 2, 0)
    assert build_runtime_kernel(1, 1, 4, merge_rows=2, device_index=0) is call


def _cpu_inputs(sq=5, pages=4, width=4, dtype=torch.bfloat16):
    q = torch.zeros(1, sq, 1, 128, dtype=dtype)
    k = torch.zeros(pages * 128, 1, 128, dtype=dtype)
    table = torch.zeros(1, width, dtype=torch.int32)
    lengths = torch.zeros(1, dtype=torch.int32)
    return q, k, k.clone(), table, lengths


def test_call_checks_run_before_any_device_work():
    call = build_runtime_kernel(1, 1, 4)
    q, k, v, table, lengths = _cpu_inputs()
    with pytest.raises(ValueError, match="Expected BF16 Q"):
        call(q.half(), k, v, table, lengths)
    with pytest.raises(ValueError, match="Expected BF16 Q"):
        call(q[:, :0], k, v, table, lengths)
    with pytest.raises(ValueError, match="Expected BF16 Q"):
        call(torch.zeros(1, 5, 1, 64, dtype=torch.bfloat16), k, v, table, lengths)
    with pytest.raises(ValueError, match="Expected matching BF16 paged K/V"):
        call(q, k[:100], v[:100], table, lengths)
    with pytest.raises(ValueError, match="Expected matching BF16 paged K/V"):
        call(q, k, v.half(), table, lengths)
    with pytest.raises(ValueError, match="sufficient split capacity"):
        call(q, k, v, table[:, :3], lengths)
    with pytest.raises(ValueError, match="sufficient split capacity"):
        call(q, k, v, table.long(), lengths)
    with pytest.raises(ValueError, match="same GPU"):
        call(q, k, v, table, lengths)


@pytest.mark.gpu
@pytest.mark.parametrize("splits", [1, 4, 16])
def test_runtime_family_parity(splits):
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    call = build_runtime_kernel(1, 1, splits)
    shapes = [(1, 16, 3), (16, 16, 0), (300, 24, 2), (1024, 16, 1), (1, 32, 0)]
    for sq, width, extra in shapes:
        g = torch.Generator().manual_seed(1000 * splits + sq + width)
        pages = width + extra
        table = torch.randperm(pages, generator=g)[:width].to(torch.int32)[None]
        capacity = width * 128
        lengths = torch.tensor([int(torch.randint(0, capacity + 1, (1,), generator=g))
                                if sq != 16 else capacity], dtype=torch.int32)
        q = torch.randn(1, sq, 1, 128, generator=g).bfloat16()
        k = torch.randn(pages * 128, 1, 128, generator=g).bfloat16()
        v = torch.randn(pages * 128, 1, 128, generator=g).bfloat16()
        k, v = O.poison_unread(k, v, table, lengths, 128)
        print(f"runtime family splits={splits} sq={sq} width={width} pool={pages * 128} "
              f"len={int(lengths[0])}", flush=True)
        got = call(*[x.cuda() for x in (q, k, v, table, lengths)])
        torch.cuda.synchronize()
        launch = call.program(sq, pages * 128, width)
        assert launch.num_splits == splits
        assert launch.execution_mode == ("direct_single_split" if splits == 1 else "split_and_merge")
        expected = (O.chunked_reference if sq > 256 else O.reference)(
            q, k, v, table, lengths, 128, False)
        got = got.cpu()
        assert got.shape == q.shape and got.dtype == torch.bfloat16
        assert torch.isfinite(got).all()
        rtol, atol = O.TOLERANCES[torch.bfloat16]
        torch.testing.assert_close(got, expected, rtol=rtol, atol=atol)
        if int(lengths[0]) == 0:
            assert torch.count_nonzero(got).item() == 0
