"""Packed K/V cache (the reference's external_cache_gather path).

CPU: the product's host layout against the oracle's, and the argument checks.
GPU: fgw_mha_pack_pages bit-exact against the oracle's page copy (NaN rows
included), zero pages for ids outside the pool, and attention over the packed
cache against the oracle on the original paged inputs.
"""
import ctypes

import pytest
import torch

from fgw_amd.operators.mha import packed_cache as P
from oracle import mha_oracle as O
from tests import mha_cases as C


@pytest.mark.parametrize("lengths,page,width", [
    ([0, 1, 128, 129, 300], 128, 3), ([5, 0, 0, 7], 4, 2), ([0], 16, 1), ([64] * 3, 64, 1)])
def test_layout_matches_oracle(lengths, page, width):
    offsets, rows, table = P.packed_layout(lengths, page, width)
    o_offsets, o_rows, o_table = O.packed_offsets(lengths, page, width)
    assert offsets == o_offsets and rows == o_rows and table == o_table.tolist()


def test_checks_run_before_any_device_work():
    k = torch.zeros(8, 2, 16, dtype=torch.bfloat16)
    table = torch.zeros(2, 2, dtype=torch.int32)
    with pytest.raises(ValueError, match="same GPU"):
        P.pack_paged_cache(k, k.clone(), table, [1, 2], 4)
    with pytest.raises(ValueError, match="K/V shape mismatch"):
        P.pack_paged_cache(k, k[:4], table, [1, 2], 4)
    with pytest.raises(ValueError, match="int32 metadata"):
        P.pack_paged_cache(k, k.clone(), table.long(), [1, 2], 4)
    with pytest.raises(ValueError, match="whole pool pages"):
        P.pack_paged_cache(k, k.clone(), table, [1, 2], 3)
    with pytest.raises(ValueError, match="FP16/BF16"):
        P.pack_paged_cache(k.float(), k.float(), table, [1, 2], 4)
    with pytest.raises(ValueError, match="metadata shape mismatch"):
        P._host_lengths([1, 2, 3], 2, 8)
    with pytest.raises(ValueError, match="within table capacity"):
        P._host_lengths([1, 9], 2, 8)
    with pytest.raises(ValueError, match="host-known lengths"):
        P._host_lengths(torch.zeros(2, dtype=torch.int32, device="meta"), 2, 8)


PACK_CASES = ("tiny", "general_d48_page48", "many_queries", "page256", "split_d16_q1",
              "non_power_two_dim")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
def test_pack_bit_exact(dtype):
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    for name in PACK_CASES:
        case = C.ALL_CASES[name]
        _, b, sq, h, d, p, w = case
        for pattern in C.PATTERNS:
            q, k, v, table = O.make_inputs(case, 11, dtype)
            lengths = O.lengths_for(case, pattern, 11)
            k, v = O.poison_unread(k, v, table, torch.tensor(lengths), p)
            print(f"pack {name} {dtype} {pattern} lengths={lengths}", flush=True)
            packed = P.pack_paged_cache(k.cuda(), v.cuda(), table.cuda(), lengths, p)
            torch.cuda.synchronize()
            ek, ev, offsets = O.pack_pages(k, v, table, lengths, p)
            assert packed.offsets == offsets and packed.rows == ek.shape[0]
            assert packed.cu_rows.cpu().tolist() == offsets
            torch.testing.assert_close(packed.k.cpu(), ek, rtol=0, atol=0, equal_nan=True)
            torch.testing.assert_close(packed.v.cpu(), ev, rtol=0, atol=0, equal_nan=True)


@pytest.mark.gpu
def test_pack_zero_pages_for_ids_outside_the_pool():
    g = torch.Generator().manual_seed(5)
    page, h, d = 16, 2, 64
    k = torch.randn(4 * page, h, d, generator=g).bfloat16()
    v = torch.randn(4 * page, h, d, generator=g).bfloat16()
    table = torch.tensor([[2, -1, 9], [1, 0, 3]], dtype=torch.int32)
    packed = P.pack_paged_cache(k.cuda(), v.cuda(), table.cuda(), [40, 33], page)
    torch.cuda.synchronize()
    pk = packed.k.cpu()
    assert packed.offsets == [0, 48, 96]
    assert torch.equal(pk[0:16], k[32:48])
    assert torch.count_nonzero(pk[16:48]) == 0  # ids -1 and 9 are outside the 4-page pool
    assert torch.equal(pk[48:64], k[16:32]) and torch.equal(pk[80:96], k[48:64])


@pytest.mark.gpu
@pytest.mark.parametrize("name,causal,splits", [
    ("tiny", False, None), ("many_queries", True, None), ("page256", False, 4),
    ("general_d48_page48", False, 2)])
def test_gather_attention_matches_paged_attention(name, causal, splits):
    from fgw_amd.operators.mha import current
    case = C.ALL_CASES[name]
    _, b, sq, h, d, p, w = case
    dtype = torch.bfloat16
    q, k, v, table = O.make_inputs(case, 3, dtype)
    lengths = O.lengths_for(case, "mixed", 3)
    lt = torch.tensor(lengths, dtype=torch.int32)
    k, v = O.poison_unread(k, v, table, lt, p)
    inputs = tuple(x.cuda() for x in (q, k, v, table, lt))
    print(f"gather attention {name} causal={causal} splits={splits} lengths={lengths}", flush=True)
    combined, info = P.build_gather_attention(
        (name, b, sq, h, d, p, w, lengths, causal), "bfloat16", inputs, current, splits, 0)
    assert info["live_rows"] == sum(lengths) and info["packed_rows"] == combined.packed_rows
    assert info["gather_accuracy"] == "exact_passed"
    # The packed rows, row-exact against the pool pages (external_cache_gather.py:55-64).
    dense_k, dense_v = combined.pack()
    ek, ev, offsets = O.pack_pages(k, v, table, lengths, p)
    live = offsets[-1]
    torch.testing.assert_close(dense_k[:live].cpu(), ek[:live], rtol=0, atol=0, equal_nan=True)
    torch.testing.assert_close(dense_v[:live].cpu(), ev[:live], rtol=0, atol=0, equal_nan=True)
    got = combined()
    torch.cuda.synchronize()
    expected = O.reference(q, k, v, table, lt, p, causal)
    rtol, atol = O.TOLERANCES[dtype]
    torch.testing.assert_close(got.cpu(), expected, rtol=rtol, atol=atol)


def test_packed_row_check_on_host_tensors():
    """check_packed_rows (the reference helper's row-exact check,
    external_cache_gather.py:55-64) accepts the oracle's packing, NaN rows and
    zero pages for ids outside the pool included, and names the request of a
    single flipped bit."""
    g = torch.Generator().manual_seed(9)
    page, h, d = 16, 2, 32
    k = torch.randn(5 * page, h, d, generator=g).bfloat16()
    v = torch.randn(5 * page, h, d, generator=g).bfloat16()
    k[3 * page + 2, 1, 5] = float("nan")
    table = torch.tensor([[3, 2, 0], [1, 0, 4]], dtype=torch.int32)
    lengths = [40, 20]
    ek, ev, offsets = O.pack_pages(k, v, table, lengths, page)
    plan = P._PackPlan(offsets, ek.shape[0], None, None, offsets[-1] // page)
    P.check_packed_rows(k, v, table, plan, page, ek, ev)
    # Page ids -1 and 9 lie outside the 5-page pool: their packed pages are zero.
    outside = torch.tensor([[3, -1, 9], [1, 0, 4]], dtype=torch.int32)
    zk, zv = ek.clone(), ev.clone()
    zk[page:3 * page] = 0
    zv[page:3 * page] = 0
    P.check_packed_rows(k, v, outside, plan, page, zk, zv)
    with pytest.raises(AssertionError, match="K rows of request 0"):
        P.check_packed_rows(k, v, outside, plan, page, ek, ev)
    bad = ev.clone()
    bad.view(torch.int16)[offsets[1] + 3, 0, 7] ^= 1
    with pytest.raises(AssertionError, match="V rows of request 1"):
        P.check_packed_rows(k, v, table, plan, page, ek, bad)
