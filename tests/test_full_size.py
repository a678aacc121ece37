"""The benchmark configurations at their full sizes (MI355X only).

At Q32768/KV2048 (B2 H8 D128 BF16) the oracle runs on sampled query rows:
without a causal mask every output row depends on its own Q row only, so the
oracle over a row subset of Q is the exact reference for those rows. The
size-independent property: moving every page to another slot of the pool
(and the block table with it) leaves the output bit-identical, since the
kernels accumulate in logical key order whatever the physical placement.
"""
import pytest
import torch

from oracle import mha_oracle as O

pytestmark = pytest.mark.gpu


def _permute_pages(k, v, table, page, seed):
    """Pool with page p moved to slot perm[p]; the table follows the move."""
    pages = k.shape[0] // page
    perm = torch.randperm(pages, generator=torch.Generator().manual_seed(seed))
    k2, v2 = torch.empty_like(k), torch.empty_like(v)
    k2.view(pages, page, *k.shape[1:])[perm] = k.view(pages, page, *k.shape[1:])
    v2.view(pages, page, *v.shape[1:])[perm] = v.view(pages, page, *v.shape[1:])
    return k2, v2, perm.to(torch.int32)[table.long()]


@pytest.mark.parametrize("b,sq,h,kv", [(2, 32768, 8, 2048), (2, 1, 8, 32768), (2, 4096, 8, 2048)])
def test_full_size_rows_and_page_placement(b, sq, h, kv):
    from fgw_amd.operators.mha.current import build_kernel
    page, d = 128, 128
    q, k, v, table, lengths = O.bench_inputs(b, sq, h, d, page, kv, torch.bfloat16)
    kern = build_kernel(b, sq, h, d, k.shape[0], kv // page, page, False, "bfloat16", 0,
                        full_kv_cache=True)
    print(f"full size B{b} Q{sq} H{h} KV{kv}: layout={kern.layout} splits={kern.num_splits} "
          f"grid={kern.compute_grid}", flush=True)
    dq, dl = q.cuda(), lengths.cuda()
    got = kern(dq, k.cuda(), v.cuda(), table.cuda(), dl)
    k2, v2, table2 = _permute_pages(k, v, table, page, seed=sq + kv)
    moved = kern(dq, k2.cuda(), v2.cuda(), table2.cuda(), dl)
    torch.cuda.synchronize()
    assert torch.equal(got, moved), "output depends on the physical page placement"
    got = got.cpu()
    gen = torch.Generator().manual_seed(kv)
    rows = torch.cat([torch.arange(min(sq, 64)), torch.arange(max(0, sq - 64), sq),
                      torch.randint(0, sq, (128,), generator=gen)]).unique()
    expected = O.chunked_reference(q[:, rows].contiguous(), k, v, table, lengths, page, False, 128)
    rtol, atol = O.TOLERANCES[torch.bfloat16]
    torch.testing.assert_close(got[:, rows], expected, rtol=rtol, atol=atol)


@pytest.mark.parametrize("sq,layout", [(1, None), (16, None), (96, "query"), (1024, None)])
def test_pages_beyond_4_gib_into_the_pool(sq, layout):
    """64-bit pool addressing: the same pages placed more than 4 GiB (K and V
    each) into a large pool, the table shifted with them, give the same bits
    as in a small pool; decode (key layout), query and prefill layouts. The
    rest of the large pool is never written (uninitialised memory the
    kernels must not read)."""
    from fgw_amd.operators.mha.current import build_kernel
    b, h, d, page, kv = 2, 8, 128, 128, 4096
    q, k, v, table, lengths = O.bench_inputs(b, sq, h, d, page, kv, torch.bfloat16)
    rows = k.shape[0]
    row_bytes = h * d * 2
    shift_pages = -(-(9 << 29) // (page * row_bytes))  # 4.5 GiB of rows, whole pages
    shift = shift_pages * page
    dq, dl = q.cuda(), lengths.cuda()
    small = build_kernel(b, sq, h, d, rows, kv // page, page, False, "bfloat16", 0,
                         full_kv_cache=True, layout=layout)
    want = small(dq, k.cuda(), v.cuda(), table.cuda(), dl)
    big_k = torch.empty(shift + rows, h, d, dtype=torch.bfloat16, device="cuda")
    big_v = torch.empty_like(big_k)
    big_k[shift:].copy_(k)
    big_v[shift:].copy_(v)
    big = build_kernel(b, sq, h, d, shift + rows, kv // page, page, False, "bfloat16", 0,
                       full_kv_cache=True, layout=layout)
    print(f"pool offset {shift * row_bytes / 2**30:.2f} GiB: Sq{sq} layout={big.layout} "
          f"splits={big.num_splits}", flush=True)
    assert (big.layout, big.num_splits) == (small.layout, small.num_splits)
    got = big(dq, big_k, big_v, (table + shift_pages).cuda(), dl)
    torch.cuda.synchronize()
    assert shift * row_bytes > 4 << 30
    assert torch.equal(got, want), "output depends on the pool offset"
    del big_k, big_v
    torch.cuda.empty_cache()
