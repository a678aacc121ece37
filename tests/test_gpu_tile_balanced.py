"""Tile-balanced causal splits of the prefill layout against the CPU oracle
(MI355X only): each 256-row query tile takes clamp(ceil(visible keys at
capacity / split_keys), 1, num_splits) work items and the merge reads each
tile's own slot count. Ragged and short lengths (empty rows), NaN in every
unread pool row, both dtypes, head dims on the fast and the per-key path, the
merge of one workgroup per row (more than 16 slots) and persistent grids.
"""
import pytest
import torch

from oracle import mha_oracle as O
from tests.test_gpu_parity import check_output

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dim,page", [(64, 64), (96, 16), (128, 128)])
def test_tile_balanced_causal_matches_the_oracle(dtype, dim, page):
    from fgw_amd.operators.mha.current import build_kernel
    b, sq, h = 2, 700, 3
    width = (1500 + page - 1) // page
    case = (f"tiles_d{dim}_p{page}", b, sq, h, dim, page, width)
    q, k, v, table = O.make_inputs(case, 5, dtype)
    lengths = torch.tensor([1500, 611], dtype=torch.int32)  # 611 < Sq: empty rows
    k, v = O.poison_unread(k, v, table, lengths, page)
    dev = [x.cuda() for x in (q, k, v, table, lengths)]
    expected = O.reference(q, k, v, table, lengths, page, True)
    name = "float16" if dtype == torch.float16 else "bfloat16"
    outs = []
    for splits, split_keys, persistent in ((4, 256, "device"), (4, 256, 5), (32, 64, "device"),
                                           (2, 1024, None)):
        kern = build_kernel(b, sq, h, dim, k.shape[0], width, page, True, name, 0,
                            num_splits=splits, split_keys=split_keys, layout="prefill",
                            persistent_programs=persistent)
        assert kern.split_balance == "tile" and kern.layout == "prefill"
        label = (f"tile-balanced d={dim} page={page} {name} splits={splits} "
                 f"split_keys={split_keys} persistent={persistent} work={kern.compute_work}")
        print(label, flush=True)
        got = kern(*dev)
        torch.cuda.synchronize()
        check_output(got, expected, q, lengths, True, label)
        outs.append((splits, split_keys, got.cpu()))
    # Work placement never changes the arithmetic of a work item.
    assert torch.equal(outs[0][2], outs[1][2])


def test_tile_balanced_components_equal_the_full_call():
    from fgw_amd.operators.mha.current import build_kernel
    b, sq, h, dim, page, kv = 1, 1000, 4, 128, 128, 2048
    width = kv // page
    case = ("tiles_parts", b, sq, h, dim, page, width)
    q, k, v, table = O.make_inputs(case, 9, torch.bfloat16)
    lengths = torch.tensor([kv], dtype=torch.int32)
    dev = [x.cuda() for x in (q, k, v, table, lengths)]
    kern = build_kernel(b, sq, h, dim, k.shape[0], width, page, True, "bfloat16", 0,
                        num_splits=8, split_keys=512, layout="prefill")
    full = kern(*dev)
    parts, lse = kern.partial_kernel(*dev)
    merged = kern.merge_kernel(parts, lse)
    torch.cuda.synchronize()
    assert torch.equal(full, merged)
    check_output(full.cpu(), O.chunked_reference(q, k, v, table, lengths, page, True, 128), q,
                 lengths, True, "tile-balanced components")


def test_automatic_tile_balanced_plan():
    # Causal self-attention in 64 query tiles of 256..4096 visible keys: the planner
    # picks a tile-balanced plan by itself.
    from fgw_amd.operators.mha.current import build_kernel
    b, sq, h, dim, page = 1, 4096, 4, 128, 128
    width = sq // page
    case = ("tiles_auto", b, sq, h, dim, page, width)
    q, k, v, table = O.make_inputs(case, 13, torch.bfloat16)
    lengths = torch.tensor([sq], dtype=torch.int32)
    kern = build_kernel(b, sq, h, dim, k.shape[0], width, page, True, "bfloat16", 0,
                        full_kv_cache=True)
    assert kern.layout == "prefill" and kern.split_balance == "tile" and kern.split_keys > 0
    got = kern(*(x.cuda() for x in (q, k, v, table, lengths)))
    torch.cuda.synchronize()
    check_output(got.cpu(), O.chunked_reference(q, k, v, table, lengths, page, True, 128), q,
                 lengths, True, f"automatic tile-balanced plan splits={kern.num_splits} "
                                f"split_keys={kern.split_keys}")
