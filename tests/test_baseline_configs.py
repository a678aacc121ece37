"""GPU parity over the benchmark configurations' own grids (MI355X only).

- Config 2, the short-Q grid: B1 H1 D128 BF16, page 128, full cache,
  shuffled table, Q {1..512} x KV {128..16384}; every spec as one direct
  kernel (split 1), with the automatic split and with a forced split + merge.
- Config 4, split-KV decode: B2 H8 D128 page 128, Q {1, 16} x KV
  {512, 2048, 8192, 32768}, FP16 and BF16, at the automatic split and at
  splits 1/2/4/8/16/32 (benchmarks/mha/bench_v7_split_scan.py:88-120); and the
  imbalanced B4 variant, lengths drawn uniformly in [KV/8, KV] (seeded), at
  every KV.
- Config 5, generalised edges: D {16, 32, 64, 128, 256} x page {16, 64, 128},
  FP16 and BF16, Q {1, 7, 64} causal and not, ragged lengths 1000 and 4099
  and an empty cache in one batch, B {1, 3}, H {1, 8}.

Inputs follow the benchmark recipe (bench_mha_mfu.py:179-188) or the accuracy
recipe with NaN in every unread pool row (test_mha_paged_accuracy.py:
232-238); outputs are compared with the oracle at the reference tolerances,
rows with no visible key must be exactly zero.
"""
import pytest
import torch

from oracle import mha_oracle as O
from tests.test_gpu_parity import check_output, log

pytestmark = pytest.mark.gpu

GRID_Q = (1, 2, 4, 8, 16, 32, 64, 128, 256, 512)
GRID_KV = (128, 256, 512, 1024, 2048, 4096, 8192, 16384)
DECODE_KV = (512, 2048, 8192, 32768)
DECODE_SPLITS = (None, 1, 2, 4, 8, 16, 32)


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    torch.cuda.set_device(0)


def _name(dtype):
    return "float16" if dtype == torch.float16 else "bfloat16"


def forced_split(kv):
    """A split + merge request every KV of the grid admits (2 .. 16)."""
    return max(2, min(16, kv // 256))


@pytest.mark.parametrize("sq", GRID_Q)
def test_config2_short_q_grid(sq):
    from fgw_amd.operators.mha.current import build_kernel
    for kv in GRID_KV:
        host = O.bench_inputs(1, sq, 1, 128, 128, kv, torch.bfloat16)
        dev = [x.cuda() for x in host]
        expected = O.chunked_reference(*host, 128, False, 128)
        for splits in (1, None, forced_split(kv)):
            kern = build_kernel(1, sq, 1, 128, host[1].shape[0], kv // 128, 128, False,
                                "bfloat16", 0, num_splits=splits, full_kv_cache=True)
            label = (f"config2 Q{sq} KV{kv} request={splits} -> splits={kern.num_splits} "
                     f"layout={kern.layout}")
            log(label)
            if splits is not None and splits > 1:
                assert kern.execution_mode == "split_and_merge", label
            got = kern(*dev)
            torch.cuda.synchronize()
            check_output(got, expected, host[0], host[4], False, label)


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
@pytest.mark.parametrize("sq", (1, 16))
@pytest.mark.parametrize("kv", DECODE_KV)
def test_config4_decode_split_scan(dtype, sq, kv):
    from fgw_amd.operators.mha.current import build_kernel
    host = O.bench_inputs(2, sq, 8, 128, 128, kv, dtype)
    dev = [x.cuda() for x in host]
    expected = O.chunked_reference(*host, 128, False, 128)
    for splits in DECODE_SPLITS:
        if splits is not None and splits > kv // 32:
            continue  # more splits than 32-token KV tiles is rejected (the scan skips it)
        kern = build_kernel(2, sq, 8, 128, host[1].shape[0], kv // 128, 128, False, _name(dtype),
                            0, num_splits=splits, full_kv_cache=True)
        label = f"config4 {dtype} Q{sq} KV{kv} request={splits} -> splits={kern.num_splits}"
        log(label)
        got = kern(*dev)
        torch.cuda.synchronize()
        check_output(got, expected, host[0], host[4], False, label)


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
@pytest.mark.parametrize("kv", DECODE_KV)
def test_config4_imbalanced_b4(dtype, kv):
    """B4, lengths uniform in [KV/8, KV] from Generator().manual_seed(7), table
    width KV / page; through the public entry (automatic split from the
    host-known ragged lengths) and at forced splits."""
    from fgw_amd.operators.mha.current import build_kernel, mha_paged_decode
    lengths = O.imbalanced_lengths(kv)
    for sq in (1, 16):
        q, k, v, table, _ = O.bench_inputs(4, sq, 8, 128, 128, kv, dtype)
        k, v = O.poison_unread(k, v, table, lengths, 128)
        dev = [x.cuda() for x in (q, k, v, table, lengths)]
        expected = O.chunked_reference(q, k, v, table, lengths, 128, False, 128)
        label = f"config4 imbalanced {dtype} Q{sq} KV{kv} lengths={lengths.tolist()}"
        log(label + " auto")
        got = mha_paged_decode(*dev, page_size=128)
        torch.cuda.synchronize()
        check_output(got, expected, q, lengths, False, label + " auto")
        for splits in (1, 4, 16):
            kern = build_kernel(4, sq, 8, 128, k.shape[0], kv // 128, 128, False, _name(dtype), 0,
                                num_splits=splits)
            log(f"{label} splits={splits}")
            got = kern(*dev)
            torch.cuda.synchronize()
            check_output(got, expected, q, lengths, False, f"{label} splits={splits}")


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
@pytest.mark.parametrize("dim", (16, 32, 64, 128, 256))
@pytest.mark.parametrize("page", (16, 64, 128))
def test_config5_general_edges(dtype, dim, page):
    from fgw_amd.operators.mha.current import mha_paged_decode
    width = (4099 + page - 1) // page
    for b, h, lens in ((3, 8, [1000, 4099, 0]), (1, 1, [4099])):
        lengths = torch.tensor(lens, dtype=torch.int32)
        for sq, causal in ((1, False), (1, True), (7, True), (64, True), (64, False)):
            case = (f"config5_d{dim}_p{page}", b, sq, h, dim, page, width)
            q, k, v, table = O.make_inputs(case, 2026, dtype)
            k, v = O.poison_unread(k, v, table, lengths, page)
            dev = [x.cuda() for x in (q, k, v, table, lengths)]
            label = (f"config5 {dtype} D{dim} page{page} B{b} H{h} Q{sq} causal={causal} "
                     f"lengths={lens}")
            log(label)
            got = mha_paged_decode(*dev, page_size=page, is_causal=causal)
            torch.cuda.synchronize()
            expected = O.reference(q, k, v, table, lengths, page, causal)
            check_output(got, expected, q, lengths, causal, label)
