"""HIP graph capture of the launch callables (MI355X only).

One call of each path is captured into a graph. Before every replay Q is
rewritten in place and the eager call runs on the same inputs, with device
synchronisations in between; each replay must equal the eager output bit for
bit (the same kernels on the same data), and the last one must match the
oracle. This covers the split workspaces and the merge kernel under capture
(graph-pool allocations reused across replays) and that no launch path
synchronises or records a memset.
"""
import pytest
import torch

from oracle import mha_oracle as O

pytestmark = pytest.mark.gpu

CASES = [
    # name, B, Sq, H, D, page, KV, causal, splits, layout
    ("prefill_direct", 2, 512, 2, 128, 128, 1024, False, 1, "prefill"),
    ("prefill_split", 1, 1024, 2, 128, 64, 2048, False, 4, "prefill"),
    ("key_split_decode", 2, 1, 8, 128, 128, 4096, False, None, "key"),
    ("query_causal_ragged", 1, 300, 2, 64, 48, 1000, True, 2, "query"),
    ("fp16_d256", 2, 7, 1, 256, 16, 200, True, None, None),
]


def _capture(call):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call()
    return graph, out


def _replay_matches_eager(graph, out, call, q, dtype, reps=3):
    gen = torch.Generator().manual_seed(17)
    eager = None
    for _ in range(reps):
        q.copy_(torch.randn(q.shape, generator=gen).to(dtype))
        eager = call()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), "graph replay differs from the eager call"
    return eager


@pytest.mark.parametrize("name,b,sq,h,d,page,kv,causal,splits,layout", CASES)
def test_graph_replays_match_eager_and_oracle(name, b, sq, h, d, page, kv, causal, splits, layout):
    from fgw_amd.operators.mha.current import build_kernel
    dtype = torch.float16 if name.startswith("fp16") else torch.bfloat16
    width = (kv + page - 1) // page
    case = (name, b, sq, h, d, page, width)
    q, k, v, table = O.make_inputs(case, 4, dtype)
    lengths = torch.tensor([kv - 17 * i for i in range(b)], dtype=torch.int32)
    k, v = O.poison_unread(k, v, table, lengths, page)
    dq, dk, dv, dt, dl = (x.cuda() for x in (q, k, v, table, lengths))
    print(f"graph replay {name}: B{b} Sq{sq} H{h} D{d} page{page} KV{kv} causal={causal} "
          f"splits={splits} layout={layout}", flush=True)
    kern = build_kernel(b, sq, h, d, k.shape[0], width, page, causal,
                        "float16" if dtype == torch.float16 else "bfloat16", 0,
                        num_splits=splits, layout=layout, cache_lengths=tuple(lengths.tolist()))
    call = lambda: kern(dq, dk, dv, dt, dl)  # noqa: E731
    graph, out = _capture(call)
    _replay_matches_eager(graph, out, call, dq, dtype)
    expected = O.reference(dq.cpu(), k, v, table, lengths, page, causal)
    rtol, atol = O.TOLERANCES[dtype]
    torch.testing.assert_close(out.cpu(), expected, rtol=rtol, atol=atol)


def test_graph_replays_of_the_static_fused_path():
    from fgw_amd.operators.mha.kernels.mha_static_host_hip import build_fused_kernel
    sq, kv = 512, 2048
    host = O.bench_inputs(1, sq, 1, 128, 128, kv, torch.bfloat16)
    dq, dk, dv, dt, dl = (x.cuda() for x in host)
    kern = build_fused_kernel(sq, kv, host[1].shape[0], 0, fallback=False)
    assert kern.execution == "static"
    print(f"graph replay static fused: Q{sq} KV{kv} {kern.plan.describe()}", flush=True)
    assert kern.plan.merges  # cut tiles: the merge launch is captured too
    call = lambda: kern(dq, dk, dv, dt, dl)  # noqa: E731
    graph, out = _capture(call)
    _replay_matches_eager(graph, out, call, dq, torch.bfloat16)
    expected = O.chunked_reference(dq.cpu(), *host[1:], 128, False)
    rtol, atol = O.TOLERANCES[torch.bfloat16]
    torch.testing.assert_close(out.cpu(), expected, rtol=rtol, atol=atol)


def test_graph_replays_of_a_balanced_plan_with_new_lengths():
    """A length-balanced decode plan reads the lengths on the device (split
    counts, work items, merge): one captured graph replays correctly after
    the lengths are rewritten in place, bit for bit against the eager call,
    and against the oracle for the last lengths."""
    from fgw_amd.operators.mha.current import build_kernel
    b, sq, h, d, page, kv = 4, 1, 8, 128, 128, 8192
    width = kv // page
    case = ("balanced_graph", b, sq, h, d, page, width)
    q, k, v, table = O.make_inputs(case, 6, torch.bfloat16)
    first = [4635, 4285, 4326, 1917]
    kern = build_kernel(b, sq, h, d, k.shape[0], width, page, False, "bfloat16", 0,
                        num_splits=16, layout="key", split_keys=491)
    assert kern.split_balance == "length"
    dq, dk, dv, dt = (x.cuda() for x in (q, k, v, table))
    dl = torch.tensor(first, dtype=torch.int32, device="cuda")
    call = lambda: kern(dq, dk, dv, dt, dl)  # noqa: E731
    graph, out = _capture(call)
    for lens in ([4635, 4285, 4326, 1917], [8192, 0, 100, 5000], [1, 8192, 8192, 3000]):
        dl.copy_(torch.tensor(lens, dtype=torch.int32))
        eager = call()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"graph replay differs from the eager call at {lens}"
    lengths = torch.tensor(lens, dtype=torch.int32)
    expected = O.reference(q, k, v, table, lengths, page, False)
    rtol, atol = O.TOLERANCES[torch.bfloat16]
    torch.testing.assert_close(out.cpu(), expected, rtol=rtol, atol=atol)
