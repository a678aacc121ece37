"""Launches on several streams at once, and the per-call checks on device tensors
(MI355X only).

Streams: calls on two side streams (default priority) run concurrently with
their own inputs; each result must equal the same call made alone on the
current stream, bit for bit, because every call owns its output and split
workspace and the library keeps no device state between calls.
Checks: a launch callable rejects device tensors that do not match its
specialisation (shape, dtype, metadata dtype, contiguity, device) with a
ValueError before anything is launched.
"""
import pytest
import torch

from oracle import mha_oracle as O

pytestmark = pytest.mark.gpu


def _kernel(b, sq, h, kv, layout, splits=None):
    from fgw_amd.operators.mha.current import build_kernel
    host = O.bench_inputs(b, sq, h, 128, 128, kv, torch.bfloat16)
    kern = build_kernel(b, sq, h, 128, host[1].shape[0], host[3].shape[1], 128, False,
                        "bfloat16", 0, num_splits=splits, layout=layout)
    return kern, [x.cuda() for x in host]


def test_concurrent_streams_match_single_stream_calls():
    decode, dec_in = _kernel(2, 1, 8, 8192, "key")          # partial + merge
    prefill, pre_in = _kernel(2, 1024, 2, 2048, "prefill", 4)  # partial + merge
    assert decode.num_splits > 1 and prefill.num_splits == 4
    gen = torch.Generator().manual_seed(23)
    rounds = []
    for _ in range(4):
        qd = torch.randn(dec_in[0].shape, generator=gen).to(torch.bfloat16).cuda()
        qp = torch.randn(pre_in[0].shape, generator=gen).to(torch.bfloat16).cuda()
        rounds.append((qd, qp, decode(qd, *dec_in[1:]), prefill(qp, *pre_in[1:])))
    torch.cuda.synchronize()
    print("concurrent streams: 4 rounds of split decode and split prefill", flush=True)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    outs = []
    for qd, qp, _, _ in rounds:
        with torch.cuda.stream(s1):
            od = decode(qd, *dec_in[1:])
        with torch.cuda.stream(s2):
            op = prefill(qp, *pre_in[1:])
        outs.append((od, op))
    torch.cuda.current_stream().wait_stream(s1)
    torch.cuda.current_stream().wait_stream(s2)
    torch.cuda.synchronize()
    for (od, op), (_, _, ed, ep) in zip(outs, rounds):
        assert torch.equal(od, ed) and torch.equal(op, ep)


def test_launch_callable_rejects_mismatched_device_tensors():
    kern, (q, k, v, table, lengths) = _kernel(2, 4, 2, 512, "query", 2)
    cases = [
        ((q[:, :2], k, v, table, lengths), "do not match the built kernel"),
        ((q, k[:-128], v, table, lengths), "do not match the built kernel"),
        ((q, k, v, table[:, :1], lengths), "do not match the built kernel"),
        ((q.half(), k, v, table, lengths), "matching FP16/BF16"),
        ((q, k, v.half(), table, lengths), "matching FP16/BF16"),
        ((q, k, v, table.long(), lengths), "int32 metadata"),
        ((q, k, v, table, lengths.long()), "int32 metadata"),
        ((q.transpose(1, 2).contiguous().transpose(1, 2), k, v, table, lengths), "contiguous"),
        ((q, k, v, table, lengths.cpu()), "same GPU"),
    ]
    for args, message in cases:
        with pytest.raises(ValueError, match=message):
            kern(*args)
    out = kern(q, k, v, table, lengths)  # the valid call still runs
    torch.cuda.synchronize()
    expected = O.reference(q.cpu(), k.cpu(), v.cpu(), table.cpu(), lengths.cpu(), 128, False)
    rtol, atol = O.TOLERANCES[torch.bfloat16]
    torch.testing.assert_close(out.cpu(), expected, rtol=rtol, atol=atol)
