"""Runtime-shape family of the paged attention entry.

Mirrors the reference's opt-in runtime-shape families
(operators/mha/runtime_lengths.py:1-44; kernel side
mha_paged_decode_ascend_v7_experimental.py:153-168): batch, heads, the split
count and the merge row tile are fixed when the family is built; the query
length, the physical pool rows and the page-table width are taken from the
tensors of each call, and the logical KV lengths stay device data.

The hand-written kernels behind build_kernel are shape-generic at run time
(every extent is a kernel argument), so a family member for a new
(Q, pool rows, width) is only a launch plan: the C planner runs once for that
shape and the plan is kept by build_kernel's cache. Like the reference
family, a call reads nothing back from the device.
"""
from __future__ import annotations

from functools import lru_cache

import torch

from fgw_amd.operators.mha.kernels.mha_paged_decode_hip import build_kernel

RUNTIME_SPLITS = (1, 2, 4, 8, 16)
MERGE_ROWS = (1, 2, 4, 8)
DIM = 128
PAGE = 128


@lru_cache(maxsize=64)
def build_runtime_kernel(batch, heads, num_splits, merge_rows=8, device_index=0):
    """Return the family callable `call(q, k, v, table, lengths) -> O`.

    Same arguments and build-time checks as the reference
    (runtime_lengths.py:10-14): B1H1, num_splits in {1, 2, 4, 8, 16},
    merge_rows in {1, 2, 4, 8}. merge_rows is the reference merge kernel's
    row tile; the merge here is one thread per (row, 4 dims) whatever it is,
    so it is validated and recorded in family_key only.
    """
    if batch != 1 or heads != 1 or num_splits not in RUNTIME_SPLITS:
        raise ValueError("Runtime candidate requires B1H1 and split1/2/4/8/16")
    if merge_rows not in MERGE_ROWS:
        raise ValueError("merge_rows must be 1/2/4/8")

    def program(sq, pool_rows, width):
        """The plan of one runtime shape (a build_kernel launch callable)."""
        return build_kernel(batch, sq, heads, DIM, pool_rows, width, PAGE, False, "bfloat16",
                            device_index, num_splits=num_splits, split_policy="legacy")

    def call(q, k, v, table, lengths):
        # Checks and messages of runtime_lengths.py:23-38, with the device
        # type of this build.
        if (q.ndim != 4 or q.shape[0] != batch or tuple(q.shape[2:]) != (heads, DIM)
                or q.shape[1] <= 0 or q.dtype != torch.bfloat16):
            raise ValueError("Expected BF16 Q[B,Q,H,128] with positive Q")
        if (k.ndim != 3 or tuple(k.shape[1:]) != (heads, DIM) or k.shape[0] <= 0
                or k.shape[0] % PAGE or v.shape != k.shape
                or k.dtype != q.dtype or v.dtype != q.dtype):
            raise ValueError("Expected matching BF16 paged K/V[pool_rows,H,128]")
        if (table.ndim != 2 or table.shape[0] != batch or table.shape[1] < num_splits
                or table.dtype != torch.int32 or tuple(lengths.shape) != (batch,)
                or lengths.dtype != torch.int32):
            raise ValueError("Expected int32 table/lengths with sufficient split capacity")
        if any(t.device != q.device or t.device.type != "cuda" or t.device.index != device_index
               or not t.is_contiguous() for t in (q, k, v, table, lengths)):
            raise ValueError("All inputs must be contiguous on the same GPU")
        # No host read of lengths or page ids: the caller keeps them within
        # the table capacity, as for the reference family.
        return program(q.shape[1], k.shape[0], table.shape[1])(q, k, v, table, lengths)

    call.family_key = (batch, heads, num_splits, merge_rows, device_index)
    call.program = program
    return call
