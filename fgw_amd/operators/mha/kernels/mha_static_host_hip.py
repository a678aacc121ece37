"""Static host KV-block schedule path: B1H1, BF16, D128, full page-128 KV.

Mirrors the reference's static-plan kernel modules:
  build_kernel        operators/mha/kernels/mha_static_host_candidate.py:17-553
                      (plan_policy balanced / cost / tail / stream)
  build_fused_kernel  operators/mha/kernels/mha_paged_decode_ascend_fused.py:357-680
                      (choose_stream_plan, merge fused behind the local phase)
Both return a launch callable with the reference attributes (plan,
prepare_plan, validate_inputs, run_local, local_kernel, merge_kernel,
compute, finish, merge_assignment). The local phase is
fgw_mha_static_local: the query-layout kernel runs each program's segments
of the host plan (fgw_amd.operators.mha.static_schedule), writing whole
tiles to the output and cut tiles to partial slots; the merge phase is
fgw_mha_static_merge, one workgroup per cut tile. The reference's merge
variants (merge_policy, merge_rows, merge_programs) tile its Ascend vector
merge; here one merge serves them all, so those arguments are validated and
recorded only.
"""
from __future__ import annotations

import ctypes
from functools import lru_cache

import torch

from fgw_amd import _lib
from fgw_amd.operators.mha import static_schedule as S
from fgw_amd.operators.mha.kernels.mha_paged_decode_hip import _current_stream, _device_info

D = 128
PAGE = 128
MERGE_POLICIES = ("fixed", "weighted", "grouped", "preweighted", "prefetch", "simd", "rawsimd",
                  "rawrecip")


def _device_programs(device_index):
    info = _device_info(device_index)
    return max(1, min(S.MAX_CORES, info.num_cus * info.wg_per_cu[_lib.LAYOUT_QUERY]))


class _StaticLaunch:
    """Launch callable of one (plan, Q, KV, pool) specialisation."""

    execution = "static"

    def __init__(self, plan, sq, kv, pool_rows, device_index, meta):
        self.plan = plan
        self._sq, self._kv, self._pool = sq, kv, pool_rows
        self._width = kv // PAGE
        self._index = device_index
        self._device = torch.device("cuda", device_index)
        self._lib = _lib.load()
        self._shape = _lib.Shape(1, sq, 1, D, pool_rows, self._width, PAGE, 0, _lib.DTYPE_BFLOAT16)
        self._slots = plan.partial_count
        self._uploaded = {}
        self._sched = {}
        self.merge_assignment = dict(policy=meta["merge_policy"], tasks=plan.merges,
                                     programs=len(plan.merges), max_rows=S.BLOCK, max_chunks=1)
        self.merge_policy = meta["merge_policy"]
        self.plan_policy = meta["plan_policy"]
        self.compute_grid = len(plan.programs)
        self.local_kernel = self._local
        self.merge_kernel = self._merge if plan.merges else None
        self.fixed_merge_kernel = self.merge_kernel
        self.fixed_launch = self.__call__

    # -- plan tables -----------------------------------------------------
    def prepare_plan(self, device=None):
        """Device tables (segments [n, 4], seg_offsets [programs + 1], merges [m, 3])."""
        device = torch.device(device) if device is not None else self._device
        if device not in self._uploaded:
            segs, offsets = [], [0]
            for program in self.plan.programs:
                segs.extend(program)
                offsets.append(len(segs))
            merges = list(self.plan.merges) or [(-1, -1, -1)]
            self._uploaded[device] = tuple(
                torch.tensor(x, dtype=torch.int32, device=device)
                for x in (segs, offsets, merges))
        return self._uploaded[device]

    def _schedule(self, device):
        """The C schedule over the device tables, built once per device."""
        sched = self._sched.get(device)
        if sched is None:
            segs, offsets, merges = self.prepare_plan(device)
            sched = _lib.Schedule(segs.data_ptr(), offsets.data_ptr(), merges.data_ptr(),
                                  len(self.plan.programs), len(self.plan.merges), self._slots,
                                  S.BLOCK)
            self._sched[device] = sched
        return sched

    # -- reference-shaped entry points -------------------------------------
    def validate_inputs(self, q, k, v, table, lengths):
        """The reference's input assertions (mha_static_host_candidate.py:502-509)."""
        assert tuple(q.shape) == (1, self._sq, 1, D) and tuple(k.shape) == (self._pool, 1, D)
        assert v.shape == k.shape
        assert tuple(table.shape) == (1, self._width) and lengths.cpu().tolist() == [self._kv]
        assert q.dtype == k.dtype == v.dtype == torch.bfloat16
        assert table.dtype == lengths.dtype == torch.int32
        assert q.device.type == "cuda" and all(
            x.device == q.device and x.is_contiguous() for x in (q, k, v, table, lengths))

    def _check(self, q, k, v, table, lengths):
        if (tuple(q.shape) != (1, self._sq, 1, D) or tuple(k.shape) != (self._pool, 1, D)
                or v.shape != k.shape or tuple(table.shape) != (1, self._width)
                or tuple(lengths.shape) != (1,)):
            raise ValueError("tensor shapes do not match the built kernel")
        if q.dtype != torch.bfloat16 or k.dtype != q.dtype or v.dtype != q.dtype:
            raise ValueError("matching FP16/BF16 Q/K/V required")
        if table.dtype != torch.int32 or lengths.dtype != torch.int32:
            raise ValueError("int32 metadata required")
        if any(x.device != self._device or not x.is_contiguous() for x in (q, k, v, table, lengths)):
            raise ValueError("contiguous inputs on the same GPU required")

    def _local(self, q, k, v, table, lengths):
        """Local phase -> (parts, lse, output); parts/lse are None without cut tiles."""
        self._check(q, k, v, table, lengths)
        out = torch.empty((1, self._sq, D), dtype=torch.bfloat16, device=self._device)
        parts = lse = None
        if self._slots:
            ws = torch.empty(self._slots * S.BLOCK * (D + 1), dtype=torch.float32,
                             device=self._device)
            parts, lse = ws[:self._slots * S.BLOCK * D], ws[self._slots * S.BLOCK * D:]
        t = _lib.Tensors(q.data_ptr(), k.data_ptr(), v.data_ptr(), table.data_ptr(),
                         lengths.data_ptr(), out.data_ptr(),
                         None if parts is None else parts.data_ptr(),
                         None if lse is None else lse.data_ptr())
        sched = self._schedule(self._device)
        _lib.check(self._lib.fgw_mha_static_local(ctypes.byref(self._shape), ctypes.byref(t),
                                                  ctypes.byref(sched),
                                                  _current_stream(self._index)))
        return parts, lse, out

    def _merge(self, parts, lse, output):
        t = _lib.Tensors(None, None, None, None, None, output.data_ptr(), parts.data_ptr(),
                         lse.data_ptr())
        sched = self._schedule(output.device)
        _lib.check(self._lib.fgw_mha_static_merge(ctypes.byref(self._shape), ctypes.byref(t),
                                                  ctypes.byref(sched),
                                                  _current_stream(self._index)))

    def run_local(self, prepared, k, v, table, lengths):
        return self._local(prepared, k, v, table, lengths)

    def compute(self, q, k, v, table, lengths):
        # Q is read in place as [1, Sq, 1, D]; no head-major copy is prepared.
        return self._local(q, k, v, table, lengths)

    def finish(self, parts, lse, output):
        if self.merge_kernel is not None:
            self._merge(parts, lse, output)
        return output.view(1, self._sq, 1, D)

    def __call__(self, q, k, v, table, lengths):
        return self.finish(*self.compute(q, k, v, table, lengths))


def _check_pool(kv, pool_rows):
    if type(pool_rows) is not int or pool_rows <= 0 or pool_rows % PAGE or pool_rows < kv:
        raise ValueError("whole physical pool pages, at least KV capacity required")


@lru_cache(maxsize=64)
def build_kernel(sq, kv, pool_rows, plan_policy="balanced", programs=None, merge_rows=8,
                 tail_pieces=None, merge_policy="fixed", merge_programs=56,
                 include_fixed_control=True, row_softmax=False, fused_output=False,
                 device_index=None):
    """Static-plan B1H1 attention (mha_static_host_candidate.py:17-553).

    Same argument checks; `programs` defaults to every resident query-layout
    workgroup of the device (the reference: 28 Cube cores).
    """
    if fused_output and merge_policy != "rawsimd":
        raise ValueError("fused_output experiment requires rawsimd")
    if plan_policy not in ("balanced", "cost", "tail", "stream"):
        raise ValueError("plan_policy must be balanced, cost or tail")
    if merge_policy not in MERGE_POLICIES:
        raise ValueError("merge_policy must be fixed or weighted")
    if merge_programs not in (28, 56):
        raise ValueError("merge_programs must be 28 or 56")
    if merge_policy == "grouped" and merge_rows != 8:
        raise ValueError("grouped comparison requires original R8")
    if merge_rows not in (8, 16, 32):
        raise ValueError("merge_rows must be 8, 16 or 32")
    if programs is not None and plan_policy in ("cost", "stream"):
        raise ValueError("explicit programs require balanced policy")
    if device_index is None:
        device_index = torch.cuda.current_device()
    cores = programs if programs is not None else _device_programs(int(device_index))
    if plan_policy == "cost":
        plan = S.choose_plan(sq, kv, cores)
    elif plan_policy == "tail":
        plan = S.make_tail_plan(sq, kv, cores, tail_pieces)
    elif plan_policy == "stream":
        plan = S.choose_stream_plan(sq, kv, cores)
    else:
        plan = S.make_plan(sq, kv, cores)
    _check_pool(kv, pool_rows)
    meta = dict(plan_policy=plan_policy, merge_policy=merge_policy)
    launch = _StaticLaunch(plan, sq, kv, pool_rows, int(device_index), meta)
    launch.merge_rows, launch.merge_programs = merge_rows, merge_programs
    launch.row_softmax, launch.fused_output = row_softmax, fused_output
    launch.include_fixed_control = include_fixed_control
    return launch


class _AutomaticLaunch:
    """The static builder's fallback: the same call signature and two-phase
    entry points (compute, then finish) over the automatic split path
    (build_kernel of the main entry), for shapes where that path measured
    faster. `plan` is the static plan it replaced (for describe()); `execution`
    says which path runs."""

    execution = "automatic"

    def __init__(self, plan, sq, kv, pool_rows, device_index):
        from fgw_amd.operators.mha.kernels.mha_paged_decode_hip import build_kernel as _build
        self.plan = plan
        self._sq, self._kv, self._pool, self._width = sq, kv, pool_rows, kv // PAGE
        self._kernel = _build(1, sq, 1, D, pool_rows, self._width, PAGE, False, "bfloat16",
                              device_index, full_kv_cache=True)
        self.compute_grid = self._kernel.compute_grid
        self.num_splits = self._kernel.num_splits
        self.layout = self._kernel.layout
        self.plan_policy = "automatic"
        self.merge_policy = "rawsimd"
        self.local_kernel = self.compute
        self.merge_kernel = None
        self.fixed_merge_kernel = None
        self.merge_assignment = dict(policy="automatic", tasks=(), programs=0, max_rows=S.BLOCK,
                                     max_chunks=1)

    def validate_inputs(self, q, k, v, table, lengths):
        """The reference's input assertions (mha_static_host_candidate.py:502-509)."""
        assert tuple(q.shape) == (1, self._sq, 1, D) and tuple(k.shape) == (self._pool, 1, D)
        assert v.shape == k.shape
        assert tuple(table.shape) == (1, self._width) and lengths.cpu().tolist() == [self._kv]
        assert q.dtype == k.dtype == v.dtype == torch.bfloat16
        assert table.dtype == lengths.dtype == torch.int32

    def compute(self, q, k, v, table, lengths):
        return None, None, self._kernel(q, k, v, table, lengths)

    def run_local(self, prepared, k, v, table, lengths):
        return self.compute(prepared, k, v, table, lengths)

    def finish(self, parts, lse, output):
        return output.view(1, self._sq, 1, D)

    def __call__(self, q, k, v, table, lengths):
        return self.finish(*self.compute(q, k, v, table, lengths))


@lru_cache(maxsize=64)
def build_fused_kernel(sq, kv, pool_rows, device_index=None, fallback=True):
    """Fused-output static path (mha_paged_decode_ascend_fused.py:357-680):
    choose_stream_plan over the device's programs.

    fallback (default): where the automatic split path of the main entry
    measured faster (static_schedule.static_preferred: the nearest shape of the
    committed MI355X static-scan calibration, static kept from 1.02x), the
    returned callable runs that path instead (`execution` == "automatic");
    fallback=False always runs the static plan (`execution` == "static")."""
    if device_index is None:
        device_index = torch.cuda.current_device()
    plan = S.choose_stream_plan(sq, kv, _device_programs(int(device_index)))
    _check_pool(kv, pool_rows)
    if fallback and not S.static_preferred(sq, kv):
        return _AutomaticLaunch(plan, sq, kv, pool_rows, int(device_index))
    launch = _StaticLaunch(plan, sq, kv, pool_rows, int(device_index),
                           dict(plan_policy="stream", merge_policy="rawsimd"))
    launch.fixed_merge_kernel = None
    return launch
