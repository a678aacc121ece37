"""ctypes binding of libfgw_mha.so (C ABI declared in include/fgw_mha.h).

The library is loaded on first use. A missing or stale library raises
RuntimeError: there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
import pathlib
import threading

LIBRARY = pathlib.Path(__file__).resolve().with_name("libfgw_mha.so")
ABI_VERSION = 6

FGW_MHA_OK, FGW_MHA_EINVAL, FGW_MHA_EUNSUPPORTED, FGW_MHA_EHIP = 0, -1, -2, -3
NOALLOC_SCRATCH_BYTES = 32 << 20  # FGW_MHA_NOALLOC_SCRATCH_BYTES
NOALLOC_ARRIVALS = 65536  # FGW_MHA_NOALLOC_ARRIVALS
DTYPE_FLOAT16, DTYPE_BFLOAT16 = 0, 1
LAYOUT_AUTO, LAYOUT_QUERY, LAYOUT_KEY, LAYOUT_PREFILL = -1, 0, 1, 2
NUM_LAYOUTS = 3

c_int32, c_int64, c_void_p = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p


class Shape(ctypes.Structure):
    _fields_ = [("batch", c_int32), ("sq", c_int32), ("heads", c_int32), ("dim", c_int32),
                ("pool_rows", c_int64), ("width", c_int32), ("page_size", c_int32),
                ("causal", c_int32), ("dtype", c_int32)]


class Request(ctypes.Structure):
    _fields_ = [("num_splits", c_int32), ("persistent_programs", c_int32), ("layout", c_int32),
                ("split_keys", c_int32), ("stages", c_int32)]


class DeviceInfo(ctypes.Structure):
    _fields_ = [("num_cus", c_int32), ("wg_per_cu", c_int32 * NUM_LAYOUTS), ("arch_gfx950", c_int32),
                ("wg_per_cu_key_single", c_int32)]


class Plan(ctypes.Structure):
    _fields_ = [("layout", c_int32), ("rows_per_tile", c_int32), ("q_tiles", c_int32),
                ("num_splits", c_int32), ("query_tile_tasks", c_int32),
                ("work_items", c_int32), ("grid", c_int32), ("threads", c_int32),
                ("execution_mode", c_int32), ("dim_padded", c_int32),
                ("parts_floats", c_int64), ("lse_floats", c_int64), ("split_keys", c_int32),
                ("stages", c_int32), ("arrival_counters", c_int32)]


class Tensors(ctypes.Structure):
    _fields_ = [("q", c_void_p), ("k_cache", c_void_p), ("v_cache", c_void_p),
                ("block_table", c_void_p), ("cache_seqlens", c_void_p), ("out", c_void_p),
                ("parts", c_void_p), ("lse", c_void_p), ("arrivals", c_void_p)]


class Schedule(ctypes.Structure):
    _fields_ = [("segments", c_void_p), ("seg_offsets", c_void_p), ("merges", c_void_p),
                ("programs", c_int32), ("n_merges", c_int32), ("slots", c_int32),
                ("block_keys", c_int32)]


# name -> (argtypes); every function returns int.
SIGNATURES = {
    "fgw_mha_abi_version": (),
    "fgw_mha_last_error": (),
    "fgw_mha_query_device": (ctypes.c_int, ctypes.POINTER(DeviceInfo)),
    "fgw_mha_plan": (ctypes.POINTER(Shape), ctypes.POINTER(Request), ctypes.POINTER(DeviceInfo),
                     ctypes.POINTER(Plan)),
    "fgw_mha_fwd": (ctypes.POINTER(Shape), ctypes.POINTER(Plan), ctypes.POINTER(Tensors), c_void_p),
    "fgw_mha_fwd_noalloc": (ctypes.POINTER(Shape), ctypes.POINTER(Plan),
                            ctypes.POINTER(Tensors), c_void_p),
    "fgw_mha_partial": (ctypes.POINTER(Shape), ctypes.POINTER(Plan), ctypes.POINTER(Tensors),
                        c_void_p),
    "fgw_mha_merge": (ctypes.POINTER(Shape), ctypes.POINTER(Plan), ctypes.POINTER(Tensors),
                      c_void_p),
    "fgw_mha_gather_kv": (ctypes.POINTER(Shape), ctypes.POINTER(Tensors), c_void_p, c_void_p,
                          c_int32, c_void_p),
    "fgw_mha_pack_pages": (ctypes.POINTER(Shape), ctypes.POINTER(Tensors), c_void_p, c_int32,
                           c_void_p, c_void_p, c_void_p),
    "fgw_mha_static_local": (ctypes.POINTER(Shape), ctypes.POINTER(Tensors),
                             ctypes.POINTER(Schedule), c_void_p),
    "fgw_mha_static_merge": (ctypes.POINTER(Shape), ctypes.POINTER(Tensors),
                             ctypes.POINTER(Schedule), c_void_p),
}

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load and type the library once; raise RuntimeError if it is absent or stale."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIBRARY.exists():
            raise RuntimeError(
                f"{LIBRARY} is missing: build it with `python -m fgw_amd.build` "
                "(the operator has no non-HIP implementation)")
        lib = ctypes.CDLL(str(LIBRARY))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = list(argtypes)
            fn.restype = ctypes.c_char_p if name == "fgw_mha_last_error" else ctypes.c_int
        version = lib.fgw_mha_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{LIBRARY} has ABI {version}, expected {ABI_VERSION}; rebuild it")
        _lib = lib
        return lib


def entry_address(name: str) -> int:
    """Address of a C entry point of the loaded library (for the launch shim)."""
    return ctypes.cast(getattr(load(), name), c_void_p).value


def load_launch_module():
    """The C++ launch callable type (fgw_amd._launch); raises if it was not built."""
    try:
        from fgw_amd import _launch
    except ImportError as exc:
        raise RuntimeError("fgw_amd._launch is missing: build it with `python -m fgw_amd.build` "
                           "(the operator has no other launch path)") from exc
    return _launch


def check(status: int) -> None:
    """Map a C status to the reference's exception types."""
    if status == FGW_MHA_OK:
        return
    message = load().fgw_mha_last_error().decode("utf-8", "replace")
    if status in (FGW_MHA_EINVAL, FGW_MHA_EUNSUPPORTED):
        raise ValueError(message)
    raise RuntimeError(message)


def query_device(index: int) -> DeviceInfo:
    info = DeviceInfo()
    check(load().fgw_mha_query_device(int(index), ctypes.byref(info)))
    return info


def plan(shape: Shape, request: Request, device: DeviceInfo) -> Plan:
    out = Plan()
    check(load().fgw_mha_plan(ctypes.byref(shape), ctypes.byref(request), ctypes.byref(device),
                              ctypes.byref(out)))
    return out
