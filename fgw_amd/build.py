"""Compile the HIP sources under fgw_amd/csrc into fgw_amd/libfgw_mha.so for gfx950,
and the host-only launch shim (csrc/launch_shim.cpp) into the Python module
fgw_amd._launch.

Every call rebuilds from scratch (objects under fgw_amd/_build). Run directly
(`python -m fgw_amd.build`) or through __graft_entry__.build().
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys
import sysconfig

PACKAGE = pathlib.Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "libfgw_mha.so"
ARCH = "gfx950"

# Packed FP32 instructions stay disabled in all device code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the softmax and rescale read them with
    # plain VALU ops instead of v_accvgpr copies.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def hipcc() -> str:
    path = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not pathlib.Path(path).exists():
        raise RuntimeError(f"hipcc not found (looked for {path})")
    return path


def _compile(source: pathlib.Path) -> pathlib.Path:
    obj = BUILD / (source.stem + ".o")
    cmd = [hipcc(), *HIP_FLAGS, "-c", str(source), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    log = "\n".join(line for line in (proc.stdout + proc.stderr).splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{log}")
    if log.strip():
        print(log, file=sys.stderr)
    return obj


SHIM_SOURCE = CSRC / "launch_shim.cpp"


def shim_path() -> pathlib.Path:
    return PACKAGE / ("_launch" + sysconfig.get_config_var("EXT_SUFFIX"))


def _build_shim() -> pathlib.Path:
    """Host-only C++ extension over the C ABI (torch headers for tensors,
    allocation and the current HIP stream). Built with g++: no device code."""
    import torch
    tdir = pathlib.Path(torch.__file__).resolve().parent
    out = shim_path()
    tmp = out.with_name(out.name + ".tmp")
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wno-unused-function",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           # The C++ ABI torch itself was built with (torch.utils.cpp_extension
           # passes the same define).
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           f"-I{tdir / 'include'}", f"-I{tdir / 'include' / 'torch' / 'csrc' / 'api' / 'include'}",
           "-I/opt/rocm/include", f"-I{sysconfig.get_paths()['include']}",
           str(SHIM_SOURCE), "-o", str(tmp), f"-L{tdir / 'lib'}", f"-Wl,-rpath,{tdir / 'lib'}",
           "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_python",
           "-L/opt/rocm/lib", "-Wl,-rpath,/opt/rocm/lib", "-lamdhip64"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"launch shim build failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, out)
    return out


def build(jobs: int | None = None, verbose: bool = True) -> pathlib.Path:
    """Compile all csrc/*.hip, link the shared library and build the launch
    shim; returns the library path."""
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    if BUILD.exists():
        shutil.rmtree(BUILD)
    BUILD.mkdir(parents=True)
    jobs = jobs or min(len(sources) + 1, max(1, min(16, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        shim = pool.submit(_build_shim)
        objects = list(pool.map(_compile, sources))
        shim_lib = shim.result()
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY} from {len(sources)} sources and {shim_lib.name}", file=sys.stderr)
    return LIBRARY


if __name__ == "__main__":
    build()
