"""Build the gfx950 HIP library and the torch op extension in-tree.

Outputs (next to this file):
  libgrm_hip.so    - the HIP kernels behind the C ABI of include/grm_hip.h
  grm_cuda_ext.so  - registers torch.ops.grm_cuda.* and calls libgrm_hip.so

Run ``python -m rnn_with_grm_amd.build`` (or ``__graft_entry__.build()``).
hipcc cross-compiles for gfx950, so no GPU is needed to build.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path
from typing import List, Optional

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
BUILD_DIR = PKG_DIR / "_build"
LIB_HIP = PKG_DIR / "libgrm_hip.so"
LIB_EXT = PKG_DIR / "grm_cuda_ext.so"

OFFLOAD_ARCH = "gfx950"
HIP_SOURCES = ["grm_capi.hip", "chunk_scan.hip", "chunk_scan_wide.hip", "chunk_scan_vsplit.hip", "chunk_bwd.hip",
               "gather_apply.hip", "retrieve.hip", "retrieve_window.hip", "route_fuse.hip", "route_select.hip",
               "layer_glue.hip"]
EXT_SOURCE = "grm_torch_ops.cpp"

# Packed fp32 instructions are kept out of every kernel (the flag is for the
# device pass; the host pass warns that it does not know it, harmlessly).
HIP_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found; set ROCM_PATH")
    return found


def _run(cmd: List[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def _stale(target: Path, deps: List[Path]) -> bool:
    if not target.exists():
        return True
    t = target.stat().st_mtime
    return any(d.stat().st_mtime > t for d in deps)


def _headers() -> List[Path]:
    return [INCLUDE / "grm_hip.h", CSRC / "grm_hip_common.h", CSRC / "chunk_scan.h", CSRC / "route_select.h",
            CSRC / "retrieve.h"]


def build_hip_library(force: bool = True, verbose: bool = False, jobs: Optional[int] = None) -> Path:
    """Compile every .hip file for gfx950 and link libgrm_hip.so."""
    BUILD_DIR.mkdir(exist_ok=True)
    hipcc = _hipcc()
    objs = []
    todo = []
    for src in HIP_SOURCES:
        obj = BUILD_DIR / (Path(src).stem + ".o")
        objs.append(obj)
        if force or _stale(obj, [CSRC / src] + _headers()):
            todo.append([hipcc, *HIP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(CSRC / src), "-o", str(obj)])
    workers = jobs or min(len(todo) or 1, 8)
    with ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(lambda c: _run(c, verbose), todo))
    if force or todo or _stale(LIB_HIP, objs):
        tmp = LIB_HIP.with_suffix(".so.tmp")
        _run([hipcc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
              "-Wl,-soname,libgrm_hip.so"], verbose)
        os.replace(tmp, LIB_HIP)
    return LIB_HIP


def build_torch_extension(force: bool = True, verbose: bool = False) -> Path:
    """Compile the torch.ops.grm_cuda shim and link it against libgrm_hip.so."""
    import torch
    from torch.utils import cpp_extension

    BUILD_DIR.mkdir(exist_ok=True)
    src = CSRC / EXT_SOURCE
    if not force and not _stale(LIB_EXT, [src, LIB_HIP] + _headers()):
        return LIB_EXT
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"], str(INCLUDE), f"{rocm}/include"]
    torch_lib = cpp_extension.library_paths()[0]
    obj = BUILD_DIR / "grm_torch_ops.o"
    cxx = os.environ.get("CXX", "g++")
    _run([cxx, "-O2", "-std=c++17", "-fPIC", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
          f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_EXTENSION_NAME=grm_cuda_ext",
          "-DTORCH_API_INCLUDE_EXTENSION_H", *[f"-I{i}" for i in incs], "-c", str(src), "-o", str(obj)],
         verbose)
    tmp = LIB_EXT.with_suffix(".so.tmp")
    _run([cxx, "-shared", "-o", str(tmp), str(obj), f"-L{PKG_DIR}", "-lgrm_hip", f"-L{torch_lib}",
          "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
          "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}"], verbose)
    os.replace(tmp, LIB_EXT)
    return LIB_EXT


def build(force: bool = True, verbose: bool = False) -> None:
    build_hip_library(force=force, verbose=verbose)
    build_torch_extension(force=force, verbose=verbose)


if __name__ == "__main__":
    build(force="--incremental" not in sys.argv, verbose="-v" in sys.argv)
    print(f"built {LIB_HIP.name} and {LIB_EXT.name} in {PKG_DIR}")
