"""Build oracle/_ref/grm_ref_harness.so from the reference's CPU sources.

TEST INFRASTRUCTURE ONLY.  Compiles /root/reference/grm/csrc/grm_cuda.cpp
(plain ATen; the reference's CPU op implementations) where it lies, with the
harness in this directory, using g++ directly.  Nothing from the reference is
copied; outputs go only to oracle/_ref/ (git-ignored).  The reference's
bindings.cpp is not built: it binds CUDA symbols that exist only in its .cu
files, which need nvcc.

Usage: python oracle/ref/build_ref.py [--reference /root/reference]
"""

from __future__ import annotations

import argparse
import subprocess
import sys
import sysconfig
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT_DIR = HERE.parent / "_ref"


def build(reference: Path = Path("/root/reference"), verbose: bool = False) -> Path:
    import torch
    from torch.utils import cpp_extension

    src_dir = reference / "grm" / "csrc"
    srcs = [src_dir / "grm_cuda.cpp", HERE / "ref_harness.cpp"]
    if not all(s.exists() for s in srcs):
        raise FileNotFoundError(f"reference sources not found under {src_dir}")
    OUT_DIR.mkdir(exist_ok=True)
    out = OUT_DIR / "grm_ref_harness.so"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"], str(src_dir)]
    torch_lib = cpp_extension.library_paths()[0]
    objs = []
    for s in srcs:
        obj = OUT_DIR / (s.stem + ".o")
        cmd = ["g++", "-O2", "-std=c++17", "-fPIC", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
               "-DTORCH_EXTENSION_NAME=grm_ref_harness", "-DTORCH_API_INCLUDE_EXTENSION_H",
               *[f"-I{i}" for i in incs], "-c", str(s), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        objs.append(str(obj))
    cmd = ["g++", "-shared", "-o", str(out), *objs, f"-L{torch_lib}", "-lc10", "-ltorch", "-ltorch_cpu",
           "-ltorch_python", f"-Wl,-rpath,{torch_lib}"]
    subprocess.run(cmd, check=True)
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    ap.add_argument("-v", action="store_true")
    a = ap.parse_args()
    print(build(Path(a.reference), a.v))
    sys.exit(0)
