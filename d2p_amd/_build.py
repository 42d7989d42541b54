"""In-tree build of the d2p_amd native libraries (no JIT cache, no pip install).

* ``libd2p_amd.so`` -- the HIP kernels for gfx950 and their C ABI
  (``include/d2p_amd.h``), compiled with hipcc;
* ``_C.so``         -- the PyTorch operator layer (``csrc/torch_ops.cpp``),
  compiled with g++ against the installed torch and linked to libd2p_amd.so
  through an ``$ORIGIN`` rpath.

Both land next to this file so they travel with the source tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
ROOT = os.path.dirname(PKG)
INCLUDE = os.path.join(ROOT, "include")
OBJ = os.path.join(PKG, "_build")
KERNEL_LIB = os.path.join(PKG, "libd2p_amd.so")
OP_LIB = os.path.join(PKG, "_C.so")

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # packed-FP32 VALU forms are kept out of the generated code on purpose
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def _run(cmd, cwd=None):
    r = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}):\n{' '.join(cmd)}\n"
                           f"{r.stdout}\n{r.stderr}")
    return r


def _compile_hip(src: str) -> str:
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    _run([HIPCC, *HIP_FLAGS, "-c", src, "-o", obj])
    return obj


def build_kernels(jobs: int = 8) -> str:
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs)))) as ex:
        objs = list(ex.map(_compile_hip, srcs))
    tmp = KERNEL_LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, KERNEL_LIB)
    return KERNEL_LIB


def build_ops() -> str:
    import torch
    tdir = os.path.dirname(torch.__file__)
    tinc = os.path.join(tdir, "include")
    tlib = os.path.join(tdir, "lib")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    src = os.path.join(CSRC, "torch_ops.cpp")
    tmp = OP_LIB + ".tmp"
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-w",
        f"-I{tinc}", f"-I{os.path.join(tinc, 'torch', 'csrc', 'api', 'include')}",
        f"-I{os.path.join(ROCM, 'include')}", f"-I{INCLUDE}",
        src, "-o", tmp,
        f"-L{PKG}", "-ld2p_amd", f"-L{tlib}", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
        "-lc10", "-lc10_hip", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{tlib}",
    ]
    _run(cmd)
    os.replace(tmp, OP_LIB)
    return OP_LIB


def build(verbose: bool = False) -> None:
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    k = build_kernels()
    o = build_ops()
    if verbose:
        print(f"built {k}\nbuilt {o}")


def clean() -> None:
    shutil.rmtree(OBJ, ignore_errors=True)
    for f in (KERNEL_LIB, OP_LIB):
        if os.path.exists(f):
            os.remove(f)


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
