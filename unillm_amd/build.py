"""Build libunillm_hip.so in-tree with hipcc for gfx950.

    python -m unillm_amd.build

Each translation unit compiles to unillm_amd/_build/*.o in parallel, then one
hipcc -shared link writes unillm_amd/libunillm_hip.so.  Packed-fp32 VALU ops
are disabled (-packed-fp32-ops) on every device pass.

The C++ host layer (unillm_amd/host: GGUF reader, loader, QuantLinear) uses
only the C ABI, so g++ builds it into libunillm_host.so, linked against
libunillm_hip.so; its test program tests/cpp/test_host is built beside it.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libunillm_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["capi.hip", "weights.hip", "gemv.hip", "decode.hip", "prefill.hip", "attention.hip",
           "dense.hip"]
# the dense (F32 / F16 / BF16) weights' f32 GEMM
LIBS = ["-L/opt/rocm/lib", "-lrocblas", "-Wl,-rpath,/opt/rocm/lib"]
HOST_SOURCES = ["gguf.cpp", "unillm_host.cpp"]
HOST_LIB = os.path.join(HERE, "libunillm_host.so")
HOST_TEST = os.path.join(os.path.dirname(HERE), "tests", "cpp", "test_host")
CXX = os.environ.get("CXX", "g++")
CXXFLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra"]
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs, *LIBS]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    build_host(verbose)
    return LIB


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{' '.join(cmd)} failed:\n{r.stdout}\n{r.stderr}")


def build_host(verbose: bool = False) -> str:
    host = os.path.join(HERE, "host")
    tmp = HOST_LIB + ".tmp"
    _run([CXX, *CXXFLAGS, "-shared", "-o", tmp,
          *[os.path.join(host, s) for s in HOST_SOURCES],
          "-L" + HERE, "-lunillm_hip", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, HOST_LIB)
    _run([CXX, *CXXFLAGS, "-o", HOST_TEST, HOST_TEST + ".cpp",
          "-L" + HERE, "-lunillm_host", "-lunillm_hip",
          "-Wl,-rpath,$ORIGIN/../../unillm_amd"])
    if verbose:
        print(f"built {HOST_LIB} and {HOST_TEST}")
    return HOST_LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
