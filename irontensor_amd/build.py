"""Builds libirontensor_hip.so (the C-ABI library) in-tree with hipcc for gfx950.

Usage: python -m irontensor_amd.build   (or irontensor_amd.build.build_library()).
The compile always runs; objects go to irontensor_amd/_build/ and the shared library next to this
file, so it travels with the repository snapshot to the GPU box.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libirontensor_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["runtime.cpp", "api.cpp", "api_train.cpp", "kernels_gemm.hip", "kernels_misc.hip", "kernels_flash.hip",
           "kernels_gemv.hip", "kernels_train.hip", "noalloc.hip",
           "kernels_flash2.hip"]

# -packed-fp32-ops: hipcc must not emit packed FP32 ALU ops (v_pk_*_f32) on this pool.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]


def _compile(src: Path, obj: Path) -> subprocess.Popen:
    lang = ["-x", "hip"] if src.suffix == ".hip" else []
    cmd = [HIPCC, *HIP_FLAGS, *lang, "-c", str(src), "-o", str(obj)]
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)


def build_library(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    procs = []
    objs = []
    for name in SOURCES:
        src = CSRC / name
        obj = BUILD / (name + ".o")
        objs.append(obj)
        procs.append((name, _compile(src, obj)))
    failed = []
    for name, p in procs:
        out, _ = p.communicate()
        if p.returncode != 0:
            failed.append((name, out))
        elif verbose and out.strip():
            print(out, file=sys.stderr)
    if failed:
        msg = "\n".join(f"--- {n} ---\n{o}" for n, o in failed)
        raise RuntimeError(f"hipcc failed:\n{msg}")
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}")
    os.replace(tmp, LIB)
    return LIB


CPP_TEST_SRC = ROOT / "tests" / "cpp" / "test_host_api.cpp"
CPP_TEST_BIN = ROOT / "tests" / "cpp" / "_build" / "test_host_api"


def build_cpp_tests() -> Path:
    """Builds the C++ host-API test program against the in-tree library (rpath-relative)."""
    CPP_TEST_BIN.parent.mkdir(parents=True, exist_ok=True)
    cmd = ["g++", "-std=c++17", "-O1", "-Wall", f"-I{ROOT / 'include'}", str(CPP_TEST_SRC),
           "-o", str(CPP_TEST_BIN), f"-L{PKG}", "-lirontensor_hip",
           "-Wl,-rpath,$ORIGIN/../../../irontensor_amd", "-Wl,-rpath,/opt/rocm/lib"]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"C++ host API test build failed:\n{res.stdout}")
    return CPP_TEST_BIN


if __name__ == "__main__":
    print(build_library(verbose=True))
    print(build_cpp_tests())
