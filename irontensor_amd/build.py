"""Builds libirontensor_hip.so (the C-ABI library) in-tree with hipcc for gfx950.

Usage: python -m irontensor_amd.build   (or irontensor_amd.build.build_library()).
The compile always runs; objects go to irontensor_amd/_build/ and the shared library next to this
file, so it travels with the repository snapshot to the GPU box.

python -m irontensor_amd.build --tuning also builds libirontensor_hip_tuning.so: the same library
with kernels_gemm.hip compiled under IT_TUNING, where the environment variable IT_PLAN="tile,
splits[,width]" forces every GEMM's plan and IT_GROUP_SPLITS an FP32 group's split count (planner
measurements only: load it with IRONTENSOR_LIB=...; nothing else uses it).
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
TUNING_LIB = PKG / "libirontensor_hip_tuning.so"
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


def build_tuning_library() -> Path:
    """The library with kernels_gemm.hip under IT_TUNING (plans forced through IT_PLAN), linked with
    the other objects of the last build_library()."""
    tdir = BUILD / "tuning"
    tdir.mkdir(parents=True, exist_ok=True)
    obj = tdir / "kernels_gemm.hip.o"
    cmd = [HIPCC, *HIP_FLAGS, "-DIT_TUNING", "-x", "hip", "-c", str(CSRC / "kernels_gemm.hip"), "-o", str(obj)]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed:\n{res.stdout}")
    objs = [str(BUILD / (name + ".o")) for name in SOURCES if name != "kernels_gemm.hip"] + [str(obj)]
    tmp = TUNING_LIB.with_suffix(".so.tmp")
    res = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *objs],
                         stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}")
    os.replace(tmp, TUNING_LIB)
    return TUNING_LIB


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


SAN_DIR = ROOT / "tests" / "cpp" / "_build" / "sanitize"
CLANG = os.environ.get("CLANGXX", "/opt/rocm/llvm/bin/clang++")
SAN_FLAGS = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g"]


def _clang_rt_dir() -> str:
    """Directory of clang's sanitizer runtimes (libclang_rt.asan-x86_64.so)."""
    res = subprocess.run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"], stdout=subprocess.PIPE, text=True)
    path = Path(res.stdout.strip())
    if not path.is_file():
        hits = sorted(Path(CLANG).resolve().parents[1].glob("lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
        path = hits[-1] if hits else path
    return str(path.parent)


def build_sanitized_host() -> Path:
    """The library's host code (runtime, argument checks, dispatch: the .cpp sources) under
    AddressSanitizer + UndefinedBehaviorSanitizer, linked with the kernel objects of the last
    build_library(), and the C++ host-API test against it: for `test_host_api --cpu`, which needs
    no GPU. Returns the test binary."""
    if not all((BUILD / (n + ".o")).exists() for n in SOURCES if n.endswith(".hip")):
        build_library()
    SAN_DIR.mkdir(parents=True, exist_ok=True)
    procs, objs = [], []
    for name in SOURCES:
        if name.endswith(".hip"):
            objs.append(BUILD / (name + ".o"))
            continue
        obj = SAN_DIR / (name + ".o")
        objs.append(obj)
        cmd = [CLANG, "-std=c++17", "-O1", "-fPIC", *SAN_FLAGS, "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
               f"-I{ROOT / 'include'}", f"-I{CSRC}", "-c", str(CSRC / name), "-o", str(obj)]
        procs.append((name, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    for name, p in procs:
        out, _ = p.communicate()
        if p.returncode != 0:
            raise RuntimeError(f"sanitized build of {name} failed:\n{out}")
    lib = SAN_DIR / "libirontensor_hip.so"
    res = subprocess.run([CLANG, "-shared", "-fPIC", *SAN_FLAGS, "-shared-libsan", "-o", str(lib), *map(str, objs),
                          "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib"],
                         stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"sanitized link failed:\n{res.stdout}")
    exe = SAN_DIR / "test_host_api"
    res = subprocess.run([CLANG, "-std=c++17", "-O1", *SAN_FLAGS, "-shared-libsan", f"-I{ROOT / 'include'}",
                          str(CPP_TEST_SRC), "-o", str(exe), f"-L{SAN_DIR}", "-lirontensor_hip",
                          f"-Wl,-rpath,{SAN_DIR}", "-Wl,-rpath,/opt/rocm/lib",
                          f"-Wl,-rpath,{_clang_rt_dir()}"],
                         stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"sanitized C++ test build failed:\n{res.stdout}")
    return exe


if __name__ == "__main__":
    print(build_library(verbose=True))
    print(build_cpp_tests())
    if "--tuning" in sys.argv[1:]:
        print(build_tuning_library())
