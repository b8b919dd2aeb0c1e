"""The CPU oracle and the library's host code under AddressSanitizer + UndefinedBehaviorSanitizer
(no GPU needed): every oracle function once on small ragged shapes (oracle/sanitize_check.c,
`make -C oracle sanitize`); the C++ host-API test's CPU cases and the Python ABI tests against the
library whose host objects (runtime, argument checks, dispatch) are instrumented
(irontensor_amd.build.build_sanitized_host). Any sanitizer report fails the test."""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
REPORTS = ("ERROR: AddressSanitizer", "runtime error:", "ERROR: LeakSanitizer")


def _clean(out: str) -> None:
    for marker in REPORTS:
        assert marker not in out, out[-4000:]


def test_oracle_under_sanitizers():
    res = subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "sanitize"], stdout=subprocess.PIPE,
                         stderr=subprocess.STDOUT, text=True, timeout=300)
    print(res.stdout)
    assert res.returncode == 0, res.stdout
    assert "oracle sanitize check: ok" in res.stdout
    _clean(res.stdout)


def test_host_code_under_sanitizers():
    from irontensor_amd.build import SAN_DIR, _clang_rt_dir, build_sanitized_host
    exe = build_sanitized_host()
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1")
    res = subprocess.run([str(exe), "--cpu"], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                         timeout=300, env=env)
    print(res.stdout)
    assert res.returncode == 0, res.stdout
    _clean(res.stdout)
    # The ABI tests (argument checks of every entry point, no device) through the instrumented library.
    # The ASan runtime goes first in the preload list (kept ahead of any entries already there).
    preload = [str(Path(_clang_rt_dir()) / "libclang_rt.asan-x86_64.so")]
    if os.environ.get("LD_PRELOAD"):
        preload.append(os.environ["LD_PRELOAD"])
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0", LD_PRELOAD=":".join(preload),
               IRONTENSOR_LIB=str(SAN_DIR / "libirontensor_hip.so"))
    res = subprocess.run([sys.executable, "-m", "pytest", "-q", "-s", "-p", "no:cacheprovider", "-m", "not gpu",
                          str(ROOT / "tests" / "test_abi.py")], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                         text=True, timeout=600, env=env, cwd=str(ROOT))
    print(res.stdout[-3000:])
    assert res.returncode == 0, res.stdout[-4000:]
    _clean(res.stdout)
