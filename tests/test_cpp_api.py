"""Runs the C++ host-API test program (tests/cpp/test_host_api.cpp, built by build())."""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

BIN = Path(__file__).resolve().parent / "cpp" / "_build" / "test_host_api"


def _run(*args):
    if not BIN.exists():
        pytest.fail(f"{BIN} is missing: run __graft_entry__.build() first")
    res = subprocess.run([str(BIN), *args], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                         text=True, timeout=300)
    print(res.stdout)
    return res


def test_cpp_host_api_cpu():
    res = _run("--cpu")
    assert res.returncode == 0, res.stdout


@pytest.mark.gpu
def test_cpp_host_api_gpu():
    res = _run()
    assert res.returncode == 0, res.stdout
    assert " 0 failed" in res.stdout
