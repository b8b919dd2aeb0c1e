"""Shared fixtures. GPU tests are marked `gpu`; CPU tests cover the oracle, fixtures and ABI."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X) and the built library")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o

    o.load()
    return o


@pytest.fixture(scope="session")
def it():
    """The product package with a live device context. Fails (never skips) without a device: the
    GPU tests must run the HIP path or report why they could not."""
    import irontensor_amd as it_pkg

    if it_pkg.device_count() == 0:
        pytest.fail("no HIP device visible: GPU tests need the MI355X box")
    ctx = it_pkg.Context.global_()
    print(f"[device] {ctx.info()}", flush=True)
    return it_pkg
