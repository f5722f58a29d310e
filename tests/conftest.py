"""Shared fixtures.  GPU tests are marked ``gpu``; everything else runs on CPU."""
from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libcx_moe.so)")


@pytest.fixture(scope="session")
def oracle():
    from oracle.oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def refcpu():
    from oracle.oracle import RefCpu
    if not RefCpu.available():
        pytest.skip("oracle/_ref (reference C++ CPU build) not present")
    return RefCpu()


@pytest.fixture(scope="session")
def gpu():
    """Session GPU context; fails loudly (never skips) when the library or GPU is missing."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    from constellation_amd.engine import Context
    ctx = Context(0)
    yield ctx
    torch.cuda.synchronize()
    ctx.close()


def flush(msg: str) -> None:
    print(msg, flush=True)
