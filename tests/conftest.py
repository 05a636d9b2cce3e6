"""Shared test fixtures.

CPU tests (-m "not gpu") check the oracle against what pins it, the host
logic and that the C-ABI library loads and exports what include/*.h declares.
GPU tests (-m gpu) are the parity tests: HIP path through the C-ABI vs the
oracle on the same seeded inputs.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

from __graft_entry__ import load_package  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through the HIP C-ABI")


SEED = 410293  # the reference's default seed (edm/main_edm.c:63, ddpm/main_ddpm.c:112)


@pytest.fixture(scope="session")
def nn():
    return load_package()


@pytest.fixture(scope="session")
def L(nn):
    """The loaded HIP library; GPU tests fail loudly when it or the GPU is missing."""
    lib = nn.lib()
    if lib.device_count() < 1:
        raise RuntimeError("no HIP device visible to a gpu-marked test")
    info = lib.device_info()
    print(f"\n[device] {info}", flush=True)
    return lib


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as o

    return o


@pytest.fixture
def rng():
    return np.random.default_rng(SEED)
