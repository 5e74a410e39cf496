"""Shared fixtures.  GPU tests are marked `gpu`; everything else runs on the CPU."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

GOLDEN = REPO / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built extension")


@pytest.fixture(scope="session")
def ref():
    from oracle.ref import RefEngine

    return RefEngine()


@pytest.fixture(scope="session")
def ext():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test selected but no GPU is visible")
    from cugo_amd import load_extension

    return load_extension()


def announce(name: str) -> None:
    print(f"[case] {name}", flush=True)
