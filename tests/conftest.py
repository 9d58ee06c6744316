"""Shared pytest setup: import paths, the `gpu` marker and device helpers."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
for p in (REPO / "flash-mlm_amd", REPO):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = REPO / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built libflash_mlm_hip.so")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from flash_mlm import _lib

    _lib.load()  # fail loudly if the native library is missing
    return torch.device("cuda", 0)


@pytest.fixture(autouse=True)
def _print_case(request):
    # name the case before any GPU step, so a fault can be attributed
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[case] {request.node.nodeid}", flush=True)
    yield
