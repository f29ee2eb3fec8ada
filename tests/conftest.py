"""Shared fixtures.  GPU tests carry ``@pytest.mark.gpu``; CPU runs use
``-m "not gpu"``.  GPU tests are skipped when torch sees no GPU."""

import importlib
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X (gfx950) GPU")


def pytest_collection_modifyitems(config, items):
    if not any("gpu" in it.keywords for it in items):
        return
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible to torch")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


@pytest.fixture(scope="session")
def fm():
    """The product package (fails loudly if libfmoe.so is not built)."""
    return importlib.import_module("frank-models_amd")


@pytest.fixture(scope="session")
def wl():
    return importlib.import_module("frank-models_amd.workloads")


@pytest.fixture
def gemm_path(fm):
    """Restores the process-wide GEMM path after a test forces one."""
    ll = fm.lowlevel
    yield ll
    ll.lib().fmoe_set_gemm_path(ll.PATH_AUTO)
