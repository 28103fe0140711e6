import importlib
import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PKG_NAME = "910b_e2e_accleration_by_codex_amd"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def gdn():
    """The package (its HIP library is loaded lazily on the first op)."""
    return importlib.import_module(PKG_NAME)


@pytest.fixture(scope="session")
def oracle():
    return importlib.import_module("oracle.gdn_oracle")


@pytest.fixture(scope="session")
def dev(gdn):
    """cuda:0 with the HIP library loaded; GPU tests fail (not skip) without them."""
    assert torch.cuda.is_available(), "GPU test run without a visible ROCm GPU"
    from importlib import import_module
    import_module(PKG_NAME + "._lib").lib()
    return torch.device("cuda:0")


def rel_l2(a, b):
    a = a.double().cpu()
    b = b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()
