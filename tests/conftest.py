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


def normal_bf16_values():
    """Every normal bf16 value and +0 (65,025 values), in bit-pattern order.  (Left out: -0 and the
    254 denormals, which torch's CPU conv turns into +0 -- it flushes denormals and adds to +0 -- and
    whose SiLU is within 1e-38 of 0 either way.)"""
    x = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    xf = x.float()
    return x[torch.isfinite(xf) & ((xf.abs() >= 2.0 ** -126) | (x.view(torch.int16) == 0))]


def assert_same_bits(got, want, inputs):
    """got == want bit for bit; the message lists the first inputs where they differ."""
    got, want = got.cpu().reshape(-1), want.cpu().reshape(-1)
    bad = got.view(torch.int16) != want.view(torch.int16)
    assert not bad.any(), (f"{int(bad.sum())} of {bad.numel()} differ; (input, got, want): "
                           f"{list(zip(inputs.reshape(-1)[bad][:8].tolist(), got[bad][:8].tolist(), want[bad][:8].tolist()))}")
