"""Test configuration: the `gpu` marker, import paths and shared fixtures."""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG_DIR = ROOT / "neurips26-tris-moe_amd"
for p in (str(ROOT), str(PKG_DIR)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def oracle_mod():
    import oracle

    oracle._load()
    return oracle


@pytest.fixture(scope="session")
def tris():
    import tris_moe_amd
    from tris_moe_amd import ext, moe, qlinear, synthetic

    tris_moe_amd.load_library()
    return {"ext": ext, "qlinear": qlinear, "synthetic": synthetic, "moe": moe}


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    return torch.device("cuda:0")
