"""Shared pytest setup: the `gpu` marker, import paths and device helpers."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "rust-deeplearning_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


@pytest.fixture(scope="session")
def rq():
    """The product binding (librdlquant.so)."""
    import rdlquant

    return rdlquant


@pytest.fixture(scope="session")
def orc():
    """The CPU restatement (oracle/), the checker."""
    from oracle import oracle

    return oracle


@pytest.fixture(scope="session")
def gpu(rq):
    """Skip-free GPU gate: a `gpu`-marked test fails loudly without a gfx950 device."""
    import torch

    assert torch.cuda.is_available(), "GPU test run without a visible device"
    assert rq.device_count() >= 1, "no gfx950 device visible to librdlquant"
    return torch.device("cuda:0")
