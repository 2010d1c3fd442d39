"""Shared pytest configuration.

``-m "not gpu"`` runs the oracle pins, the host scheduling checks and the C-ABI
library checks on the CPU; ``-m gpu`` runs the parity tests of the HIP engine on an
MI355X through the op surface and the C ABI.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "persistentkv-attention_amd")
for _p in (PKG, ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

MAX_ABS = 2e-3   # north-star tolerance (max-abs vs the fp32 SDPA oracle)
MEAN_ABS = 3e-4  # the reference's mean gate (tests/smoke_test.cu:106)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X; runs the HIP engine")


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def ext(gpu):
    """The op module.  Import errors are not skipped: on a GPU machine a missing native
    extension must fail the test."""
    import persistentkv_torch_ext
    return persistentkv_torch_ext
