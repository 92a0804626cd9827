"""pytest configuration: the `gpu` marker and import paths.

CPU tests (``-m "not gpu"``) check the oracle against golden vectors, closed forms
and brute force, and check that the C-ABI library loads and exports its symbols.
GPU tests (``-m gpu``) call the HIP library through the C ABI and compare with the
oracle on the same seeded inputs.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "star-kv-serve_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda", 0)
