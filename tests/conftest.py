"""Test configuration: import paths, the `gpu` marker, shared helpers.

`-m "not gpu"` runs on any host (oracle pins, host logic, C-ABI loading).  `-m gpu` runs the HIP kernels on an
MI355X and compares them with the CPU oracle (tests only use the oracle as the checker).
"""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROJECT = os.path.join(REPO, "rwkv-infer-next_amd")
for p in (REPO, PROJECT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP kernels); run with -m gpu")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    oracle.build()
    return oracle


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False
