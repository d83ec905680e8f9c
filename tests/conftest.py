"""Test configuration: the `gpu` marker and import paths.

`-m "not gpu"` runs on any machine (oracle checks, host logic, the C ABI
without compute calls); `-m gpu` needs an MI355X and runs the parity tests
through the C ABI.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "llama.zig_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU (MI355X); runs the HIP kernels")


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test on a machine without a GPU: run with -m 'not gpu'")
    return torch.device("cuda:0")
