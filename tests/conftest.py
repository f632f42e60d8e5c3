import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "qe-qwen36-b50_amd")
ORACLE = os.path.join(REPO, "oracle")
for p in (PKG, ORACLE, REPO):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


def pytest_sessionstart(session):
    # the checker is plain g++; build it if this tree has no copy yet
    if not os.path.exists(os.path.join(ORACLE, "libqe_oracle.so")):
        subprocess.run(["make", "-s", "-C", ORACLE], check=True)


@pytest.fixture(scope="session")
def torch_cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    return torch
