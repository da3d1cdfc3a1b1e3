"""Shared pytest configuration.

* registers the ``gpu`` marker (tests that need an MI355X);
* puts the repository root, ``oracle/`` and the package directory on sys.path.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "gdn-recoverssm-ascend_amd")
for p in (ROOT, os.path.join(ROOT, "oracle"), PKG_DIR):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def gpu_device():
    """cuda:0. A GPU test selected on a host without a GPU fails here rather
    than being skipped, so a missing device never passes as a green run."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no HIP device is visible")
    return torch.device("cuda:0")
