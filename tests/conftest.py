"""pytest setup: import paths and the ``gpu`` marker.

``-m "not gpu"`` runs the oracle checks, host logic and C-ABI export checks on
any machine; ``-m gpu`` runs the HIP parity tests on an MI355X.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "tokamax-tpu-kernel-lab_amd")
for p in (ROOT, PKG_DIR):
  if p not in sys.path:
    sys.path.insert(0, p)


def pytest_configure(config):
  config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built liblmoe.so")


@pytest.fixture(scope="session")
def gpu_device():
  import torch
  if not torch.cuda.is_available():
    pytest.fail("GPU test collected on a machine without a GPU (skip == fail)")
  return torch.device("cuda:0")
