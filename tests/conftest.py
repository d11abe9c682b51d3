"""Shared pytest configuration.

Markers:
  gpu  -- needs a ROCm device and the built HIP library; run with ``-m gpu``.
Everything unmarked runs on the CPU (oracle pinning, host logic, C-ABI load).
"""

from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: requires a ROCm GPU and the built libmsa_mi355x.so")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda:0")


def cu_of(lengths):
    import torch

    out = [0]
    for n in lengths:
        out.append(out[-1] + n)
    return torch.tensor(out, dtype=torch.int32)
