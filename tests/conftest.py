"""Shared pytest setup: the `gpu` marker, import paths, and the oracle."""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libunifur_nf4.so on cuda:0)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    O.lib()  # builds oracle/libnf4_oracle.so on first use
    return O


@pytest.fixture(scope="session")
def fixtures():
    import numpy as np
    path = os.path.join(ROOT, "tests", "golden", "nf4_fixtures.npz")
    with np.load(path, allow_pickle=False) as z:
        data = {k: z[k] for k in z.files}
    names = sorted({k.split(".")[0] for k in data})
    return names, data


@pytest.fixture(scope="session")
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test needs a HIP device (run with -m 'not gpu' on a CPU-only host)")
    return torch.device("cuda:0")
