"""Test setup: the package directory on sys.path, the `gpu` marker.

CPU tests (``-m "not gpu"``) check the oracle against golden vectors and
closed forms, the host-side argument checks and the C ABI's exports.  GPU
tests (``-m gpu``) run the HIP kernels through the C ABI on an MI355X and
compare them with the oracle on identical seeded inputs.
"""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "paris-hackathon-2026-inference_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def golden():
    import numpy as np
    z = np.load(os.path.join(REPO, "tests", "golden", "golden_gdn.npz"))
    return {k: z[k] for k in z.files}


def golden_case(golden, name):
    return {k.split(".", 1)[1]: v for k, v in golden.items() if k.startswith(name + ".")}
