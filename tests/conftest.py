"""Shared test set-up.

Markers: ``gpu`` - needs an MI355X (run with ``-m gpu`` on the GPU box);
everything else runs on the CPU.  The GPU tests call the HIP library
through its C ABI and compare with the CPU oracle (oracle/) on the same
seeded inputs.
"""
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "llama2-min-inference_amd")
for p in (PKG, os.path.join(REPO, "oracle"), REPO):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(REPO, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU (MI355X); run with -m gpu")


def rel_err(a, b) -> float:
    """Norm-wise relative error ||a-b|| / ||b||."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def assert_close(actual, expected, rtol, floor_scale=None, what=""):
    """Elementwise |a-e| <= rtol * max(|e|, floor) where floor defaults to
    the RMS of `expected` (outputs near zero have unbounded relative error,
    so the bound has an absolute floor tied to the vector's scale)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    floor = float(np.sqrt(np.mean(e * e))) if floor_scale is None else float(floor_scale)
    bound = rtol * np.maximum(np.abs(e), floor)
    bad = np.abs(a - e) > bound
    if bad.any():
        i = int(np.argmax(np.abs(a - e) - bound))
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside rtol {rtol} "
                             f"(worst idx {i}: got {a.flat[i]!r}, want {e.flat[i]!r}, floor {floor:.3g})")


@pytest.fixture(scope="session")
def torch_cuda():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    return torch


@pytest.fixture(scope="session")
def gpu_lib(torch_cuda):
    from llama2q import abi
    lib = abi.lib()
    assert lib.l2q_device_count() >= 1
    return abi
