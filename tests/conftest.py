"""Test configuration: the ``gpu`` marker and shared helpers.

``-m "not gpu"`` tests run on the CPU (oracle pinning, dispatch contracts,
C-ABI exports). ``-m gpu`` tests need an MI355X and compare the HIP kernels
with the CPU oracle.
"""

import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def device():
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    return torch.device("cuda", 0)


def max_rel(actual, expected):
    """Largest |a - e| over the largest |e| (worst-relative error)."""
    a = actual.double().cpu()
    e = expected.double().cpu()
    return float((a - e).abs().max() / e.abs().max().clamp_min(1e-30))


def frob_rel(actual, expected):
    a = actual.double().cpu()
    e = expected.double().cpu()
    return float((a - e).norm() / e.norm().clamp_min(1e-30))


def worst_cell_rel(actual, expected, row_bounds, block=128):
    """Largest relative Frobenius error over the output's cells: the rows of
    each group (between consecutive ``row_bounds``) by each ``block``-column
    slice; empty groups are skipped. This is the reference's GEMM metric
    (tests/test_block_fp8_transpose_gemm.py:390-406)."""
    a = actual.double().cpu().reshape(-1, actual.shape[-1])
    e = expected.double().cpu().reshape(-1, expected.shape[-1])
    worst = 0.0
    for lo, hi in zip(row_bounds[:-1], row_bounds[1:]):
        if hi <= lo:
            continue
        for col in range(0, e.shape[1], block):
            ac, ec = a[lo:hi, col:col + block], e[lo:hi, col:col + block]
            worst = max(worst, float((ac - ec).norm() / ec.norm().clamp_min(1e-6)))
    return worst
