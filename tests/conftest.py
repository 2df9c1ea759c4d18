"""Shared test setup: import paths, the `gpu` marker, device fixtures and the
parity metrics used throughout (bf16: relative L2 error + cosine similarity;
fp32: element-wise |d| <= 1e-5 * max(|ref|, 1))."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "diffusers-cpp_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

# Tolerances of the parity contract.
FP32_TOL = 1e-5          # element-wise, relative to max(|ref|, 1)
BF16_REL_L2 = 1e-2       # ||y - ref||_2 / ||ref||_2
BF16_COS = 0.9999        # cosine similarity


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.load()
    return oracle


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import dit_hip
    dit_hip.load()
    return torch.device("cuda:0")


def assert_fp32(actual, expected, tol=FP32_TOL, what=""):
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, f"{what}: shape {a.shape} != {e.shape}"
    bound = tol * np.maximum(np.abs(e), 1.0)
    err = np.abs(a - e)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err / bound), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} of {err.size} elements exceed {tol} "
                             f"(worst at {i}: got {a[i]!r}, want {e[i]!r})")


def bf16_metrics(actual, expected):
    a = np.asarray(actual, dtype=np.float64).ravel()
    e = np.asarray(expected, dtype=np.float64).ravel()
    rel = np.linalg.norm(a - e) / max(np.linalg.norm(e), 1e-30)
    cos = float(a @ e / max(np.linalg.norm(a) * np.linalg.norm(e), 1e-30))
    return rel, cos


def assert_bf16(actual, expected, what=""):
    rel, cos = bf16_metrics(actual, expected)
    assert rel <= BF16_REL_L2 and cos >= BF16_COS, f"{what}: rel_l2={rel:.3e} cos={cos:.6f}"
