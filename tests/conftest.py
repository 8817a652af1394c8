import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP kernels through the C ABI")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O

    O.lib()
    return O


@pytest.fixture(scope="session")
def gpu():
    """Initialise device 0 for the C ABI (fails loudly without a GPU)."""
    import torch

    from inferq_amd import qgemm

    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    qgemm.init(0)
    return torch.device("cuda", 0)


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_bitexact(actual: np.ndarray, expected: np.ndarray, what: str = "") -> None:
    """Bit-identical f32 arrays; on failure report the normwise error too."""
    actual = np.asarray(actual, np.float32)
    expected = np.asarray(expected, np.float32)
    assert actual.shape == expected.shape, (actual.shape, expected.shape)
    if not np.array_equal(bits(actual), bits(expected)):
        diff = np.abs(actual.astype(np.float64) - expected)
        n = int((bits(actual) != bits(expected)).sum())
        rel = diff.max() / max(np.abs(expected).max(), 1e-30)
        raise AssertionError(f"{what}: {n}/{actual.size} values differ; normwise rel err {rel:.3e}")


def assert_close_normwise(actual, expected, tol=1e-4, what=""):
    """max_i |a-e| / max_i |e| <= tol (the path's stated f32 tolerance)."""
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    scale = max(np.abs(expected).max(), 1e-30)
    err = np.abs(actual - expected).max() / scale
    assert err <= tol, f"{what}: normwise rel err {err:.3e} > {tol}"
