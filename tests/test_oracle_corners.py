"""The oracle's two restatements of the row kernels (AVX2 intrinsics and
scalar lanes, src/qgemm.rs:99-443) on corner-byte blocks: every payload
byte 0xFF, 0x00, 0x80 or a mix of corner bytes, against activation rows
at the Q8K / Q8_0 extremes (constant rows, a zero row, alternating signs,
mixed magnitudes).  The two share no code past the block layout, so a
sign, shift or carry slip at a corner shows as a difference; the GPU
corner tests compare against the same restatement."""
import numpy as np
import pytest

from test_gpu_extreme_blocks import FMT_IDS, FORMATS, corner_activations, corner_matrix


@pytest.mark.parametrize("mode", ["ff", "00", "80", "mix"])
@pytest.mark.parametrize("dtype", FORMATS, ids=FMT_IDS)
def test_corner_blocks_avx2_equals_lanes(oracle, dtype, mode):
    if not oracle.have_avx2():
        pytest.skip("no AVX2 on this host")
    rows, cols = 64, 2048
    w = corner_matrix(dtype, rows, cols, mode, 17 + len(mode))
    x = corner_activations(12, cols, 5)
    a = oracle.matmul(dtype, w, rows, cols, x, impl=1)
    b = oracle.matmul(dtype, w, rows, cols, x, impl=0)
    assert np.isfinite(a).all()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"dtype {dtype} bytes {mode}"
    assert not np.any(a[3::6]), "a zero activation row gives zero outputs"
