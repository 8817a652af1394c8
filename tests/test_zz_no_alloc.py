"""The allocation-free product (iq_matmul_noalloc) through the C ABI: two
calls in a row, the second with fewer rows, each bitwise equal to
iq_matmul's output on the same inputs (the same kernels, a fixed scratch
array instead of the library workspace); oversized calls are refused
before any launch.  Collected last, so a failure here hides no other test.
"""
import ctypes

import numpy as np
import pytest
import torch

from conftest import assert_bitexact
from inferq_amd import _lib
from inferq_amd import qgemm as Q
from inferq_amd import synth as S

pytestmark = pytest.mark.gpu


def _noalloc(mat, x, m, y):
    rc = _lib.lib().iq_matmul_noalloc(mat.handle, x.data_ptr(), m, y.data_ptr(),
                                      ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(rc)


@pytest.mark.parametrize("dtype,rows,cols,m1,m2", [
    (S.Q4_K, 8192, 2048, 40, 3),    # exact lane-order MFMA tile, then split-K GEMV
    (S.Q6_K, 40960, 2048, 8, 1),    # LM-head-like: MFMA tile at 8 rows, GEMV at 1
    (S.Q8_0, 4096, 2048, 70, 9),    # lane kernel, then GEMV tiles
    (S.Q5_K, 2048, 4096, 16, 2),    # lane kernel
    (S.Q4_K, 1024, 2048, 256, 64),  # prefill widths on the MFMA tile
])
def test_noalloc_equals_matmul_on_two_calls(gpu, dtype, rows, cols, m1, m2):
    g = torch.Generator(device=gpu).manual_seed(rows + m1)
    mat = Q.QuantizedMatrix.view(S.random_matrix_device(dtype, rows, cols, gpu, rows + dtype), dtype, rows, cols)
    for m in (m1, m2):
        x = torch.randn(m, cols, device=gpu, generator=g)
        y = torch.full((m, rows), float("nan"), device=gpu)
        _noalloc(mat, x, m, y)
        assert_bitexact(y.cpu().numpy(), mat.forward(x).cpu().numpy(), f"{S.NAMES[dtype]} m={m}")


def test_noalloc_refuses_oversized_calls(gpu):
    L = _lib.lib()
    cap = L.iq_matmul_noalloc_max_bytes()
    assert cap == 16 << 20
    mat = Q.QuantizedMatrix.view(S.random_matrix_device(S.Q8_0, 64, 4096, gpu, 5), S.Q8_0, 64, 4096)
    m = 8192
    assert L.iq_matmul_workspace_size(mat.handle, m) > cap
    x = torch.zeros(m, 4096, device=gpu)
    y = torch.zeros(m, 64, device=gpu)
    with pytest.raises(_lib.QgemmError, match="need .* bytes of scratch"):
        _noalloc(mat, x, m, y)
    # the library still works after the refusal
    x2 = torch.randn(4, 4096, device=gpu)
    y2 = torch.empty(4, 64, device=gpu)
    _noalloc(mat, x2, 4, y2)
    assert_bitexact(y2.cpu().numpy(), mat.forward(x2).cpu().numpy(), "after a refused call")
