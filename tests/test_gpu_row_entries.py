"""GPU parity of the per-row entries in the reference's argument order
(q4k_q8k_row / q6k_q8k_row / q80_q80_row, src/qgemm.rs:447-468) through the
C ABI: one weight row against block-major quantised inputs, bitwise equal
to the oracle's restatement of the same kernel."""
import numpy as np
import pytest

from conftest import assert_bitexact
from inferq_amd import qgemm as Q
from inferq_amd import synth as S

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,cols", [(S.Q4_K, 2048), (S.Q6_K, 4096), (S.Q8_0, 2048), (S.Q6_K, 768),
                                        (S.Q8_0, 96)])
def test_row_entries_match_the_oracle(gpu, oracle, dtype, cols):
    rng = np.random.default_rng(cols + dtype)
    wrow = S.random_matrix(dtype, 1, cols, rng)
    for rows in (1, 3, 8, 16):
        x = S.normal((rows, cols), rng)
        q = np.stack([oracle.quantize_q80(r) if dtype == S.Q8_0 else oracle.quantize_q8k(r) for r in x])
        block_major = np.ascontiguousarray(q.T)  # inputs[block * rows + r]
        got = Q.row_kernel(dtype, wrow, block_major, rows)
        expected = oracle.row_kernel(dtype, wrow.view(oracle.BLOCK[dtype]), block_major, rows, impl="lanes")
        assert_bitexact(got, expected, f"{S.NAMES[dtype]} cols={cols} rows={rows}")
        # and the matrix-level product of the same row agrees
        assert_bitexact(got, oracle.matmul(dtype, wrow, 1, cols, x)[:, 0], "row entry vs matmul")
