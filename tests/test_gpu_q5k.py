"""GPU parity of Q5_K matrices (attn_output of Q4_K_M checkpoints) through
the C ABI.

The reference runs Q5_K on candle's per-row vec_dot (src/gguf.rs:593),
whose AVX2 code (candle-core 0.11.0, a port of ggml's vec_dot_q5_K_q8_K) is
not in the reference tree.  The oracle restates ggml's published order: the
Q4_K lane structure, the mins as one f32 scalar per row.  Tolerance: the
stated 1e-4 normwise against candle itself (that order is unpinned here);
the tests assert the stronger facts that hold by construction -- outputs
bitwise equal to the oracle's restatement and per-block lane integers
exact.
"""
import numpy as np
import pytest
import torch

from conftest import assert_bitexact, assert_close_normwise
from inferq_amd import qgemm as Q
from inferq_amd import synth as S

pytestmark = pytest.mark.gpu

Q5 = S.Q5_K


@pytest.mark.parametrize("rows,cols", [(96, 512), (2048, 4096), (300, 2048), (7, 256)])
def test_q5k_matches_oracle(gpu, oracle, rows, cols):
    rng = np.random.default_rng(rows + cols)
    w = S.random_matrix(Q5, rows, cols, rng)
    mat = Q.QuantizedMatrix.upload(w, Q5, rows, cols)
    assert mat.dtype() == "Q5K" and mat.storage_bytes() == rows * cols // 256 * 176
    W = oracle.dequantize(Q5, w, rows, cols).astype(np.float64)
    for m in (1, 2, 5, 8, 16, 64):
        x = S.normal((m, cols), np.random.default_rng(m))
        got = mat.forward(torch.from_numpy(x).to(gpu)).cpu().numpy()
        expected = oracle.matmul(Q5, w, rows, cols, x, nthreads=8)
        assert_bitexact(got, expected, f"Q5_K [{rows}x{cols}] m={m}")
        # and the closed form, independent of any lane order
        q = oracle.quantize_q8k(x.reshape(-1))
        xq = (q["qs"].astype(np.float64) * q["d"].astype(np.float64)[:, None]).reshape(m, cols)
        assert_close_normwise(got, xq @ W.T, 1e-4, "Q5_K closed form")


def test_q5k_block_integers_exact(gpu, oracle):
    rng = np.random.default_rng(5)
    rows, cols = 24, 512
    w = S.random_matrix(Q5, rows, cols, rng)
    x = S.normal((3, cols), rng)
    mat = Q.QuantizedMatrix.upload(w, Q5, rows, cols)
    y, isum, msum = mat.block_sums(torch.from_numpy(x).to(gpu))
    isum, msum = isum.cpu().numpy(), msum.cpu().numpy()
    wb = w.view(oracle.BLOCK[Q5]).reshape(rows, cols // 256)
    for r in range(3):
        q = oracle.quantize_q8k(x[r])
        for n in range(rows):
            for b in range(cols // 256):
                ei, em = oracle.block_lanes(Q5, wb[n, b], q[b])
                assert np.array_equal(isum[r, n, b], ei) and np.array_equal(msum[r, n, b], em), (r, n, b)
    assert_bitexact(y.cpu().numpy(), oracle.matmul(Q5, w, rows, cols, x), "block_sums output")


def test_q5k_m_invariance_and_concat(gpu):
    rng = np.random.default_rng(6)
    a = Q.QuantizedMatrix.upload(S.random_matrix(Q5, 512, 2048, rng), Q5, 512, 2048)
    b = Q.QuantizedMatrix.upload(S.random_matrix(Q5, 64, 2048, rng), Q5, 64, 2048)
    x = torch.from_numpy(S.normal((16, 2048), rng)).to(gpu)
    singles = torch.cat([a.forward(x[i:i + 1]) for i in range(16)]).cpu().numpy()
    assert_bitexact(a.forward(x).cpu().numpy(), singles, "Q5_K 16 rows vs one-row calls")
    joined = a.concatenate_rows(b)
    assert_bitexact(joined.forward(x).cpu().numpy(), torch.cat([a.forward(x), b.forward(x)], 1).cpu().numpy(),
                    "Q5_K concatenate_rows")


def test_moe_refuses_unknown_expert_dtypes(gpu):
    from inferq_amd import moe as MOE

    t = torch.zeros(4 * 256 * 176, dtype=torch.uint8, device=gpu)
    with pytest.raises(Q.QgemmError, match="unsupported expert dtypes"):
        MOE.QuantizedMoeLayer(256, 256, 4, 2, 2, S.Q6_K, t, t, t)  # 2 = Q4_0, not executable


@pytest.mark.parametrize("cols", [2048, 4096])
def test_q5k_split_kernels_equal_the_lane_kernel(gpu, cols):
    """At one to eight rows of width 2048 or 4096 the dispatch runs Q5_K on
    the split-K kernels (each wave forms a quarter of the blocks' exact
    lane integers, one chain per row in block order, the mins as one f32
    scalar per row); every row count gives the lane kernel's bits."""
    from inferq_amd import _lib

    rng = np.random.default_rng(cols)
    rows = 1000
    mat = Q.QuantizedMatrix.upload(S.random_matrix(Q5, rows, cols, rng), Q5, rows, cols)
    for m in (1, 2, 3, 4, 6, 7, 8):
        x = torch.from_numpy(S.normal((m, cols), np.random.default_rng(m))).to(gpu)
        assert_bitexact(mat.forward(x).cpu().numpy(), mat.forward_via(x, _lib.PATH_LANES).cpu().numpy(),
                        f"Q5_K [{rows} x {cols}] m={m} split vs lanes")
        assert_bitexact(mat.forward_via(x, _lib.PATH_GEMV).cpu().numpy(), mat.forward(x).cpu().numpy(),
                        f"Q5_K m={m} gemv path")


@pytest.mark.parametrize("rows,cols", [(1000, 2048), (200, 4096), (64, 1024), (5, 256)])
def test_q5k_mfma_tiles_equal_the_lane_kernel(gpu, rows, cols):
    """From 9 rows the dispatch runs Q5_K on the exact lane-order int8 MFMA
    tiles (three scaled-weight streams, the mins as one f32 scalar per row
    and block from one f16 MFMA): the lane kernel's bits at every row count,
    16- and 32-row tiles, ragged row and column tiles."""
    from inferq_amd import _lib

    rng = np.random.default_rng(rows + 7 * cols)
    mat = Q.QuantizedMatrix.upload(S.random_matrix(Q5, rows, cols, rng), Q5, rows, cols)
    for m in (9, 17, 33, 64, 100, 256):
        x = torch.from_numpy(S.normal((m, cols), np.random.default_rng(m))).to(gpu)
        lanes = mat.forward_via(x, _lib.PATH_LANES).cpu().numpy()
        assert_bitexact(mat.forward(x).cpu().numpy(), lanes, f"Q5_K [{rows} x {cols}] m={m} MFMA vs lanes")
        assert_bitexact(mat.forward_via(x, _lib.PATH_LANE_MFMA).cpu().numpy(), lanes, f"Q5_K m={m} explicit path")
