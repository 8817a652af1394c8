"""GPU parity of the int8-MFMA prefill-tile path (Q4_K, 64 or more input
rows), which a caller requests explicitly (iq_matmul_via with
IQ_PATH_PREFILL_TILES; the dispatch never picks it), through the C ABI.

Tolerance: per-block integers (the block's total integer dot and its mins
term) are compared bit for bit with the oracle; outputs within a normwise
relative error of 1e-4 per output row (max_j |g - r| / max_j |r|), the
path's stated f32 bar -- this path combines the block integers in f32 in a
different order than the reference's per-lane FMA chains.
"""
import numpy as np
import pytest
import torch

from conftest import assert_bitexact, assert_close_normwise
from inferq_amd import _lib
from inferq_amd import qgemm as Q
from inferq_amd import synth as S

pytestmark = pytest.mark.gpu

Q4 = S.Q4_K


def _rowwise_close(got, ref, tol, what):
    for r in range(ref.shape[0]):
        assert_close_normwise(got[r], ref[r], tol, f"{what} row {r}")


@pytest.mark.parametrize("rows,cols,m,sample", [(40, 512, 70, None), (8192, 512, 256, 4000)])
def test_prefill_block_integers_exact(gpu, oracle, rows, cols, m, sample):
    """Every (row, column, block) integer pair of a ragged call on the
    small 32 x 64 tiles (70 rows, not a multiple of 16; 40 columns, not a
    multiple of 32), and a seeded sample of the pairs of a call that fills
    the GPU with the large 64 x 128 tiles, equal the oracle's textbook
    integers."""
    rng = np.random.default_rng(61 + rows)
    w = S.random_matrix(Q4, rows, cols, rng)
    x = S.normal((m, cols), rng)
    mat = Q.QuantizedMatrix.upload(w, Q4, rows, cols)
    y, isum, msum = mat.prefill_block_sums(torch.from_numpy(x).to(gpu))
    isum, msum = isum.cpu().numpy(), msum.cpu().numpy()
    wb = w.view(oracle.BLOCK[Q4]).reshape(rows, cols // 256)
    if sample is None:
        picks = [(t, n, b) for t in range(m) for n in range(rows) for b in range(cols // 256)]
    else:
        picks = list(zip(rng.integers(0, m, sample), rng.integers(0, rows, sample), rng.integers(0, cols // 256, sample)))
    qs = {}
    for t, n, b in picks:
        if t not in qs:
            qs[t] = oracle.quantize_q8k(x[t])
        ti, tm = oracle.block_textbook(Q4, wb[n, b], qs[t][b])
        assert isum[t, n, b] == ti and msum[t, n, b] == tm, (t, n, b)
    _rowwise_close(y.cpu().numpy(), oracle.matmul(Q4, w, rows, cols, x, nthreads=8), 1e-4, "prefill product")


@pytest.mark.parametrize("rows,cols,m", [(8192, 2048, 256), (1024, 2048, 256), (2048, 4096, 256), (300, 2048, 100),
                                         (64, 256, 64)])
def test_prefill_matches_oracle(gpu, oracle, rows, cols, m):
    """BASELINE configs[3] shapes: [256 x 2048] -> 8192 at full size (256
    large tiles) and [256 x 4096] -> 2048 (256 unsplit small tiles);
    [1024 x 2048] (small tiles split over K) and ragged sizes."""
    rng = np.random.default_rng(rows + cols + m)
    w = S.random_matrix(Q4, rows, cols, rng)
    x = S.normal((m, cols), rng)
    mat = Q.QuantizedMatrix.upload(w, Q4, rows, cols)
    got = mat.forward_via(torch.from_numpy(x).to(gpu), _lib.PATH_PREFILL_TILES).cpu().numpy()
    ref = oracle.matmul(Q4, w, rows, cols, x, nthreads=8)
    _rowwise_close(got, ref, 1e-4, f"prefill [{rows}x{cols}] m={m}")


def test_prefill_is_deterministic(gpu):
    rng = np.random.default_rng(62)
    w = S.random_matrix(Q4, 2048, 4096, rng)
    mat = Q.QuantizedMatrix.upload(w, Q4, 2048, 4096)
    x = torch.from_numpy(S.normal((256, 4096), rng)).to(gpu)
    a = mat.forward_via(x, _lib.PATH_PREFILL_TILES).cpu().numpy()
    b = mat.forward_via(x, _lib.PATH_PREFILL_TILES).cpu().numpy()
    assert_bitexact(a, b, "run to run")


def test_prefill_tiles_only_on_request(gpu, oracle):
    """The dispatch keeps the reference's bits at 64+ rows; the tile path
    runs only when asked for, and refuses what it does not cover."""
    rng = np.random.default_rng(63)
    w = S.random_matrix(Q4, 256, 2048, rng)
    x = S.normal((64, 2048), rng)
    mat = Q.QuantizedMatrix.upload(w, Q4, 256, 2048)
    xt = torch.from_numpy(x).to(gpu)
    assert_bitexact(mat.forward(xt).cpu().numpy(), oracle.matmul(Q4, w, 256, 2048, x, nthreads=8), "dispatch, 64 rows")
    _rowwise_close(mat.forward_via(xt, _lib.PATH_PREFILL_TILES).cpu().numpy(),
                   oracle.matmul(Q4, w, 256, 2048, x, nthreads=8), 1e-4, "tiles, 64 rows")
    with pytest.raises(Q.QgemmError, match="prefill tiles kernel for 63 input rows"):
        mat.forward_via(xt[:63], _lib.PATH_PREFILL_TILES)
    q6 = Q.QuantizedMatrix.upload(S.random_matrix(S.Q6_K, 64, 2048, rng), S.Q6_K, 64, 2048)
    with pytest.raises(Q.QgemmError, match="Q6K has no prefill tiles kernel"):
        q6.forward_via(xt, _lib.PATH_PREFILL_TILES)
