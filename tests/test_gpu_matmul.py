"""GPU parity of the quantised matmul through the C ABI.

Tolerance: the path's stated bar is per-block integers bit-exact and f32
outputs within a normwise relative error of 1e-4.  These kernels follow the
reference's per-lane f32 order, so the tests assert the stronger property:
every output is bit-identical to the oracle (the reference's fused kernel
restated), and the per-block lane integers are identical.
"""
import numpy as np
import pytest
import torch

from conftest import assert_bitexact
from inferq_amd import qgemm as Q
from inferq_amd import synth as S

pytestmark = pytest.mark.gpu

Q4, Q6, Q8 = S.Q4_K, S.Q6_K, S.Q8_0

# (dtype, rows, cols): the reference test matrix shape [96 x 512] for each
# format (src/gguf.rs:1630-1677), the BASELINE shapes, ragged row counts
# (not a multiple of 8 or 4, down to matrices of fewer rows than one GEMV
# row group) and an odd number of Q6_K blocks per row.  Widths
# whose block count suits the GEMV kernel (iq_gemv.hip) run it, in tiles of
# 8 rows past 8 input rows (up to 63 on matrices this small); the others run
# the lane kernel (iq_lanes.hip).
SHAPES = [
    (Q4, 96, 512), (Q6, 96, 512), (Q8, 96, 512),
    (Q4, 1024, 2048), (Q6, 2048, 512), (Q8, 4096, 2048),
    (Q4, 2048, 4096), (Q6, 37, 768), (Q8, 45, 96), (Q4, 13, 256),
    (Q6, 300, 2048), (Q6, 64, 4096), (Q4, 77, 2048), (Q8, 19, 1024), (Q6, 5, 6144), (Q8, 40, 4096),
    (Q8, 3, 2048), (Q8, 1, 4096), (Q4, 2, 2048), (Q6, 3, 4096),
]
ROWS = [1, 2, 3, 4, 7, 8, 9, 15, 16, 17, 33, 48, 63]


def _case(dtype, rows, cols, m, seed):
    rng = np.random.default_rng(seed)
    w = S.random_matrix(dtype, rows, cols, rng)
    x = S.normal((m, cols), rng)
    return w, x


@pytest.mark.parametrize("dtype,rows,cols", SHAPES)
def test_matmul_bitexact_across_row_counts(gpu, oracle, dtype, rows, cols):
    w, _ = _case(dtype, rows, cols, 1, seed=rows * 131 + cols + dtype)
    mat = Q.QuantizedMatrix.upload(w, dtype, rows, cols)
    assert mat.shape() == [rows, cols] and mat.storage_bytes() == w.size
    for m in ROWS:
        x = S.normal((m, cols), np.random.default_rng(1000 + m))
        expected = oracle.matmul(dtype, w, rows, cols, x, impl=0)
        got = mat.forward(torch.from_numpy(x).to(gpu)).cpu().numpy()
        assert_bitexact(got, expected, f"{S.NAMES[dtype]} [{rows}x{cols}] m={m}")


@pytest.mark.parametrize("dtype,rows,cols", [(Q4, 64, 512), (Q6, 40, 512), (Q8, 24, 256)])
def test_block_lane_integers_bitexact(gpu, oracle, dtype, rows, cols):
    w, x = _case(dtype, rows, cols, 3, seed=7)
    mat = Q.QuantizedMatrix.upload(w, dtype, rows, cols)
    y, isum, msum = mat.block_sums(torch.from_numpy(x).to(gpu))
    isum = isum.cpu().numpy()
    msum = msum.cpu().numpy() if msum is not None else None
    nb = cols // S.BLOCK_ELEMS[dtype]
    wb = w.view(oracle.BLOCK[dtype]).reshape(rows, nb)
    for r in range(x.shape[0]):
        q = oracle.quantize_q80(x[r]) if dtype == Q8 else oracle.quantize_q8k(x[r])
        for n in range(rows):
            for b in range(nb):
                ei, em = oracle.block_lanes(dtype, wb[n, b], q[b])
                assert np.array_equal(isum[r, n, b], ei), (r, n, b)
                if em is not None:
                    assert np.array_equal(msum[r, n, b], em), (r, n, b)
    assert_bitexact(y.cpu().numpy(), oracle.matmul(dtype, w, rows, cols, x), "block_sums output")


def _edge_rows(k, rng):
    rows = [
        np.zeros(k, np.float32),                         # amax == 0: d = 0, q = 0
        S.normal(k, rng),
        np.where(np.arange(k) == 5, np.float32(-3.0), np.float32(0)),  # one nonzero (negative max)
        np.tile(np.float32([1.0, -1.0]), k // 2),        # |max| tied everywhere: first index wins
        (np.arange(k, dtype=np.float32) - k / 2) / 64,   # values on exact .5 ties after scaling
        S.normal(k, rng) * np.float32(1e-30),            # tiny magnitudes
        S.normal(k, rng) * np.float32(1e30),             # huge magnitudes
    ]
    return np.stack(rows).astype(np.float32)


def test_quantize_q8k_bitexact(gpu, oracle):
    rng = np.random.default_rng(3)
    x = _edge_rows(1024, rng)
    got = Q.quantize_q8k(torch.from_numpy(x).to(gpu)).cpu().numpy()
    expected = np.concatenate([oracle.quantize_q8k(r) for r in x]).view(np.uint8)
    assert np.array_equal(got, expected.reshape(-1))


def test_quantize_q80_bitexact(gpu, oracle):
    rng = np.random.default_rng(4)
    x = _edge_rows(512, rng)
    got = Q.quantize_q80(torch.from_numpy(x).to(gpu)).cpu().numpy()
    expected = np.concatenate([oracle.quantize_q80(r) for r in x]).view(np.uint8)
    assert np.array_equal(got, expected.reshape(-1))


@pytest.mark.parametrize("m", [1, 8])
def test_lm_head_slice_bitexact(gpu, oracle, m):
    """A 20000-row slice of the Q6_K LM head shape [248320 x 2048]: many row
    groups per wave in the LDS-staged kernel."""
    rng = np.random.default_rng(4242 + m)
    w = S.random_matrix(Q6, 20000, 2048, rng)
    x = S.normal((m, 2048), rng)
    mat = Q.QuantizedMatrix.upload(w, Q6, 20000, 2048)
    got = mat.forward(torch.from_numpy(x).to(gpu)).cpu().numpy()
    assert_bitexact(got, oracle.matmul(Q6, w, 20000, 2048, x, nthreads=8), f"LM-head slice m={m}")


def test_m_invariance_bitwise(gpu):
    """One row alone equals the same row inside 4-, 8- and 16-row passes
    (tests/speculative_policy.rs:373-450 in the reference)."""
    rng = np.random.default_rng(11)
    for dtype, rows, cols in [(Q4, 512, 2048), (Q6, 512, 2048), (Q8, 512, 2048)]:
        w = S.random_matrix(dtype, rows, cols, rng)
        mat = Q.QuantizedMatrix.upload(w, dtype, rows, cols)
        x = torch.from_numpy(S.normal((16, cols), rng)).to(gpu)
        singles = torch.cat([mat.forward(x[i:i + 1]) for i in range(16)]).cpu().numpy()
        for m in (4, 8, 16):
            multi = mat.forward(x[:m]).cpu().numpy()
            assert_bitexact(multi, singles[:m], f"{S.NAMES[dtype]} m={m}")


def test_concatenated_rows_match_separate_matrices(gpu):
    rng = np.random.default_rng(5)
    for dtype in (Q4, Q6, Q8):
        a = Q.QuantizedMatrix.upload(S.random_matrix(dtype, 16, 512, rng), dtype, 16, 512)
        b = Q.QuantizedMatrix.upload(S.random_matrix(dtype, 24, 512, rng), dtype, 24, 512)
        c = a.concatenate_rows(b)
        assert c.shape() == [40, 512]
        x = torch.from_numpy(S.normal((3, 512), rng)).to(gpu)
        expected = torch.cat([a.forward(x), b.forward(x)], dim=1).cpu().numpy()
        assert_bitexact(c.forward(x).cpu().numpy(), expected, "concatenate_rows")
        lead = c.leading_rows(16)
        assert_bitexact(lead.forward(x).cpu().numpy(), a.forward(x).cpu().numpy(), "leading_rows")


@pytest.fixture(scope="module")
def large_matrices():
    """Matrices past the size where 2..63-row calls take the exact-order MFMA
    kernel (iq_dense_mfma.hip) and one-row calls the four-row GEMV items:
    Q6_K [40962 x 2048] (68.8 MB, LM-head-like) and Q4_K [61441 x 2048]
    (70.8 MB); neither row count is a multiple of 4 or 8, so every kernel
    ends on a ragged group."""
    rng = np.random.default_rng(77)
    return {Q6: (S.random_matrix(Q6, 40962, 2048, rng), 40962), Q4: (S.random_matrix(Q4, 61441, 2048, rng), 61441)}


@pytest.mark.parametrize("dtype", [Q6, Q4], ids=["q6k", "q4k"])
def test_large_matrix_rows_bitexact(gpu, oracle, large_matrices, dtype):
    """2..63 input rows on a large matrix (pair-lane tiles up to 8 rows, one
    and two 16-row tiles, ragged tails) are bitwise the oracle's, hence
    bitwise the one-row results."""
    w, rows = large_matrices[dtype]
    mat = Q.QuantizedMatrix.upload(w, dtype, rows, 2048)
    impl = 1 if oracle.have_avx2() else 0
    for m in (1, 2, 3, 5, 8, 9, 16, 17, 33, 63):
        x = S.normal((m, 2048), np.random.default_rng(2000 + m))
        expected = oracle.matmul(dtype, w, rows, 2048, x, impl=impl, nthreads=8)
        got = mat.forward(torch.from_numpy(x).to(gpu)).cpu().numpy()
        assert_bitexact(got, expected, f"{S.NAMES[dtype]} [{rows}x2048] m={m}")


@pytest.mark.parametrize("rows,cols", [(100001, 512), (70001, 2048)])
def test_q6k_many_pair_lane_tiles_bitexact(gpu, oracle, rows, cols):
    """Q6_K matrices of more 64-row pair-lane tiles than the GPU holds
    workgroups at once (1563 and 1094 tiles) at 3 and 8 rows, with 2 and 8
    blocks per row (block shifts 0 and 2) and a ragged last tile.  Bitwise
    the oracle's."""
    rng = np.random.default_rng(rows + cols)
    w = S.random_matrix(Q6, rows, cols, rng)
    mat = Q.QuantizedMatrix.upload(w, Q6, rows, cols)
    impl = 1 if oracle.have_avx2() else 0
    for m in (3, 8):
        x = S.normal((m, cols), np.random.default_rng(2200 + m))
        expected = oracle.matmul(Q6, w, rows, cols, x, impl=impl, nthreads=8)
        got = mat.forward(torch.from_numpy(x).to(gpu)).cpu().numpy()
        assert_bitexact(got, expected, f"Q6_K [{rows}x{cols}] m={m}")


def test_large_wide_matrix_rows_bitexact(gpu, oracle):
    """Width 4096 past 64 MiB (Q4_K [30000 x 4096], 69 MB): one row takes the
    four-row GEMV items over two slices per row, 2..8 rows the pair-lane
    tile over 16 blocks per row, 9+ rows the 16-row tile; all bitwise the
    oracle's."""
    rng = np.random.default_rng(78)
    rows = 30000
    w = S.random_matrix(Q4, rows, 4096, rng)
    mat = Q.QuantizedMatrix.upload(w, Q4, rows, 4096)
    impl = 1 if oracle.have_avx2() else 0
    for m in (1, 2, 5, 8, 9):
        x = S.normal((m, 4096), np.random.default_rng(2100 + m))
        expected = oracle.matmul(Q4, w, rows, 4096, x, impl=impl, nthreads=8)
        got = mat.forward(torch.from_numpy(x).to(gpu)).cpu().numpy()
        assert_bitexact(got, expected, f"Q4_K [{rows}x4096] m={m}")


@pytest.mark.parametrize("m", [1, 2, 8, 16])
def test_joined_attention_projections_match_separate_calls(gpu, m):
    """q/gate [8192 x 2048], k and v [512 x 2048] joined by rows give bitwise
    the three separate products at decode and verify widths (the
    decode-step benchmark's joined form)."""
    mats = [Q.QuantizedMatrix.view(S.random_matrix_device(Q4, r, 2048, gpu, 40 + j), Q4, r, 2048)
            for j, r in enumerate((8192, 512, 512))]
    joined = mats[0].concatenate_rows(mats[1]).concatenate_rows(mats[2])
    x = torch.randn(m, 2048, device=gpu, generator=torch.Generator(device=gpu).manual_seed(m))
    expected = torch.cat([mt.forward(x) for mt in mats], dim=1).cpu().numpy()
    assert_bitexact(joined.forward(x).cpu().numpy(), expected, f"joined qkv m={m}")


def test_host_entry_matches_device_entry(gpu, oracle):
    rng = np.random.default_rng(6)
    w = S.random_matrix(Q4, 128, 1024, rng)
    mat = Q.QuantizedMatrix.upload(w, Q4, 128, 1024)
    x = S.normal((5, 1024), rng)
    assert_bitexact(mat.forward_host(x), oracle.matmul(Q4, w, 128, 1024, x), "host entry")


def test_empty_inputs_give_empty_outputs(gpu):
    """Zero input rows (src/gguf.rs:433-456 with input_rows == 0): an empty
    result of the right shape, and no launch."""
    rng = np.random.default_rng(8)
    mat = Q.QuantizedMatrix.upload(S.random_matrix(Q4, 24, 512, rng), Q4, 24, 512)
    assert mat.forward(torch.zeros(0, 512, device=gpu)).shape == (0, 24)
    assert mat.forward(torch.zeros(3, 0, 512, device=gpu)).shape == (3, 0, 24)
    assert mat.forward_rows(torch.zeros(0, device=gpu), 0).numel() == 0
    x = S.normal((2, 512), rng)
    y = mat.forward(torch.from_numpy(x).to(gpu))  # the library still works after the empty calls
    assert_bitexact(y.cpu().numpy(), mat.forward_host(x), "after empty calls")


def test_call_time_errors(gpu):
    mat = Q.QuantizedMatrix.upload(np.zeros(144, np.uint8), Q4, 1, 256)
    with pytest.raises(Q.QgemmError, match="final dimension 128, expected 256"):
        mat.forward(torch.zeros(1, 128, device=gpu))
    with pytest.raises(Q.QgemmError, match="rank at least two"):
        mat.forward(torch.zeros(256, device=gpu))
    with pytest.raises(Q.QgemmError, match="cannot take 2 leading rows of a 1-row matrix"):
        mat.leading_rows(2)
    other = Q.QuantizedMatrix.upload(np.zeros(34 * 8, np.uint8), Q8, 1, 256)
    with pytest.raises(Q.QgemmError, match="cannot concatenate quantized matrices with dtypes"):
        mat.concatenate_rows(other)


def test_random_shapes_bitexact(gpu, oracle):
    """A seeded sweep of shapes the named tests do not pin -- every format,
    widths from one block to 24, row counts from 1 to about 20000 and input
    rows from 1 to 70, whichever kernel the dispatch picks -- each output
    bitwise the oracle's."""
    rng = np.random.default_rng(4242)
    impl = 1 if oracle.have_avx2() else 0
    fmts = (Q4, S.Q5_K, Q6, Q8)
    for case in range(64):
        dtype = fmts[case % 4]
        nb = int(rng.choice([1, 2, 3, 4, 8, 12, 16, 24]))
        cols = 256 * nb
        rows = int(rng.choice([int(rng.integers(1, 40)), int(rng.integers(40, 3000)), int(rng.integers(3000, 20000))]))
        m = int(rng.choice([1, 2, int(rng.integers(3, 9)), int(rng.integers(9, 64)), int(rng.integers(64, 71))]))
        w = S.random_matrix(dtype, rows, cols, rng)
        x = S.normal((m, cols), rng)
        mat = Q.QuantizedMatrix.upload(w, dtype, rows, cols)
        got = mat.forward(torch.from_numpy(x).to(gpu)).cpu().numpy()
        expected = oracle.matmul(dtype, w, rows, cols, x, impl=impl, nthreads=8)
        assert_bitexact(got, expected, f"case {case}: {S.NAMES[dtype]} [{rows}x{cols}] m={m}")
