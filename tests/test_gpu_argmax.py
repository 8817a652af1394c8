"""GPU parity of greedy selection (sampling::argmax, src/sampling.rs:
104-110) and of the LM head fused with it, through the C ABI.

The checker restates the reference's rule on the host: among the finite
values (NaN and +-inf dropped by is_finite) the maximum under partial_cmp
(-0 equal to +0), the LAST of equal maxima (Rust's Iterator::max_by), -1
when no value is finite.  It is pinned by the reference's own case
(greedy_is_deterministic: [-1, 3, 2] -> 1).  Bitwise: indices must be equal
and values bit-identical to the logits they index.
"""
import numpy as np
import pytest
import torch

from conftest import assert_bitexact
from inferq_amd import qgemm as Q
from inferq_amd import synth as S

pytestmark = pytest.mark.gpu


def ref_argmax(row: np.ndarray) -> int:
    """sampling::argmax restated: last index of the largest finite value."""
    row = np.asarray(row, np.float32)
    fin = np.flatnonzero(np.isfinite(row))
    if fin.size == 0:
        return -1
    best = row[fin].max()
    return int(fin[row[fin] == best][-1])


def _gpu_argmax(gpu, rows):
    y = torch.from_numpy(np.ascontiguousarray(rows, np.float32)).to(gpu)
    idx, val = Q.argmax(y)
    return idx.cpu().numpy(), val.cpu().numpy()


def test_reference_greedy_case(gpu):
    idx, val = _gpu_argmax(gpu, [[-1.0, 3.0, 2.0]])
    assert idx.tolist() == [1] and val.tolist() == [3.0]


def test_ties_non_finite_and_signed_zero(gpu):
    nan, inf = np.float32("nan"), np.float32("inf")
    rows = [
        [1.0, 5.0, 2.0, 5.0, 5.0, 0.0],          # equal maxima: the last one
        [nan, 2.0, inf, 2.0, -inf, 1.0],        # non-finite skipped
        [-0.0, 0.0, -0.0, -1.0, -2.0, -3.0],    # -0 == +0: last of the zeros
        [nan, nan, inf, -inf, nan, inf],        # nothing finite
        [-5.0, -7.0, -5.0, -9.0, -6.0, -5.5],   # all negative
        [3.0, nan, nan, nan, nan, nan],         # the only finite value first
    ]
    idx, val = _gpu_argmax(gpu, rows)
    assert idx.tolist() == [ref_argmax(r) for r in rows] == [4, 3, 2, -1, 2, 0]
    for r, i in enumerate(idx):
        if i >= 0:
            assert np.float32(val[r]).view(np.uint32) == np.float32(rows[r][i]).view(np.uint32)
        else:
            assert np.isnan(val[r])


@pytest.mark.parametrize("n", [1, 255, 4096, 4097, 100003, 248320])
def test_long_rows_match_the_rule(gpu, n):
    """Chunk boundaries (4096 values per chunk), ragged tails, and maxima
    placed at the first and last index and duplicated across chunks."""
    rng = np.random.default_rng(n)
    rows = rng.standard_normal((4, n), dtype=np.float32)
    rows[1, -1] = 100.0
    rows[2, 0] = 100.0
    if n > 4100:
        rows[3, [10, 4096, n - 2]] = 50.0  # equal maxima in different chunks
        rows[3, 5000 % n] = np.nan
    idx, val = _gpu_argmax(gpu, rows)
    assert idx.tolist() == [ref_argmax(r) for r in rows]


@pytest.fixture(scope="module")
def lm_head(gpu):
    t = S.random_matrix_device(S.Q6_K, 248320, 2048, gpu, 6000)
    return Q.QuantizedMatrix.view(t, S.Q6_K, 248320, 2048)


@pytest.mark.parametrize("m", [1, 8])
def test_lm_head_argmax_equals_argmax_of_logits(gpu, lm_head, m):
    """The fused entry selects from exactly iq_matmul's logits."""
    x = torch.randn(m, 2048, device=gpu, generator=torch.Generator(device=gpu).manual_seed(m))
    logits = lm_head.forward(x).cpu().numpy()
    idx, val = lm_head.forward_argmax(x)
    idx, val = idx.cpu().numpy(), val.cpu().numpy()
    assert idx.tolist() == [ref_argmax(r) for r in logits]
    assert_bitexact(val, logits[np.arange(m), idx], f"LM head argmax values m={m}")


def test_vocab_prefix_draft_head(gpu, lm_head):
    """leading_rows(vocab) then greedy selection: the MTP draft head
    (src/qwen/quantized_mtp.rs:142-143) selects within the prefix."""
    draft = lm_head.leading_rows(32768)
    x = torch.randn(4, 2048, device=gpu, generator=torch.Generator(device=gpu).manual_seed(77))
    full = lm_head.forward(x).cpu().numpy()
    idx, _ = draft.forward_argmax(x)
    assert idx.cpu().numpy().tolist() == [ref_argmax(r[:32768]) for r in full]


def _check_selection(mat, x, what):
    """forward_argmax against the rule over forward()'s logits: indices
    equal, values bit-identical to the logits they index."""
    logits = mat.forward(x).cpu().numpy()
    idx, val = mat.forward_argmax(x)
    idx, val = idx.cpu().numpy(), val.cpu().numpy()
    assert idx.tolist() == [ref_argmax(r) for r in logits], what
    assert_bitexact(val, logits[np.arange(len(idx)), idx], what)


@pytest.mark.parametrize("rows,cols", [(1, 2048), (3, 2048), (5, 1024), (4099, 2048), (40961, 4096), (65537, 3072)])
def test_one_row_fused_selection_ragged_shapes(gpu, rows, cols):
    """At one input row the selection is fused into the four-row-item
    product (every Q8_0 matrix takes it): each wave reduces its own rows,
    one launch joins the waves.  Row counts that leave partial items,
    partial workgroups and waves without rows."""
    t = S.random_matrix_device(S.Q8_0, rows, cols, gpu, 7000 + rows)
    mat = Q.QuantizedMatrix.view(t, S.Q8_0, rows, cols)
    x = torch.randn(1, cols, device=gpu, generator=torch.Generator(device=gpu).manual_seed(rows))
    _check_selection(mat, x, f"fused selection [{rows} x {cols}] Q8_0")


@pytest.mark.parametrize("dtype,period,reps", [(S.Q8_0, 7, 10001), (S.Q6_K, 61, 700), (S.Q4_K, 13, 5000)])
def test_one_row_fused_selection_ties_across_waves(gpu, dtype, period, reps):
    """Rows repeating with a short period give bit-equal logits at indices
    spread over every wave and workgroup: the LAST of the equal maxima must
    win (Rust's max_by).  The Q6_K and Q4_K matrices are past the split
    kernel's 64 MiB, as the LM head is, so they take the fused product
    too."""
    base = S.random_matrix_device(dtype, period, 2048, gpu, 7100 + period)
    t = base.repeat(reps)
    rows = period * reps
    mat = Q.QuantizedMatrix.view(t, dtype, rows, 2048)
    x = torch.randn(1, 2048, device=gpu, generator=torch.Generator(device=gpu).manual_seed(period))
    logits = mat.forward(x).cpu().numpy()[0]
    assert np.array_equal(logits[:period].view(np.uint32), logits[-period:].view(np.uint32))
    want = ref_argmax(logits)
    assert want >= rows - period  # the last period holds the last maximum
    _check_selection(mat, x, f"ties, period {period}")


def test_one_row_fused_selection_in_graph_replays(gpu, lm_head):
    """The fused selection captured after a reserve, replayed with eager
    work between the replays: every replay equals the eager call."""
    g = torch.Generator(device=gpu).manual_seed(99)
    xs = [torch.randn(1, 2048, device=gpu, generator=g) for _ in range(3)]
    x = torch.empty(1, 2048, device=gpu)
    idx = torch.empty(1, dtype=torch.int32, device=gpu)
    val = torch.empty(1, dtype=torch.float32, device=gpu)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        lm_head.reserve(1)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            Q.check(Q.lib().iq_matmul_argmax(lm_head.handle, x.data_ptr(), 1, idx.data_ptr(), val.data_ptr(),
                                             Q._stream()))
    for xi in xs:
        x.copy_(xi)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want_i, want_v = lm_head.forward_argmax(xi)
        torch.cuda.synchronize()
        assert idx.cpu().tolist() == want_i.cpu().tolist()
        assert_bitexact(val.cpu().numpy(), want_v.cpu().numpy(), "graph replay of the fused selection")


@pytest.mark.parametrize("m", [2, 3, 5, 8])
def test_verify_width_fused_selection(gpu, lm_head, m):
    """At 2..8 rows on a large matrix the selection is fused into the
    pair-lane MFMA tile (each workgroup reduces its 64 columns per input
    row): the same indices and values as the rule over the logits."""
    x = torch.randn(m, 2048, device=gpu, generator=torch.Generator(device=gpu).manual_seed(300 + m))
    _check_selection(lm_head, x, f"LM head fused selection m={m}")


@pytest.mark.parametrize("dtype,period,reps,m", [(S.Q6_K, 61, 700, 4), (S.Q4_K, 13, 5000, 8), (S.Q6_K, 64, 667, 3)])
def test_verify_width_fused_selection_ties(gpu, dtype, period, reps, m):
    """Periodic rows (bit-equal logits in every workgroup) on the pair-lane
    tile, and a row count that leaves a partial last workgroup (61 x 700 =
    42700 = 667 x 64 + 12): the last of the equal maxima wins in every
    input row."""
    base = S.random_matrix_device(dtype, period, 2048, gpu, 7200 + period)
    t = base.repeat(reps)
    rows = period * reps
    mat = Q.QuantizedMatrix.view(t, dtype, rows, 2048)
    x = torch.randn(m, 2048, device=gpu, generator=torch.Generator(device=gpu).manual_seed(period + m))
    logits = mat.forward(x).cpu().numpy()
    assert all(ref_argmax(r) >= rows - period for r in logits)
    _check_selection(mat, x, f"fused selection ties, period {period}, m={m}")


@pytest.mark.parametrize("dtype,reps", [(S.Q8_0, 4099), (S.Q6_K, 40960), (S.Q4_K, 65536)])
@pytest.mark.parametrize("m", [1, 4, 8])
def test_fused_selection_over_a_matrix_of_equal_logits(gpu, dtype, reps, m):
    """Every quant and scale byte zero (d finite): every logit of a row is
    zero (+0 or -0, which rank equal), so the last index of the matrix must
    win in every input row, across every wave and workgroup of the fused
    product and of the joining launch.  The K-quant matrices are past
    64 MiB, as the LM head is."""
    bb = S.BLOCK_BYTES[dtype]
    nb = 2048 // S.BLOCK_ELEMS[dtype]
    base = S.random_matrix_device(dtype, 1, 2048, gpu, 7300 + dtype).reshape(nb, bb)
    lo, hi = {S.Q4_K: (0, 4), S.Q6_K: (208, 210), S.Q8_0: (0, 2)}[dtype]
    zero = torch.zeros_like(base)
    zero[:, lo:hi] = base[:, lo:hi]
    rows = reps
    t = zero.reshape(-1).repeat(rows)
    mat = Q.QuantizedMatrix.view(t, dtype, rows, 2048)
    x = torch.randn(m, 2048, device=gpu, generator=torch.Generator(device=gpu).manual_seed(m))
    logits = mat.forward(x).cpu().numpy()
    assert not np.any(logits)
    assert [ref_argmax(r) for r in logits] == [rows - 1] * m
    _check_selection(mat, x, f"equal logits {S.NAMES[dtype]} [{rows} x 2048] m={m}")
