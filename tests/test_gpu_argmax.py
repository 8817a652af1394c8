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
