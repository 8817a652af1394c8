"""GPU parity on blocks and activations at the edges of their integer ranges.

The int8 MFMA tiles split each block's scales into several int8 weight
streams (Q4_K: 8 (sc >> 3) q + (sc & 7) q; Q5_K: a third stream for the
fifth bit; Q6_K: signed scales split by radix), and every such stream must
stay inside int8 for every legal byte.  Random blocks rarely reach the
corners, so these matrices set every payload byte (quants, high bits,
scales; the f16 d / dmin fields stay finite) to 0xFF, 0x00, 0x80 or a
random mix of corner bytes, and multiply them with activation rows that
quantise to the Q8K / Q8_0 extremes: constant rows (every value -128), a
zero row (scale 0), alternating +-1 and mixed magnitudes.  Every row count
the dispatch splits at (split-K GEMV, row-tiled GEMV, pair-lane and exact
MFMA tiles) is compared bit for bit with the oracle (src/qgemm.rs:175-397
restated), and the explicit lane and MFMA paths with the dispatch.
"""
import numpy as np
import pytest
import torch

from conftest import assert_bitexact, assert_close_normwise
from inferq_amd import _lib
from inferq_amd import qgemm as Q
from inferq_amd import synth as S

pytestmark = pytest.mark.gpu

# byte ranges of the f16 scale fields, which stay as drawn (finite)
F16_FIELDS = {S.Q4_K: (0, 4), S.Q5_K: (0, 4), S.Q6_K: (208, 210), S.Q8_0: (0, 2)}
CORNERS = np.array([0x00, 0xFF, 0x80, 0x7F, 0x0F, 0xF0, 0x01, 0xFE], np.uint8)


def corner_matrix(dtype, rows, cols, mode, seed):
    rng = np.random.default_rng(seed)
    return corner_bytes(dtype, S.random_matrix(dtype, rows, cols, rng), mode, rng)


def corner_bytes(dtype, flat, mode, rng):
    """Random blocks with every payload byte replaced by a corner byte."""
    raw = flat.reshape(-1, S.BLOCK_BYTES[dtype]).copy()
    lo, hi = F16_FIELDS[dtype]
    keep = raw[:, lo:hi].copy()
    if mode == "mix":
        raw[:] = CORNERS[rng.integers(0, len(CORNERS), size=raw.shape)]
    else:
        raw[:] = {"ff": 0xFF, "00": 0x00, "80": 0x80}[mode]
    raw[:, lo:hi] = keep
    return raw.reshape(-1)


def corner_activations(m, cols, seed):
    """m rows cycling through the Q8K / Q8_0 corner cases."""
    rng = np.random.default_rng(seed)
    x = S.normal((m, cols), rng)
    for r in range(m):
        kind = r % 6
        if kind == 1:
            x[r] = 1.0  # every value quantises to -128
        elif kind == 2:
            x[r] = -3.5
        elif kind == 3:
            x[r] = 0.0  # a zero row: scale 0
        elif kind == 4:
            x[r] = np.where(np.arange(cols) % 2 == 0, 1.0, -1.0)
        elif kind == 5:
            x[r] *= np.float32(10.0) ** rng.integers(-3, 4, size=cols).astype(np.float32)
    return x


def _impl(oracle):
    return 1 if oracle.have_avx2() else 0


def _check(oracle, gpu, dtype, rows, cols, mode, ms):
    w = corner_matrix(dtype, rows, cols, mode, rows + cols + len(mode))
    mat = Q.QuantizedMatrix.upload(w, dtype, rows, cols)
    for m in ms:
        x = corner_activations(m, cols, m)
        expected = oracle.matmul(dtype, w, rows, cols, x, impl=_impl(oracle), nthreads=8)
        assert np.isfinite(expected).all()
        xt = torch.from_numpy(x).to(gpu)
        got = mat.forward(xt).cpu().numpy()
        what = f"{mat.dtype()} [{rows} x {cols}] bytes {mode} m={m}"
        assert_bitexact(got, expected, what)
        assert_bitexact(mat.forward_via(xt, _lib.PATH_LANES).cpu().numpy(), expected, what + " lanes")
        if dtype != S.Q8_0 and m >= (9 if dtype == S.Q5_K else 2):  # Q5_K tiles from 9 rows
            assert_bitexact(mat.forward_via(xt, _lib.PATH_LANE_MFMA).cpu().numpy(), expected, what + " MFMA")
        if dtype == S.Q4_K and m >= 64:
            tiles = mat.forward_via(xt, _lib.PATH_PREFILL_TILES).cpu().numpy()
            for r in range(m):
                assert_close_normwise(tiles[r], expected[r], 1e-4, what + f" prefill tiles row {r}")


FORMATS = [S.Q4_K, S.Q5_K, S.Q6_K, S.Q8_0]
FMT_IDS = ["q4k", "q5k", "q6k", "q80"]


@pytest.mark.parametrize("mode", ["ff", "00", "80", "mix"])
@pytest.mark.parametrize("dtype", FORMATS, ids=FMT_IDS)
def test_corner_blocks_small_matrix(gpu, oracle, dtype, mode):
    """[320 x 2048]: the split-K GEMV (1..8 rows), the row-tiled GEMV (9..63)
    and the exact MFMA tiles (64 and up)."""
    _check(oracle, gpu, dtype, 320, 2048, mode, (1, 2, 3, 8, 9, 17, 64, 100))


@pytest.mark.parametrize("dtype", FORMATS, ids=FMT_IDS)
def test_corner_blocks_wide_rows(gpu, oracle, dtype):
    """Width 4096 and a ragged row count."""
    _check(oracle, gpu, dtype, 197, 4096, "mix", (1, 4, 8, 33, 64))


@pytest.mark.parametrize("dtype", [S.Q4_K, S.Q6_K], ids=["q4k", "q6k"])
def test_corner_blocks_large_matrix(gpu, oracle, dtype):
    """[8192 x 2048] (past 8 MiB): the split-K pair-lane MFMA tile at 3..8
    rows and the 32-row exact tiles at 256."""
    _check(oracle, gpu, dtype, 8192, 2048, "mix", (1, 3, 8, 256))


MOE_LAYERS = {}


def corner_moe_layer(formats):
    """Config-2 shaped routed experts (hidden 2048, intermediate 512, 256
    experts) whose every payload byte is a corner byte."""
    if formats not in MOE_LAYERS:
        rng = np.random.default_rng(31337 + sum(formats))
        layer = S.random_moe_layer(2048, 512, 256, formats[0], formats[1], rng, shared=False)
        for name, dtype in (("gate", formats[0]), ("up", formats[0]), ("down", formats[1])):
            layer[name] = corner_bytes(dtype, layer[name], "mix", rng)
        MOE_LAYERS[formats] = layer
    return MOE_LAYERS[formats]


@pytest.mark.parametrize("formats", [(S.Q4_K, S.Q6_K), (S.Q5_K, S.Q5_K)], ids=["q4q6", "q5q5"])
@pytest.mark.parametrize("m", [1, 8, 16, 33, 256])
def test_corner_experts(gpu, oracle, formats, m):
    """MoE layers of corner-byte experts on the token-major kernels (1, 8 and
    16 tokens) and the grouped MFMA path (33 and 256): routes equal the
    oracle's (src/qwen/quantized_moe.rs:253-406 restated), every output row
    within 1e-4 of it (the bar for MoE layers: their SwiGLU exp is
    correctly rounded here, while the oracle calls glibc's expf), one token
    bit for bit, and the first tokens of a wide call
    (one of each activation kind) bitwise equal to one-token calls."""
    from inferq_amd import moe as MOE

    layer = corner_moe_layer(formats)
    t = {k: torch.from_numpy(v).to(gpu) for k, v in layer.items() if isinstance(v, np.ndarray)}
    moe = MOE.QuantizedMoeLayer(2048, 512, 256, 8, formats[0], formats[1], t["gate"], t["up"], t["down"])
    rng = np.random.default_rng(900 + m)
    x = corner_activations(m, 2048, 900 + m)
    logits = S.normal((m, 256), rng)
    d = dict(layer, top_k=8, normalize=True)
    ref, ref_e, _ = oracle.moe_forward(d, x, logits, mode=1, impl=_impl(oracle), nthreads=8)
    assert np.isfinite(ref).all()
    out = moe.forward(torch.from_numpy(x).to(gpu), torch.from_numpy(logits).to(gpu))
    assert [r.experts for r in out.routes] == ref_e.tolist(), f"routes m={m}"
    got = out.hidden.cpu().numpy()
    for r in range(m):
        assert_close_normwise(got[r], ref[r], 1e-4, f"corner experts {formats} m={m} row {r}")
    if m == 1:
        assert_bitexact(got, ref, f"corner experts {formats} one token")
    for r in range(min(m, 6) if m > 1 else 0):
        one = moe.forward(torch.from_numpy(x[r:r + 1]).to(gpu), torch.from_numpy(logits[r:r + 1]).to(gpu))
        assert_bitexact(got[r], one.hidden.cpu().numpy()[0], f"corner experts {formats} m={m} token {r} vs one-token call")


@pytest.mark.parametrize("mode", ["ff", "80", "mix"])
@pytest.mark.parametrize("dtype", [S.Q4_K, S.Q6_K, S.Q8_0], ids=["q4k", "q6k", "q80"])
def test_corner_row_entries(gpu, oracle, dtype, mode):
    """The per-row entries (q4k_q8k_row / q6k_q8k_row / q80_q80_row,
    src/qgemm.rs:447-468) on a corner-byte row and corner activation rows,
    bitwise to the oracle's restatement."""
    cols = 2048
    wrow = corner_matrix(dtype, 1, cols, mode, 41 + dtype)
    for rows in (1, 6, 12):
        x = corner_activations(rows, cols, rows)
        q = np.stack([oracle.quantize_q80(r) if dtype == S.Q8_0 else oracle.quantize_q8k(r) for r in x])
        block_major = np.ascontiguousarray(q.T)
        got = Q.row_kernel(dtype, wrow, block_major, rows)
        expected = oracle.row_kernel(dtype, wrow.view(oracle.BLOCK[dtype]), block_major, rows, impl="lanes")
        assert_bitexact(got, expected, f"{S.NAMES[dtype]} row entry bytes {mode} rows={rows}")


@pytest.mark.parametrize("dtype", FORMATS, ids=FMT_IDS)
def test_corner_block_integers(gpu, oracle, dtype):
    """The per-block lane integers (isum, and msum for Q4_K / Q5_K) of
    corner-byte blocks against corner activations, exact."""
    rows, cols = 16, 512
    w = corner_matrix(dtype, rows, cols, "mix", 77 + dtype)
    x = corner_activations(6, cols, 6)
    mat = Q.QuantizedMatrix.upload(w, dtype, rows, cols)
    y, isum, msum = mat.block_sums(torch.from_numpy(x).to(gpu))
    isum = isum.cpu().numpy()
    msum = msum.cpu().numpy() if msum is not None else None
    nb = cols // S.BLOCK_ELEMS[dtype]
    wb = w.view(oracle.BLOCK[dtype]).reshape(rows, nb)
    for r in range(x.shape[0]):
        q = oracle.quantize_q80(x[r]) if dtype == S.Q8_0 else oracle.quantize_q8k(x[r])
        for n in range(rows):
            for b in range(nb):
                ei, em = oracle.block_lanes(dtype, wb[n, b], q[b])
                assert np.array_equal(isum[r, n, b], ei), (r, n, b)
                if em is not None:
                    assert np.array_equal(msum[r, n, b], em), (r, n, b)
    assert_bitexact(y.cpu().numpy(), oracle.matmul(dtype, w, rows, cols, x), "corner block_sums output")
