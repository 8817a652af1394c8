"""The parity oracle (oracle/) pinned by checks that do not restate its own
formulas: the reference's AVX2 intrinsic sequence against the scalar lane
emulation, per-block lane integers against the textbook dequantisation
integers, closed forms in f64, exact-integer special cases, numpy's IEEE
half conversions, the reference's own test cases, and invariances the
reference asserts (row count, tiling, spread, concatenation, grouped vs
token-major MoE).  CPU only.
"""
import os

import numpy as np
import pytest

from conftest import assert_bitexact, assert_close_normwise
from inferq_amd import synth as S

Q4, Q6, Q8 = S.Q4_K, S.Q6_K, S.Q8_0
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "qgemm_golden.npz")


def _avx2(oracle):
    if not oracle.have_avx2():
        pytest.skip("host has no AVX2/FMA: the intrinsic form cannot run")


# ---------------------------------------------------------------- formats
def test_f16_to_f32_matches_numpy_for_every_half(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.isnan(got[~np.isfinite(ref) & np.isnan(ref)]).all()


def test_f32_to_f16_rounds_like_numpy(oracle):
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 5, 20000),
        np.float32([0.0, -0.0, 65504, 65519.99, 65520, 1e-8, 5.96e-8, 2.98e-8, 2.9802326e-08, 6.1e-5]),
        # exact halfway cases between adjacent halves (ties to even)
        (np.arange(1024, 2048, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10),
    ])
    got = np.array([oracle.f32_to_f16(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_block_sizes_match_the_reference_asserts(oracle):
    # src/qgemm.rs:36-43 asserts the candle block sizes
    assert [oracle.BLOCK[d].itemsize for d in (Q4, Q6, Q8)] == [144, 210, 34]
    assert oracle.Q8K_BLOCK.itemsize == 292


# ------------------------------------------------------- from_float (Q8K)
def test_q8k_zero_block(oracle):
    b = oracle.quantize_q8k(np.zeros(256, np.float32))[0]
    assert b["d"] == 0 and not b["qs"].any() and not b["bsums"].any()


def test_q8k_single_value_maps_to_minus_128(oracle):
    x = np.zeros(256, np.float32)
    x[17] = 3.0
    b = oracle.quantize_q8k(x)[0]
    assert b["qs"][17] == -128 and np.count_nonzero(b["qs"]) == 1
    assert b["d"] == np.float32(1.0) / (np.float32(-128.0) / np.float32(3.0))
    assert b["bsums"][1] == -128


def test_q8k_first_index_of_the_maximum_sets_the_sign(oracle):
    # |x| ties everywhere: the first element (+0.75) is `max`, so positive
    # values map to -128 and negative ones to +128 clamped to 127
    x = np.tile(np.float32([0.75, -0.75]), 128)
    q = oracle.quantize_q8k(x)[0]["qs"]
    assert (q[0::2] == -128).all() and (q[1::2] == 127).all()
    y = -x
    q = oracle.quantize_q8k(y)[0]["qs"]
    assert (q[0::2] == -128).all() and (q[1::2] == 127).all()


def test_q8k_rounds_half_away_from_zero(oracle):
    # max = -8 gives iscale = 16, so x = (k + 0.5) / 16 lands on a tie
    x = np.zeros(256, np.float32)
    x[0] = -8.0
    x[1:6] = np.float32([0.5, 1.5, -0.5, -1.5, 2.5]) / np.float32(16)
    q = oracle.quantize_q8k(x)[0]["qs"]
    assert list(q[1:6]) == [1, 2, -1, -2, 3]


def test_q8k_bsums_are_sums_of_16(oracle):
    rng = np.random.default_rng(1)
    b = oracle.quantize_q8k(S.normal(1024, rng))
    for blk in b:
        assert np.array_equal(blk["bsums"], blk["qs"].astype(np.int32).reshape(16, 16).sum(1))


def test_q80_quantisation_cases(oracle):
    x = np.zeros(64, np.float32)
    x[32:] = np.linspace(-2, 2, 32, dtype=np.float32)
    b = oracle.quantize_q80(x)
    assert b[0]["d"] == 0 and not b[0]["qs"].any()
    d = np.float32(2.0) / np.float32(127.0)
    assert b[1]["d"] == np.float32(d).astype(np.float16).view(np.uint16)
    # values quantise with the f32 d (not the stored f16 d), half away from zero
    idv = np.float32(1.0) / d
    expected = np.sign(x[32:] * idv) * np.floor(np.abs(x[32:] * idv) + np.float32(0.5))
    assert np.array_equal(b[1]["qs"], expected.astype(np.int8))


# ------------------------------------------------- per-block integers
@pytest.mark.parametrize("dtype", [Q4, S.Q5_K, Q6, Q8])
def test_lane_integers_sum_to_textbook_integers(oracle, dtype):
    rng = np.random.default_rng(2 + dtype)
    nb = 24
    w = S.random_blocks(dtype, nb, rng).view(oracle.BLOCK[dtype])
    k = nb * S.BLOCK_ELEMS[dtype]
    x = S.normal(k, rng)
    q = oracle.quantize_q80(x) if dtype == Q8 else oracle.quantize_q8k(x)
    for b in range(nb):
        isum, msum = oracle.block_lanes(dtype, w[b], q[b])
        ti, tm = oracle.block_textbook(dtype, w[b], q[b])
        assert int(isum.astype(np.int64).sum()) == ti
        if dtype in (Q4, S.Q5_K):
            assert int(msum.astype(np.int64).sum()) == tm


# ---------------------------------------------- the row kernels (lanes)
@pytest.mark.parametrize("dtype", [Q4, Q6, Q8])
def test_lane_emulation_equals_the_avx2_sequence(oracle, dtype):
    """Reference test fused_kernel_matches_candle_across_row_counts
    (src/gguf.rs:1630-1677): [96 x 512] at the row counts it uses."""
    _avx2(oracle)
    rng = np.random.default_rng(10 + dtype)
    w = S.random_matrix(dtype, 96, 512, rng)
    for m in (1, 2, 3, 4, 7, 8, 9, 15, 16):
        x = S.normal((m, 512), rng)
        assert_bitexact(oracle.matmul(dtype, w, 96, 512, x, impl=0), oracle.matmul(dtype, w, 96, 512, x, impl=1),
                        f"{S.NAMES[dtype]} m={m}")


@pytest.mark.parametrize("dtype", [Q4, S.Q5_K, Q6, Q8])
def test_product_matches_f64_dequantised_dot(oracle, dtype):
    """Closed form: the f32 result equals dequant(W) . dequant(quant(x)) up
    to f32 accumulation (~1e-6 normwise); a dropped term, a wrong sign or a
    transposed nibble would be O(1)."""
    rng = np.random.default_rng(20 + dtype)
    n, k = 48, 1024
    w = S.random_matrix(dtype, n, k, rng)
    x = S.normal((5, k), rng)
    W = oracle.dequantize(dtype, w, n, k).astype(np.float64)
    if dtype == Q8:
        q = oracle.quantize_q80(x.reshape(-1))
        scale = np.array([oracle.f16_to_f32(int(v)) for v in q["d"]], np.float64)
        xq = (q["qs"].astype(np.float64) * scale[:, None]).reshape(5, k)
    else:
        q = oracle.quantize_q8k(x.reshape(-1))
        xq = (q["qs"].astype(np.float64) * q["d"].astype(np.float64)[:, None]).reshape(5, k)
    assert_close_normwise(oracle.matmul(dtype, w, n, k, x), xq @ W.T, 2e-6, S.NAMES[dtype])


def test_product_within_the_activation_quantisation_bound(oracle):
    """src/gguf.rs:1741-1775 checks the quantised product against the f32
    product of the dequantised matrix (absolute 2e-2 on its small weights).
    Stated for any weights: |y - W x| <= sum_j |W_ij| e_j, with e_j the
    largest rounding error of x_j -- amax/128 per 256-block for Q8K (the
    clamp of -amax to 127 is the worst case), amax/127 * (1/2 + 2^-11 * 127)
    per 32-block for Q8_0 (f16-rounded scale) -- plus f32 accumulation."""
    rng = np.random.default_rng(30)
    x = ((np.arange(1024, dtype=np.float32) % 11) - 5) / 8
    x = np.stack([x, S.normal(1024, rng)])
    for dtype in (Q4, Q6, Q8):
        w = S.random_matrix(dtype, 8, 1024, rng)
        W = oracle.dequantize(dtype, w, 8, 1024).astype(np.float64)
        y = oracle.matmul(dtype, w, 8, 1024, x).astype(np.float64)
        blk = 32 if dtype == Q8 else 256
        amax = np.abs(x.reshape(2, -1, blk)).max(2, keepdims=True).astype(np.float64)
        e = np.broadcast_to(amax / 127 * (0.5 + 127 * 2.0 ** -11) if dtype == Q8 else amax / 128,
                            (2, 1024 // blk, blk)).reshape(2, 1024)
        bound = e @ np.abs(W).T + 1e-5 * (np.abs(x) @ np.abs(W).T)
        err = np.abs(y - x.astype(np.float64) @ W.T)
        assert (err <= bound).all(), S.NAMES[dtype]
        assert (err > 0).any()  # the bound is not vacuous: quantisation did round


def _integer_row(k, rng):
    """An activation row of integers in [-127, 127] with one -128 in every
    256-block, so that Q8K quantisation is the identity (d = 1)."""
    x = rng.integers(-127, 128, k).astype(np.float32)
    x.reshape(-1, 256)[np.arange(k // 256), rng.integers(0, 256, k // 256)] = -128
    return x


def test_q4k_with_unit_scales_is_a_plain_integer_dot(oracle):
    rng = np.random.default_rng(40)
    nb, n = 4, 6
    blocks = np.zeros(n * nb, oracle.Q4K_BLOCK)
    blocks["d"] = 0x3C00  # 1.0
    blocks["dmin"] = 0
    # six-bit scale 1 and min 0 for all 8 sub-blocks
    blocks["scales"][:, 0:4] = 1
    blocks["scales"][:, 4:8] = 0
    blocks["scales"][:, 8:12] = 0x01
    blocks["qs"] = rng.integers(0, 256, (n * nb, 128))
    w = blocks.view(np.uint8)
    x = _integer_row(256 * nb, rng)
    W = oracle.dequantize(Q4, w, n, 256 * nb)
    y = oracle.matmul(Q4, w, n, 256 * nb, x[None, :])[0]
    assert np.array_equal(y, (W.astype(np.int64) @ x.astype(np.int64)).astype(np.float32))


def test_q8_0_with_unit_scale_is_a_plain_integer_dot(oracle):
    rng = np.random.default_rng(41)
    n, k = 5, 512
    blocks = np.zeros(n * k // 32, oracle.Q80_BLOCK)
    blocks["d"] = 0x3C00
    blocks["qs"] = rng.integers(-128, 128, (n * k // 32, 32))
    x = rng.integers(-127, 128, k).astype(np.float32)
    x.reshape(-1, 32)[:, 0] = 127  # every block's amax is 127, so d = 1
    y = oracle.matmul(Q8, blocks.view(np.uint8), n, k, x[None, :])[0]
    ref = blocks["qs"].astype(np.int64).reshape(n, k) @ x.astype(np.int64)
    assert np.array_equal(y, ref.astype(np.float32))


def test_q6k_with_unit_scales_is_a_plain_integer_dot(oracle):
    rng = np.random.default_rng(42)
    n, nb = 4, 2
    blocks = S.random_blocks(Q6, n * nb, rng).view(oracle.Q6K_BLOCK).copy()
    blocks["d"] = 0x3C00
    blocks["scales"] = 1
    w = blocks.view(np.uint8)
    x = _integer_row(256 * nb, rng)
    W = oracle.dequantize(Q6, w, n, 256 * nb).astype(np.int64)
    y = oracle.matmul(Q6, w, n, 256 * nb, x[None, :])[0]
    assert np.array_equal(y, (W @ x.astype(np.int64)).astype(np.float32))


def test_zero_input_gives_zero(oracle):
    rng = np.random.default_rng(43)
    for dtype in (Q4, Q6, Q8):
        w = S.random_matrix(dtype, 8, 256, rng)
        assert not oracle.matmul(dtype, w, 8, 256, np.zeros((1, 256), np.float32)).any()


def test_single_nonzero_input_gives_scaled_column(oracle):
    rng = np.random.default_rng(44)
    for dtype in (Q4, Q6):
        w = S.random_matrix(dtype, 16, 512, rng)
        x = np.zeros((1, 512), np.float32)
        x[0, 300] = 1.75
        W = oracle.dequantize(dtype, w, 16, 512).astype(np.float64)
        assert_close_normwise(oracle.matmul(dtype, w, 16, 512, x)[0], 1.75 * W[:, 300], 1e-6, S.NAMES[dtype])


# ----------------------------------------------------------- invariances
@pytest.mark.parametrize("dtype", [Q4, Q6, Q8])
def test_row_count_tiling_and_spread_do_not_change_results(oracle, dtype):
    """src/gguf.rs:1703-1727 and tests/speculative_policy.rs:373-450: each
    row equals its one-row product, bitwise, under any tiling or spread."""
    rng = np.random.default_rng(50 + dtype)
    w = S.random_matrix(dtype, 96, 512, rng)
    x = S.normal((33, 512), rng)
    single = np.concatenate([oracle.matmul(dtype, w, 96, 512, x[i:i + 1]) for i in range(33)])
    for m in (2, 8, 15, 16, 17, 33):
        assert_bitexact(oracle.matmul(dtype, w, 96, 512, x[:m], nthreads=4), single[:m], f"m={m}")
        assert_bitexact(oracle.matmul(dtype, w, 96, 512, x[:m], tiled=True), single[:m], f"tiled m={m}")


def test_concatenated_rows_equal_separate_products(oracle):
    rng = np.random.default_rng(60)
    for dtype in (Q4, Q6, Q8):
        a = S.random_matrix(dtype, 2, 256, rng)
        b = S.random_matrix(dtype, 3, 256, rng)
        x = np.full((1, 256), 0.25, np.float32)
        both = oracle.matmul(dtype, np.concatenate([a, b]), 5, 256, x)
        assert_bitexact(both, np.concatenate([oracle.matmul(dtype, a, 2, 256, x),
                                              oracle.matmul(dtype, b, 3, 256, x)], axis=1))


# ---------------------------------------------------------------- routing
def test_router_selects_and_normalizes_top_k(oracle):
    """src/qwen/moe.rs:232-238."""
    e, w = oracle.top_k_routes(np.float32([[1, 4, 2, 3]]), 2, True)
    assert e[0].tolist() == [1, 3]
    assert abs(float(w[0].sum()) - 1.0) < 1e-6


def test_routes_follow_the_softmax(oracle):
    rng = np.random.default_rng(70)
    logits = S.normal((16, 256), rng)
    e, w = oracle.top_k_routes(logits, 8, True)
    p = np.exp(logits.astype(np.float64) - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    for r in range(16):
        assert e[r].tolist() == np.argsort(-logits[r], kind="stable")[:8].tolist()
        top = p[r, e[r]]
        assert_close_normwise(w[r], top / top.sum(), 1e-6)
    e2, w2 = oracle.top_k_routes(logits, 8, False)
    assert_close_normwise(w2, np.take_along_axis(p, e2, 1), 1e-6)


def test_equal_logits_rank_by_index(oracle):
    e, _ = oracle.top_k_routes(np.float32([[0.5, 2.0, 0.5, 2.0, 0.5]]), 4, True)
    assert e[0].tolist() == [1, 3, 0, 2]


# -------------------------------------------------------------------- MoE
def _layer(rng, n_experts=4, shared=True, top_k=2):
    layer = S.random_moe_layer(256, 256, n_experts, Q4, Q6, rng, shared=shared)
    layer.update(top_k=top_k, normalize=True)
    return layer


def test_grouped_moe_equals_token_major_bitwise(oracle):
    """src/qwen/quantized_moe.rs:570-591."""
    rng = np.random.default_rng(80)
    layer = _layer(rng, 6)
    x = S.normal((5, 256), rng)
    logits = S.normal((5, 6), rng)
    a, ea, wa = oracle.moe_forward(layer, x, logits, mode=0)
    b, eb, wb = oracle.moe_forward(layer, x, logits, mode=1, nthreads=3)
    assert_bitexact(a, b, "grouped vs token-major")
    assert np.array_equal(ea, eb) and np.array_equal(wa, wb)


def test_moe_reference_routing_case(oracle):
    """src/qwen/quantized_moe.rs:490-592: router row 1 = 0.01 everywhere and
    an all-ones input route to expert 1 at top-1; outputs are finite."""
    rng = np.random.default_rng(81)
    layer = _layer(rng, 2, top_k=1)
    router = np.stack([np.zeros(256, np.float32), np.full(256, 0.01, np.float32)])
    x = np.ones((3, 256), np.float32)
    out, e, _ = oracle.moe_forward(layer, x, x @ router.T, mode=1)
    assert (e[:, 0] == 1).all() and np.isfinite(out).all()
    ref, _, _ = oracle.moe_forward(layer, x[:1], (x @ router.T)[:1], mode=0)
    assert_bitexact(out, np.repeat(ref, 3, axis=0))


def test_moe_matches_its_definition_in_f64(oracle):
    """The layer equals sum_k w_k * down(silu(gate x) * up x) + sigmoid(x.s)
    * shared(x) built from dequantised matrices in f64 (quantisation of x
    and of the SwiGLU output included), within f32 noise."""
    rng = np.random.default_rng(82)
    layer = _layer(rng, 4, top_k=2)
    x = S.normal((2, 256), rng)
    logits = S.normal((2, 4), rng)
    out, e, w = oracle.moe_forward(layer, x, logits, mode=0)

    def mm(dt, wb, rows, cols, v):
        return oracle.matmul(dt, wb, rows, cols, v.astype(np.float32)[None, :])[0].astype(np.float64)

    per = lambda dt, r, c: r * (c // 256) * (144 if dt == Q4 else 210)  # noqa: E731
    for t in range(2):
        acc = np.zeros(256)
        for k in range(2):
            ex = int(e[t, k])
            gb = layer["gate"][ex * per(Q4, 256, 256):(ex + 1) * per(Q4, 256, 256)]
            ub = layer["up"][ex * per(Q4, 256, 256):(ex + 1) * per(Q4, 256, 256)]
            db = layer["down"][ex * per(Q6, 256, 256):(ex + 1) * per(Q6, 256, 256)]
            g, u = mm(Q4, gb, 256, 256, x[t]), mm(Q4, ub, 256, 256, x[t])
            act = g / (1 + np.exp(-g)) * u
            acc += w[t, k] * mm(Q6, db, 256, 256, act)
        g, u = mm(Q4, layer["shared_gate"], 256, 256, x[t]), mm(Q4, layer["shared_up"], 256, 256, x[t])
        act = g / (1 + np.exp(-g)) * u
        gate = 1 / (1 + np.exp(-(x[t].astype(np.float64) @ layer["selector"])))
        acc += gate * mm(Q6, layer["shared_down"], 256, 256, act)
        assert_close_normwise(out[t], acc, 1e-5, f"token {t}")


# --------------------------------------------------------- golden fixtures
@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def test_golden_fixtures_reproduce(oracle, golden):
    """Regression: the oracle reproduces its committed fixtures bit for bit."""
    for dt in (Q4, Q6, Q8):
        name = S.NAMES[dt]
        n, k = golden[f"{name}_shape"]
        w, x = golden[f"{name}_w"], golden[f"{name}_x"]
        for m in (1, 2, 4, 8, 9, 16):
            assert_bitexact(oracle.matmul(dt, w, int(n), int(k), x[:m]), golden[f"{name}_y_m{m}"], f"{name} m={m}")
    qx = golden["quant_x"]
    assert np.array_equal(np.concatenate([oracle.quantize_q8k(r) for r in qx]).view(np.uint8), golden["quant_q8k"])
    assert np.array_equal(np.concatenate([oracle.quantize_q80(r) for r in qx]).view(np.uint8), golden["quant_q80"])
    e, w = oracle.top_k_routes(golden["route_logits"], 2, True)
    assert np.array_equal(e, golden["route_experts"]) and np.array_equal(w, golden["route_weights"])
    assert golden["route_experts"][0].tolist() == [1, 3]


def test_router_logits_pins(oracle):
    """The router product (src/qwen/quantized_moe.rs:253): one-hot router
    rows pick x's columns exactly; small-integer operands give the integer
    dot exactly in both orders; double and sequential f32 sums agree within
    the f32 summation bound n * eps * sum |x r|."""
    rng = np.random.default_rng(17)
    x = rng.standard_normal((5, 512), dtype=np.float32)
    cols = np.array([0, 7, 511, 100])
    onehot = np.zeros((4, 512), np.float32)
    onehot[np.arange(4), cols] = 1.0
    for order in (0, 1):
        assert np.array_equal(oracle.router_logits(x, onehot, order), x[:, cols])
    xi = rng.integers(-8, 9, (3, 512)).astype(np.float32)
    ri = rng.integers(-8, 9, (6, 512)).astype(np.float32)
    exact = xi.astype(np.int64) @ ri.astype(np.int64).T
    for order in (0, 1):
        assert np.array_equal(oracle.router_logits(xi, ri, order), exact.astype(np.float32))
    r = rng.standard_normal((256, 512), dtype=np.float32) / np.float32(np.sqrt(512))
    a, b = oracle.router_logits(x, r, 0), oracle.router_logits(x, r, 1)
    bound = 512 * np.finfo(np.float32).eps * (np.abs(x).astype(np.float64) @ np.abs(r).astype(np.float64).T)
    assert np.all(np.abs(a.astype(np.float64) - b) <= bound + np.abs(a) * np.finfo(np.float32).eps)
    ref = (x.astype(np.float64) @ r.astype(np.float64).T)
    assert np.all(np.abs(a - ref) <= np.abs(ref) * np.finfo(np.float32).eps / 2 + 1e-30)


# --------------------------------------------------------------- Q5_K
def _q5_from_q4(q4, qh):
    """Q5_K blocks with Q4_K blocks' d, dmin, scales and nibbles, plus qh."""
    q5 = np.zeros(len(q4), oracle_mod().Q5K_BLOCK)
    for f in ("d", "dmin", "scales", "qs"):
        q5[f] = q4[f]
    q5["qh"] = qh
    return q5


def oracle_mod():
    from oracle import oracle as O

    return O


def test_q5k_without_high_bits_is_q4k(oracle):
    """qh = 0 makes a Q5_K block the Q4_K block with the same other fields
    (the Q4_K decoding is pinned above): identical dequantised weights and
    block integers, and the product within f32 rounding (the mins are
    accumulated as one scalar instead of four lanes)."""
    rng = np.random.default_rng(44)
    n, nb = 6, 4
    q4 = S.random_blocks(Q4, n * nb, rng).view(oracle.Q4K_BLOCK)
    q5 = _q5_from_q4(q4, 0)
    k = 256 * nb
    assert np.array_equal(oracle.dequantize(S.Q5_K, q5.view(np.uint8), n, k),
                          oracle.dequantize(Q4, q4.view(np.uint8), n, k))
    x = S.normal((3, k), rng)
    q = oracle.quantize_q8k(x[0])
    for b in range(nb):
        assert oracle.block_textbook(S.Q5_K, q5[b], q[b]) == oracle.block_textbook(Q4, q4[b], q[b])
        l5, m5 = oracle.block_lanes(S.Q5_K, q5[b], q[b])
        l4, m4 = oracle.block_lanes(Q4, q4[b], q[b])
        assert np.array_equal(l5, l4) and np.array_equal(m5, m4)
    assert_close_normwise(oracle.matmul(S.Q5_K, q5.view(np.uint8), n, k, x),
                          oracle.matmul(Q4, q4.view(np.uint8), n, k, x), 1e-6, "Q5_K(qh=0) vs Q4_K")


def test_q5k_high_bit_placement(oracle):
    """Bit b of qh[l] adds 16 * d * scale to weight 64 (b // 2) + 32 (b % 2)
    + l and to no other weight (ggml's Q5_K layout)."""
    rng = np.random.default_rng(45)
    q4 = S.random_blocks(Q4, 1, rng).view(oracle.Q4K_BLOCK)
    base = oracle.dequantize(S.Q5_K, _q5_from_q4(q4, 0).view(np.uint8), 1, 256)[0].astype(np.float64)
    d = oracle.f16_to_f32(int(q4["d"][0]))
    sc = np.zeros(8, np.int64)
    b12 = q4["scales"][0].astype(np.int64)
    for s_ in range(4):
        sc[s_] = b12[s_] & 63
        sc[s_ + 4] = (b12[s_ + 8] & 15) | ((b12[s_] >> 6) << 4)
    for bit in range(8):
        for l in (0, 13, 31):
            qh = np.zeros(32, np.uint8)
            qh[l] = 1 << bit
            got = oracle.dequantize(S.Q5_K, _q5_from_q4(q4, qh).view(np.uint8), 1, 256)[0].astype(np.float64)
            e = 64 * (bit // 2) + 32 * (bit % 2) + l
            delta = got - base
            assert np.count_nonzero(delta) == (1 if sc[bit] else 0)
            assert abs(delta[e] - 16 * d * sc[bit]) <= 1e-6 * max(1.0, abs(got[e]))


def test_q5k_with_unit_scales_is_a_plain_integer_dot(oracle):
    rng = np.random.default_rng(46)
    nb, n = 3, 5
    blocks = np.zeros(n * nb, oracle.Q5K_BLOCK)
    blocks["d"] = 0x3C00
    blocks["scales"][:, 0:4] = 1
    blocks["scales"][:, 8:12] = 0x01
    blocks["qs"] = rng.integers(0, 256, (n * nb, 128))
    blocks["qh"] = rng.integers(0, 256, (n * nb, 32))
    w = blocks.view(np.uint8)
    x = _integer_row(256 * nb, rng)
    W = oracle.dequantize(S.Q5_K, w, n, 256 * nb).astype(np.int64)
    assert W.max() == 31 and W.min() == 0
    y = oracle.matmul(S.Q5_K, w, n, 256 * nb, x[None, :])[0]
    assert np.array_equal(y, (W @ x.astype(np.int64)).astype(np.float32))
