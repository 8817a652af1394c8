"""GPU parity of the MoE sublayer (routing, grouped experts, SwiGLU,
ordered combine, shared expert) through the C ABI.

Tolerance: normwise relative error <= 1e-4 on the layer output (the path's
stated f32 bar).  The expert matmuls are bit-exact; what may differ from
the oracle is (a) exp: the GPU rounds exp once from double, the reference
calls glibc expf, which agree except where expf misrounds near a midpoint,
and (b) the shared-expert selector dot x.s, whose accumulation order inside
candle's f32 gemm is not visible here (a tree on the GPU, double in the
oracle).  Routes (experts) must match exactly.
"""
import numpy as np
import pytest
import torch

from conftest import assert_bitexact, assert_close_normwise
from inferq_amd import moe as MOE
from inferq_amd import synth as S

pytestmark = pytest.mark.gpu

Q4, Q6, Q8 = S.Q4_K, S.Q6_K, S.Q8_0


def _device_layer(layer, top_k, gpu, normalize=True, router=None):
    t = {k: torch.from_numpy(v).to(gpu) for k, v in layer.items() if isinstance(v, np.ndarray)}
    return MOE.QuantizedMoeLayer(
        layer["hidden"], layer["inter"], layer["n_experts"], top_k, layer["gate_dtype"], layer["down_dtype"],
        t["gate"], t["up"], t["down"], t.get("shared_gate"), t.get("shared_up"), t.get("shared_down"),
        t.get("selector"), normalize=normalize, shared_gate_dtype=layer.get("shared_gate_dtype"),
        shared_down_dtype=layer.get("shared_down_dtype"),
        router=None if router is None else torch.from_numpy(router).to(gpu)), t


def _oracle_layer(layer, top_k, normalize=True):
    d = dict(layer)
    d["top_k"] = top_k
    d["normalize"] = normalize
    return d


def _impl(oracle):
    return 1 if oracle.have_avx2() else 0


@pytest.mark.parametrize("shared", [False, True])
@pytest.mark.parametrize("m", [1, 3, 8])
def test_small_moe_matches_oracle(gpu, oracle, shared, m):
    rng = np.random.default_rng(100 + m + 10 * shared)
    layer = S.random_moe_layer(256, 256, 8, Q4, Q6, rng, shared=shared)
    moe, _ = _device_layer(layer, 2, gpu)
    x = S.normal((m, 256), rng)
    logits = S.normal((m, 8), rng)
    out = moe.forward(torch.from_numpy(x).to(gpu), torch.from_numpy(logits).to(gpu))
    ref_tm, ref_e, ref_w = oracle.moe_forward(_oracle_layer(layer, 2), x, logits, mode=0, impl=_impl(oracle))
    ref_gr, _, _ = oracle.moe_forward(_oracle_layer(layer, 2), x, logits, mode=1, impl=_impl(oracle))
    assert_bitexact(ref_gr, ref_tm, "oracle grouped vs token-major")
    assert [r.experts for r in out.routes] == ref_e.tolist()
    got = out.hidden.cpu().numpy()
    assert_close_normwise(np.array([r.weights for r in out.routes]), ref_w, 1e-6, "route weights")
    assert_close_normwise(got, ref_tm, 1e-4, f"MoE m={m} shared={shared}")
    if not shared:
        assert_bitexact(got, ref_tm, f"routed-only MoE m={m}")


@pytest.fixture(scope="module")
def qwen_layer():
    """Config-2 shaped layer: hidden 2048, 256 experts of [512 x 2048] Q4_K
    gate/up and [2048 x 512] Q6_K down, one shared expert."""
    rng = np.random.default_rng(2024)
    return S.random_moe_layer(2048, 512, 256, Q4, Q6, rng, shared=True)


@pytest.mark.parametrize("m", [1, 2, 4, 8, 11, 12])
def test_qwen_shaped_moe_matches_oracle(gpu, oracle, qwen_layer, m):
    """Token-major widths: the one-token kernel (1), the 16-row gate/up
    workgroups with their own top-k (2..11) and after a routing launch (12)."""
    moe, _ = _device_layer(qwen_layer, 8, gpu)
    rng = np.random.default_rng(7 + m)
    x = S.normal((m, 2048), rng)
    logits = S.normal((m, 256), rng)
    out = moe.forward(torch.from_numpy(x).to(gpu), torch.from_numpy(logits).to(gpu))
    ref, ref_e, ref_w = oracle.moe_forward(_oracle_layer(qwen_layer, 8), x, logits, mode=1, impl=_impl(oracle),
                                           nthreads=8)
    assert [r.experts for r in out.routes] == ref_e.tolist()
    assert_close_normwise(out.hidden.cpu().numpy(), ref, 1e-4, f"Qwen-shaped MoE m={m}")


@pytest.mark.parametrize("m", [1, 2, 4, 8, 12])
def test_tied_logits_route_like_oracle(gpu, oracle, qwen_layer, m):
    """Equal logits rank by lower index (src/qwen/moe.rs:21-54 as fixed in
    route order): logits on a half-unit grid tie often, one row ties
    everywhere, and +0 / -0 compare equal.  Covers the per-slot rank search
    of the 2..11-token gate/up workgroups and the rounds elsewhere."""
    moe, _ = _device_layer(qwen_layer, 8, gpu)
    rng = np.random.default_rng(300 + m)
    x = S.normal((m, 2048), rng)
    logits = np.round(S.normal((m, 256), rng) * 2.0).astype(np.float32) / 2.0
    logits[0, :] = 0.25
    if m > 1:
        logits[1, ::2] = -0.0
        logits[1, 1::2] = 0.0
    out = moe.forward(torch.from_numpy(x).to(gpu), torch.from_numpy(logits).to(gpu))
    ref, ref_e, _ = oracle.moe_forward(_oracle_layer(qwen_layer, 8), x, logits, mode=1, impl=_impl(oracle), nthreads=8)
    assert [r.experts for r in out.routes] == ref_e.tolist()
    assert out.routes[0].experts == list(range(8))
    assert_close_normwise(out.hidden.cpu().numpy(), ref, 1e-4, f"tied logits m={m}")


_NAMES = {Q4: "q4k", Q6: "q6k", Q8: "q80"}
_FORMAT_PAIRS = [(Q4, Q6), (Q4, Q4), (Q6, Q6), (Q6, Q4), (Q8, Q8), (Q8, Q6)]


@pytest.fixture(scope="module")
def format_layers():
    """hidden 2048, inter 512 (the shape of the token-major kernels), 16
    experts, one shared expert, one layer per gate/down format pair."""
    out = {}
    for i, (g, d) in enumerate(_FORMAT_PAIRS):
        out[(g, d)] = S.random_moe_layer(2048, 512, 16, g, d, np.random.default_rng(500 + i), shared=True)
    return out


@pytest.mark.parametrize("m", [1, 8, 64])
@pytest.mark.parametrize("fmts", _FORMAT_PAIRS, ids=lambda f: f"{_NAMES[f[0]]}-{_NAMES[f[1]]}")
def test_format_pairs_match_oracle(gpu, oracle, format_layers, fmts, m):
    """Every gate/down format pair at one row, a verify width and a prefill
    width (K-quant pairs take the token-major kernels up to 32 rows and the
    grouped MFMA kernels past that; Q8_0 the generic grouped path); a
    multi-row call equals one-row calls, bitwise."""
    layer = format_layers[fmts]
    moe, _ = _device_layer(layer, 4, gpu)
    rng = np.random.default_rng(600 + m)
    x = S.normal((m, 2048), rng)
    logits = _dirichlet_logits(m, 16, rng, alpha=1.0)
    xg, lg = torch.from_numpy(x).to(gpu), torch.from_numpy(logits).to(gpu)
    out = moe.forward(xg, lg)
    ref, ref_e, ref_w = oracle.moe_forward(_oracle_layer(layer, 4), x, logits, mode=1, impl=_impl(oracle),
                                           nthreads=8)
    assert [r.experts for r in out.routes] == ref_e.tolist()
    assert_close_normwise(np.array([r.weights for r in out.routes]), ref_w, 1e-6, "route weights")
    got = out.hidden.cpu().numpy()
    assert_close_normwise(got, ref, 1e-4, f"MoE {fmts} m={m}")
    if m > 1:
        singles = np.concatenate([moe.forward(xg[i:i + 1], lg[i:i + 1]).hidden.cpu().numpy() for i in range(m)])
        assert_bitexact(got, singles, f"grouped vs per-token {fmts} m={m}")


def _dirichlet_logits(m, n_experts, rng, alpha=0.3):
    """Router logits N(0,1) plus log p with p ~ Dirichlet(alpha): per-expert
    token counts follow that skew (prefill width)."""
    p = rng.dirichlet(np.full(n_experts, alpha))
    return (S.normal((m, n_experts), rng) + np.log(np.maximum(p, 1e-30))).astype(np.float32)


@pytest.mark.parametrize("m", [17, 28, 32, 33, 48, 256])
def test_prefill_width_moe_matches_oracle(gpu, oracle, qwen_layer, m):
    """Wide calls with skewed routing (large groups on a few experts, most
    experts idle): token-major calls (17, 28, and 32, the widest), the
    narrowest grouped MFMA call (33), 48 and the prefill width of 256."""
    moe, _ = _device_layer(qwen_layer, 8, gpu)
    rng = np.random.default_rng(300 + m)
    x = S.normal((m, 2048), rng)
    logits = _dirichlet_logits(m, 256, rng)
    out = moe.forward(torch.from_numpy(x).to(gpu), torch.from_numpy(logits).to(gpu))
    ref, ref_e, ref_w = oracle.moe_forward(_oracle_layer(qwen_layer, 8), x, logits, mode=1, impl=_impl(oracle),
                                           nthreads=8)
    assert [r.experts for r in out.routes] == ref_e.tolist()
    assert_close_normwise(np.array([r.weights for r in out.routes]), ref_w, 1e-6, "route weights")
    assert_close_normwise(out.hidden.cpu().numpy(), ref, 1e-4, f"prefill-width MoE m={m}")


@pytest.fixture(scope="module")
def qwen_layer_routed_only():
    """The config-2 shape without a shared expert (32 experts)."""
    return S.random_moe_layer(2048, 512, 32, Q4, Q6, np.random.default_rng(2025), shared=False)


@pytest.mark.parametrize("top_k", [1, 8])
@pytest.mark.parametrize("m", [1, 4, 64])
def test_routed_only_layer_matches_oracle(gpu, oracle, qwen_layer_routed_only, top_k, m):
    """No shared expert (no shared slot in the token-major grids, no shared
    rows in the grouped path) at top-1 and top-8: routes equal, outputs
    within the bar, multi-token calls equal one-token calls."""
    layer = qwen_layer_routed_only
    moe, _ = _device_layer(layer, top_k, gpu)
    rng = np.random.default_rng(900 + 10 * m + top_k)
    x = S.normal((m, 2048), rng)
    logits = S.normal((m, 32), rng)
    xg, lg = torch.from_numpy(x).to(gpu), torch.from_numpy(logits).to(gpu)
    out = moe.forward(xg, lg)
    ref, ref_e, _ = oracle.moe_forward(_oracle_layer(layer, top_k), x, logits, mode=1, impl=_impl(oracle),
                                       nthreads=8)
    assert [r.experts for r in out.routes] == ref_e.tolist()
    got = out.hidden.cpu().numpy()
    assert_close_normwise(got, ref, 1e-4, f"routed-only MoE top-{top_k} m={m}")
    if m > 1:
        singles = np.concatenate([moe.forward(xg[i:i + 1], lg[i:i + 1]).hidden.cpu().numpy() for i in range(m)])
        assert_bitexact(got, singles, f"routed-only grouped vs per-token m={m}")


@pytest.mark.parametrize("m", [3, 12, 24, 64])
def test_skewed_grouped_call_equals_single_token_calls(gpu, qwen_layer, m):
    """m rows with skewed routing in one call (token-major at 3, 12 and 24,
    grouped by expert at 64) equal m one-row calls."""
    moe, _ = _device_layer(qwen_layer, 8, gpu)
    rng = np.random.default_rng(98)
    x = torch.from_numpy(S.normal((m, 2048), rng)).to(gpu)
    logits = torch.from_numpy(_dirichlet_logits(m, 256, rng)).to(gpu)
    grouped = moe.forward(x, logits).hidden.cpu().numpy()
    singles = np.concatenate([moe.forward(x[i:i + 1], logits[i:i + 1]).hidden.cpu().numpy() for i in range(m)])
    assert_bitexact(grouped, singles, f"skewed {m}-row call vs per-token")


def test_grouped_equals_single_token_calls(gpu, qwen_layer):
    """A multi-token (grouped) call equals one call per token, bitwise
    (src/qwen/quantized_moe.rs:570-591)."""
    moe, _ = _device_layer(qwen_layer, 8, gpu)
    rng = np.random.default_rng(99)
    x = torch.from_numpy(S.normal((8, 2048), rng)).to(gpu)
    logits = torch.from_numpy(S.normal((8, 256), rng)).to(gpu)
    grouped = moe.forward(x, logits).hidden.cpu().numpy()
    singles = np.concatenate([moe.forward(x[i:i + 1], logits[i:i + 1]).hidden.cpu().numpy() for i in range(8)])
    assert_bitexact(grouped, singles, "grouped vs per-token")


def test_reference_routing_case(gpu, oracle):
    """The reference's MoE test (src/qwen/quantized_moe.rs:490-592): a router
    whose second row is 0.01 everywhere and an all-ones input pick expert 1
    at top-1; outputs are finite; three identical rows grouped equal one."""
    rng = np.random.default_rng(1)
    layer = S.random_moe_layer(256, 256, 2, Q4, Q4, rng, shared=True)
    moe, _ = _device_layer(layer, 1, gpu)
    router = np.stack([np.zeros(256, np.float32), np.full(256, 0.01, np.float32)])
    x = np.ones((1, 256), np.float32)
    logits = x @ router.T
    out = moe.forward(torch.from_numpy(x).to(gpu), torch.from_numpy(logits).to(gpu))
    assert out.routes[0].experts == [1]
    assert out.hidden.shape == (1, 256)
    h = out.hidden.cpu().numpy()
    assert np.isfinite(h).all()
    batch = np.ones((3, 256), np.float32)
    grouped = moe.forward(torch.from_numpy(batch).to(gpu), torch.from_numpy(batch @ router.T).to(gpu))
    for r in grouped.routes:
        assert r.experts == [1] and r.weights == out.routes[0].weights
    assert_bitexact(grouped.hidden.cpu().numpy(), np.repeat(h, 3, axis=0), "grouped vs token-major")


def test_empty_token_batch(gpu, oracle):
    """Zero tokens: an empty output with no routes, and the next call is
    unaffected."""
    rng = np.random.default_rng(2)
    layer = S.random_moe_layer(256, 256, 8, Q4, Q6, rng, shared=True)
    moe, _ = _device_layer(layer, 2, gpu)
    out = moe.forward(torch.zeros(0, 256, device=gpu), torch.zeros(0, 8, device=gpu))
    assert out.hidden.shape == (0, 256) and out.routes == []
    x, logits = S.normal((2, 256), rng), S.normal((2, 8), rng)
    got = moe.forward(torch.from_numpy(x).to(gpu), torch.from_numpy(logits).to(gpu))
    ref, _, _ = oracle.moe_forward(_oracle_layer(layer, 2), x, logits, mode=0, impl=_impl(oracle))
    assert_close_normwise(got.hidden.cpu().numpy(), ref, 1e-4, "MoE after an empty call")


def test_moe_load_time_errors(gpu):
    from inferq_amd import QgemmError

    rng = np.random.default_rng(2)
    layer = S.random_moe_layer(256, 256, 4, Q4, Q6, rng, shared=False)
    t = {k: torch.from_numpy(v).to(gpu) for k, v in layer.items() if isinstance(v, np.ndarray)}
    with pytest.raises(QgemmError, match="invalid top-k 5 for 4 experts"):
        MOE.QuantizedMoeLayer(256, 256, 4, 5, Q4, Q6, t["gate"], t["up"], t["down"])
    with pytest.raises(QgemmError, match="up expert shape"):
        MOE.QuantizedMoeLayer(256, 256, 4, 2, Q4, Q6, t["gate"], t["up"][:-144], t["down"])
    with pytest.raises(QgemmError, match="selector"):
        MOE.QuantizedMoeLayer(256, 256, 4, 2, Q4, Q6, t["gate"], t["up"], t["down"], t["gate"][:256 * 144],
                              t["up"][:256 * 144], t["down"][:256 * 210], None)


@pytest.mark.parametrize("m", [1, 4, 64])
def test_graph_replays_match_eager_calls(gpu, qwen_layer, m):
    """A layer call captured in a HIP graph and replayed several times, with
    fresh inputs copied into its buffers and eager work between replays,
    gives bitwise the eager call's output each time (no allocation, memset
    or host copy is recorded into the graph)."""
    moe, _ = _device_layer(qwen_layer, 8, gpu)
    rng = np.random.default_rng(300 + m)
    xs = [torch.from_numpy(S.normal((m, 2048), rng)).to(gpu) for _ in range(3)]
    ls = [torch.from_numpy(S.normal((m, 256), rng)).to(gpu) for _ in range(3)]
    eager = []
    for x, lg in zip(xs, ls):
        o = torch.empty(m, 2048, device=gpu)
        moe.forward_into(x, lg, o)
        eager.append(o.cpu().numpy())
    x_buf, l_buf, o_buf = torch.zeros(m, 2048, device=gpu), torch.zeros(m, 256, device=gpu), \
        torch.empty(m, 2048, device=gpu)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        moe.forward_into(x_buf, l_buf, o_buf)  # sizes the workspace outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        moe.forward_into(x_buf, l_buf, o_buf)
    for rep in range(2):
        for i in range(3):
            x_buf.copy_(xs[i])
            l_buf.copy_(ls[i])
            graph.replay()
            torch.cuda.synchronize()
            assert_bitexact(o_buf.cpu().numpy(), eager[i], f"replay {rep}.{i} m={m}")
            o = torch.empty(m, 2048, device=gpu)  # eager work between replays
            moe.forward_into(xs[(i + 1) % 3], ls[(i + 1) % 3], o)
            torch.cuda.synchronize()
            assert_bitexact(o.cpu().numpy(), eager[(i + 1) % 3], "eager between replays")


def _mixed_layer(rng, hidden, inter, n_experts, gate_dtype, down_dtype, shared_gate_dtype, shared_down_dtype):
    """A layer whose shared expert has its own formats (a GGUF file may mix
    them per tensor; QuantizedMoeLayer::load takes each as it comes)."""
    layer = S.random_moe_layer(hidden, inter, n_experts, gate_dtype, down_dtype, rng, shared=False)
    layer.update({
        "shared_gate_dtype": shared_gate_dtype, "shared_down_dtype": shared_down_dtype,
        "shared_gate": S.random_matrix(shared_gate_dtype, inter, hidden, rng),
        "shared_up": S.random_matrix(shared_gate_dtype, inter, hidden, rng),
        "shared_down": S.random_matrix(shared_down_dtype, hidden, inter, rng),
        "selector": rng.standard_normal(hidden, dtype=np.float32) / np.float32(np.sqrt(hidden)),
    })
    return layer


def test_reference_mixed_format_layer(gpu, oracle):
    """The reference's own MoE GGUF test layer (src/qwen/quantized_moe.rs:
    490-592): hidden and intermediate 256, two experts, top-1, Q4_K gate/up,
    Q5_K down, a Q8_0 shared expert with a zero selector, and a router whose
    second row is 0.01 everywhere.  On an input of ones the route is expert 1
    and the output is finite; three tokens in one call equal three one-token
    calls bitwise (the reference: grouped == token-major); the output matches
    the oracle within 1e-4 (Q5_K bitwise is unpinned by nature)."""
    rng = np.random.default_rng(490)
    layer = _mixed_layer(rng, 256, 256, 2, Q4, S.Q5_K, Q8, Q8)
    layer["selector"] = np.zeros(256, np.float32)
    router = np.concatenate([np.zeros(256, np.float32), np.full(256, 0.01, np.float32)]).reshape(2, 256)
    moe, _ = _device_layer(layer, 1, gpu, router=router)
    ones = torch.ones(1, 256, device=gpu)
    out = moe.forward(ones)
    assert [r.experts for r in out.routes] == [[1]]
    assert np.isfinite(out.hidden.cpu().numpy()).all()
    batch = torch.ones(3, 256, device=gpu)
    wide = moe.forward(batch).hidden.cpu().numpy()
    singles = np.concatenate([moe.forward(batch[i:i + 1]).hidden.cpu().numpy() for i in range(3)])
    assert_bitexact(wide, singles, "3 tokens vs one-token calls")
    x = S.normal((4, 256), rng)
    logits = S.normal((4, 2), rng)
    got = moe.forward(torch.from_numpy(x).to(gpu), torch.from_numpy(logits).to(gpu))
    ref, ref_e, _ = oracle.moe_forward(_oracle_layer(layer, 1), x, logits, mode=0, impl=_impl(oracle))
    assert [r.experts for r in got.routes] == ref_e.tolist()
    assert_close_normwise(got.hidden.cpu().numpy(), ref, 1e-4, "reference mixed-format layer")


@pytest.mark.parametrize("formats", [(Q4, Q6, Q6, Q4), (Q4, Q6, Q8, Q8), (S.Q5_K, Q6, Q4, Q6), (Q4, S.Q5_K, Q4, S.Q5_K)],
                         ids=["q4q6-shared-q6q4", "q4q6-shared-q8", "q5q6-shared-q4q6", "q4q5-shared-q4q5"])
def test_mixed_format_layers_match_oracle(gpu, oracle, formats):
    """Qwen-shaped layers (hidden 2048, intermediate 512, 32 experts, top-4)
    with Q5_K experts or a shared expert in other formats than the routed
    ones, at 1, 5 and 40 tokens (token-major, grouped): routes equal the
    oracle's, outputs within 1e-4 of it, and every token's output bitwise
    the one-token call's."""
    g, d, sg, sd = formats
    rng = np.random.default_rng(sum(formats))
    layer = _mixed_layer(rng, 2048, 512, 32, g, d, sg, sd)
    moe, _ = _device_layer(layer, 4, gpu)
    for m in (1, 5, 40):
        x = S.normal((m, 2048), rng)
        logits = S.normal((m, 32), rng)
        xt, lt = torch.from_numpy(x).to(gpu), torch.from_numpy(logits).to(gpu)
        out = moe.forward(xt, lt)
        ref, ref_e, _ = oracle.moe_forward(_oracle_layer(layer, 4), x, logits, mode=0, impl=_impl(oracle),
                                           nthreads=8)
        assert [r.experts for r in out.routes] == ref_e.tolist(), f"routes m={m}"
        got = out.hidden.cpu().numpy()
        assert_close_normwise(got, ref, 1e-4, f"mixed formats {formats} m={m}")
        if m > 1:
            singles = np.concatenate([moe.forward(xt[i:i + 1], lt[i:i + 1]).hidden.cpu().numpy() for i in range(m)])
            assert_bitexact(got, singles, f"{m} tokens vs one-token calls")


def test_mixed_format_residual_is_added_last(gpu):
    """With the shared expert run apart, out = residual + (routed + shared *
    gate): bitwise the output without the residual, plus the residual."""
    rng = np.random.default_rng(212)
    layer = _mixed_layer(rng, 2048, 512, 32, Q4, Q6, Q6, Q4)
    router = rng.standard_normal((32, 2048), dtype=np.float32) / np.float32(45.0)
    moe, _ = _device_layer(layer, 4, gpu, router=router)
    x = torch.from_numpy(S.normal((3, 2048), rng)).to(gpu)
    r = torch.from_numpy(S.normal((3, 2048), rng)).to(gpu)
    plain = moe.forward(x).hidden
    with_res = moe.forward(x, residual=r).hidden
    assert_bitexact(with_res.cpu().numpy(), (plain + r).cpu().numpy(), "residual + MoE(x)")


@pytest.mark.parametrize("m", [1, 40])
def test_mixed_format_graph_replays_match_eager_calls(gpu, m):
    """A layer whose shared expert runs apart (its own formats), captured in
    a HIP graph and replayed with fresh inputs and eager calls between the
    replays: bitwise the eager output each time."""
    rng = np.random.default_rng(600 + m)
    layer = _mixed_layer(rng, 2048, 512, 32, Q4, Q6, Q6, Q4)
    moe, _ = _device_layer(layer, 4, gpu)
    xs = [torch.from_numpy(S.normal((m, 2048), rng)).to(gpu) for _ in range(3)]
    ls = [torch.from_numpy(S.normal((m, 32), rng)).to(gpu) for _ in range(3)]
    eager = []
    for x, lg in zip(xs, ls):
        o = torch.empty(m, 2048, device=gpu)
        moe.forward_into(x, lg, o)
        eager.append(o.cpu().numpy())
    x_buf, l_buf, o_buf = torch.zeros(m, 2048, device=gpu), torch.zeros(m, 32, device=gpu), \
        torch.empty(m, 2048, device=gpu)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        moe.forward_into(x_buf, l_buf, o_buf)  # sizes the workspace outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        moe.forward_into(x_buf, l_buf, o_buf)
    for rep in range(2):
        for i in range(3):
            x_buf.copy_(xs[i])
            l_buf.copy_(ls[i])
            graph.replay()
            torch.cuda.synchronize()
            assert_bitexact(o_buf.cpu().numpy(), eager[i], f"replay {rep}.{i} m={m}")
            o = torch.empty(m, 2048, device=gpu)
            moe.forward_into(xs[(i + 1) % 3], ls[(i + 1) % 3], o)
            torch.cuda.synchronize()
            assert_bitexact(o.cpu().numpy(), eager[(i + 1) % 3], "eager between replays")


@pytest.fixture(scope="module")
def wide_router_layer():
    """512 experts, top-10 plus the shared expert (eleven slots; the
    Qwen3-Next routing shape at hidden 2048, intermediate 512)."""
    return S.random_moe_layer(2048, 512, 512, Q4, Q6, np.random.default_rng(2026), shared=True)


@pytest.mark.parametrize("m", [1, 5, 12, 32, 40])
def test_512_experts_top10_matches_oracle(gpu, oracle, wide_router_layer, m):
    """Eleven slots per token through every token-major form (1, 5, 12 and
    32 tokens) and the grouped MFMA path (40): routes equal the oracle's,
    outputs within 1e-4, and the call equals one call per token bitwise."""
    moe, _ = _device_layer(wide_router_layer, 10, gpu)
    rng = np.random.default_rng(3100 + m)
    x = S.normal((m, 2048), rng)
    logits = S.normal((m, 512), rng)
    xg, lg = torch.from_numpy(x).to(gpu), torch.from_numpy(logits).to(gpu)
    out = moe.forward(xg, lg)
    ref, ref_e, ref_w = oracle.moe_forward(_oracle_layer(wide_router_layer, 10), x, logits, mode=1,
                                           impl=_impl(oracle), nthreads=8)
    assert [r.experts for r in out.routes] == ref_e.tolist()
    assert_close_normwise(np.array([r.weights for r in out.routes]), ref_w, 1e-6, "route weights")
    got = out.hidden.cpu().numpy()
    assert_close_normwise(got, ref, 1e-4, f"512-expert top-10 MoE m={m}")
    if m > 1:
        singles = np.concatenate([moe.forward(xg[i:i + 1], lg[i:i + 1]).hidden.cpu().numpy() for i in range(m)])
        assert_bitexact(got, singles, f"512-expert top-10 m={m} vs per-token")


def test_random_layers_match_oracle(gpu, oracle):
    """A seeded sweep over the token-major and grouped paths: expert counts
    16-96, top-k 1-10, with or without the shared expert, Q4_K or Q6_K
    experts, 1-40 tokens.  Routes equal the oracle's, outputs within 1e-4."""
    rng = np.random.default_rng(777)
    for case in range(12):
        E = int(rng.choice([16, 40, 96]))
        K = int(rng.integers(1, 11))
        shared = bool(rng.integers(0, 2))
        g, d = [(Q4, Q6), (Q4, Q4), (Q6, Q6), (Q6, Q4)][case % 4]
        m = int(rng.choice([1, int(rng.integers(2, 9)), int(rng.integers(9, 33)), int(rng.integers(33, 41))]))
        layer = S.random_moe_layer(2048, 512, E, g, d, rng, shared=shared)
        moe, _ = _device_layer(layer, K, gpu)
        x = S.normal((m, 2048), rng)
        logits = S.normal((m, E), rng)
        out = moe.forward(torch.from_numpy(x).to(gpu), torch.from_numpy(logits).to(gpu))
        ref, ref_e, _ = oracle.moe_forward(_oracle_layer(layer, K), x, logits, mode=1, impl=_impl(oracle), nthreads=8)
        what = f"case {case}: E={E} K={K} shared={shared} {_NAMES[g]}/{_NAMES[d]} m={m}"
        assert [r.experts for r in out.routes] == ref_e.tolist(), what
        assert_close_normwise(out.hidden.cpu().numpy(), ref, 1e-4, what)


def test_reference_prefill_pass_512_tokens_top10(gpu, oracle, wide_router_layer):
    """The reference's prefill pass on its first model: 512 rows
    (src/runtime.rs:44) routed top-10 of 512 experts (Qwen3-Coder-Next,
    docs/execution-path.md:20), 5,120 assignments in one call.  The call
    runs as slices of iq_moe_slice_tokens tokens; routes equal the
    oracle's, outputs within 1e-4 (shared expert), and the 512-token call
    equals two 256-token calls bitwise."""
    moe, _ = _device_layer(wide_router_layer, 10, gpu)
    assert moe.slice_tokens() < 512
    rng = np.random.default_rng(5120)
    x = S.normal((512, 2048), rng)
    logits = S.normal((512, 512), rng)
    xg, lg = torch.from_numpy(x).to(gpu), torch.from_numpy(logits).to(gpu)
    out = moe.forward(xg, lg)
    ref, ref_e, ref_w = oracle.moe_forward(_oracle_layer(wide_router_layer, 10), x, logits, mode=1,
                                           impl=_impl(oracle), nthreads=8)
    assert [r.experts for r in out.routes] == ref_e.tolist()
    assert_close_normwise(np.array([r.weights for r in out.routes]), ref_w, 1e-6, "route weights")
    got = out.hidden.cpu().numpy()
    assert_close_normwise(got, ref, 1e-4, "512-token top-10 prefill pass")
    halves = np.concatenate([moe.forward(xg[i:i + 256], lg[i:i + 256]).hidden.cpu().numpy() for i in (0, 256)])
    assert_bitexact(got, halves, "512-token call vs two 256-token calls")


Q5_LAYERS = {}


def _q5_layer(formats):
    """Config-2 shaped layers with Q5_K experts (hidden 2048, 256 experts,
    top-8, a shared expert in the same formats), built once per formats."""
    if formats not in Q5_LAYERS:
        Q5_LAYERS[formats] = S.random_moe_layer(2048, 512, 256, formats[0], formats[1],
                                                np.random.default_rng(5150 + sum(formats)), shared=True)
    return Q5_LAYERS[formats]


@pytest.mark.parametrize("formats", [(Q4, S.Q5_K), (S.Q5_K, S.Q5_K), (S.Q5_K, Q6)], ids=["q4q5", "q5q5", "q5q6"])
@pytest.mark.parametrize("m", [1, 12, 16, 33, 256])
def test_q5k_experts_on_the_fast_paths(gpu, oracle, formats, m):
    """Q5_K gate/up or down experts run on the token-major kernels (up to 32
    tokens: the lane kernel's products and mins scalar; from 12 tokens with
    the routing launch, from 16 with the SwiGLU rows quantised once) and on
    the grouped MFMA path (16-row tiles with three weight streams): routes
    equal the oracle's, outputs within 1e-4 of it, every token bitwise the
    one-token call."""
    layer = _q5_layer(formats)
    moe, _ = _device_layer(layer, 8, gpu)
    rng = np.random.default_rng(700 + m)
    x = S.normal((m, 2048), rng)
    logits = S.normal((m, 256), rng)
    xt, lt = torch.from_numpy(x).to(gpu), torch.from_numpy(logits).to(gpu)
    out = moe.forward(xt, lt)
    ref, ref_e, _ = oracle.moe_forward(_oracle_layer(layer, 8), x, logits, mode=1, impl=_impl(oracle), nthreads=8)
    assert [r.experts for r in out.routes] == ref_e.tolist(), f"routes m={m}"
    got = out.hidden.cpu().numpy()
    for r in range(m):
        assert_close_normwise(got[r], ref[r], 1e-4, f"Q5_K experts {formats} m={m} row {r}")
    if m > 1:
        idx = sorted({0, m // 2, m - 1})
        singles = np.concatenate([moe.forward(xt[i:i + 1], lt[i:i + 1]).hidden.cpu().numpy() for i in idx])
        assert_bitexact(got[idx], singles, f"Q5_K experts {formats} m={m} vs one-token calls")
