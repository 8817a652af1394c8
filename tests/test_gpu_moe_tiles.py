"""The grouped MoE path with its down products in tile order
(iq_moe_set_path(..., IQ_PATH_PREFILL_TILES)), through the C ABI.

Bar: routes equal the oracle's; the layer output within 1e-4 normwise of
the oracle (the path's stated f32 bar).  The tile order changes only the
f32 order of the down products (exact per-block integers, one f32 step per
output and block); a wrong integer, scale or row would move the output by
far more than the few ulps the order moves it, so each case also checks
the tile output against the default (bitwise) path of the same layer to
1e-6.  Calls the token-major path serves (up to 32 tokens here) and the
default path stay bitwise.
"""
import numpy as np
import pytest
import torch

from conftest import assert_bitexact, assert_close_normwise
from inferq_amd import _lib
from inferq_amd import moe as MOE
from inferq_amd import synth as S

pytestmark = pytest.mark.gpu

Q4, Q6 = S.Q4_K, S.Q6_K
_NAMES = {Q4: "Q4_K", Q6: "Q6_K"}


def _device_layer(layer, top_k, gpu):
    t = {k: torch.from_numpy(v).to(gpu) for k, v in layer.items() if isinstance(v, np.ndarray)}
    return MOE.QuantizedMoeLayer(
        layer["hidden"], layer["inter"], layer["n_experts"], top_k, layer["gate_dtype"], layer["down_dtype"],
        t["gate"], t["up"], t["down"], t.get("shared_gate"), t.get("shared_up"), t.get("shared_down"),
        t.get("selector")), t


def _oracle(oracle, layer, top_k, x, logits):
    d = dict(layer)
    d["top_k"] = top_k
    d["normalize"] = True
    return oracle.moe_forward(d, x, logits, mode=1, impl=1 if oracle.have_avx2() else 0, nthreads=8)


def _dirichlet_logits(m, n_experts, rng, alpha=0.3):
    p = rng.dirichlet(np.full(n_experts, alpha))
    return (S.normal((m, n_experts), rng) + np.log(np.maximum(p, 1e-30))).astype(np.float32)


def _pair(layer, top_k, gpu):
    exact, _ = _device_layer(layer, top_k, gpu)
    tiles, _ = _device_layer(layer, top_k, gpu)
    tiles.set_path(_lib.PATH_PREFILL_TILES)
    return exact, tiles


def _check(oracle, layer, top_k, exact, tiles, x, logits, gpu, what):
    xg, lg = torch.from_numpy(x).to(gpu), torch.from_numpy(logits).to(gpu)
    out_t = tiles.forward(xg, lg)
    out_e = exact.forward(xg, lg)
    ref, ref_e, ref_w = _oracle(oracle, layer, top_k, x, logits)
    assert [r.experts for r in out_t.routes] == ref_e.tolist(), what
    assert_close_normwise(np.array([r.weights for r in out_t.routes]), ref_w, 1e-6, f"route weights {what}")
    got = out_t.hidden.cpu().numpy()
    assert np.isfinite(got).all(), what
    assert_close_normwise(got, ref, 1e-4, f"tile-order down vs oracle {what}")
    assert_close_normwise(got, out_e.hidden.cpu().numpy(), 1e-6, f"tile-order down vs exact path {what}")
    return got, out_e.hidden.cpu().numpy()


@pytest.fixture(scope="module")
def qwen_layer():
    """Qwen3.6-35B-A3B-shaped: 256 experts [512 x 2048] Q4_K gate/up, Q6_K down, shared expert."""
    return S.random_moe_layer(2048, 512, 256, Q4, Q6, np.random.default_rng(2024), shared=True)


@pytest.mark.parametrize("m", [33, 64, 65, 128, 256])
def test_tile_down_matches_oracle(gpu, oracle, qwen_layer, m):
    """Skewed routing at the narrowest grouped call (33), exact multiples of
    the 32-row chunk (64, 128: the shared expert's group), one past (65) and
    the prefill width (256, where the largest groups span several chunks)."""
    exact, tiles = _pair(qwen_layer, 8, gpu)
    rng = np.random.default_rng(4100 + m)
    x = S.normal((m, 2048), rng)
    logits = _dirichlet_logits(m, 256, rng)
    _check(oracle, qwen_layer, 8, exact, tiles, x, logits, gpu, f"m={m}")


def test_tile_down_one_expert_takes_every_token(gpu, oracle, qwen_layer):
    """Every token routed to the same eight experts: eight groups of 96 rows
    (whole 32-row chunks) beside the shared expert's, then 80 tokens (two
    whole chunks and a partial one per group)."""
    exact, tiles = _pair(qwen_layer, 8, gpu)
    rng = np.random.default_rng(4200)
    x = S.normal((96, 2048), rng)
    logits = S.normal((96, 256), rng)
    logits[:, 10:18] += 40.0
    _check(oracle, qwen_layer, 8, exact, tiles, x, logits, gpu, "8 experts x 96 rows")
    _check(oracle, qwen_layer, 8, exact, tiles, x[:80], logits[:80], gpu, "8 experts x 80 rows")


@pytest.fixture(scope="module")
def format_layers():
    out = {}
    for i, (g, d) in enumerate([(Q4, Q6), (Q4, Q4), (Q6, Q6), (Q6, Q4)]):
        out[(g, d)] = S.random_moe_layer(2048, 512, 16, g, d, np.random.default_rng(4300 + i), shared=True)
    return out


@pytest.mark.parametrize("fmts", [(Q4, Q6), (Q4, Q4), (Q6, Q6), (Q6, Q4)],
                         ids=lambda f: f"{_NAMES[f[0]]}-{_NAMES[f[1]]}")
def test_tile_down_format_pairs(gpu, oracle, format_layers, fmts):
    """Q4_K and Q6_K down products (the Q4_K mins through the f16 MFMA)
    under both gate formats, 80 tokens over 16 experts at top-4."""
    layer = format_layers[fmts]
    exact, tiles = _pair(layer, 4, gpu)
    rng = np.random.default_rng(4400)
    x = S.normal((80, 2048), rng)
    logits = _dirichlet_logits(80, 16, rng, alpha=1.0)
    _check(oracle, layer, 4, exact, tiles, x, logits, gpu, f"{_NAMES[fmts[0]]}/{_NAMES[fmts[1]]}")


@pytest.mark.parametrize("inter", [256, 768])
def test_tile_down_other_intermediate_widths(gpu, oracle, inter):
    """Intermediate widths of one and three blocks (the activations staged
    block by block beside the weights instead of held for the workgroup),
    hidden 1024, 32 experts at top-4, 96 tokens."""
    layer = S.random_moe_layer(1024, inter, 32, Q4, Q6, np.random.default_rng(4700 + inter), shared=True)
    exact, tiles = _pair(layer, 4, gpu)
    rng = np.random.default_rng(4701)
    x = S.normal((96, 1024), rng)
    logits = _dirichlet_logits(96, 32, rng, alpha=0.5)
    _check(oracle, layer, 4, exact, tiles, x, logits, gpu, f"intermediate {inter}")


def test_tile_down_512_experts_top10_sliced(gpu, oracle):
    """512 experts at top-10 plus the shared expert, 512 tokens: the call
    runs as slices; routes equal, output within the bar."""
    layer = S.random_moe_layer(2048, 512, 512, Q4, Q6, np.random.default_rng(4500), shared=True)
    exact, tiles = _pair(layer, 10, gpu)
    rng = np.random.default_rng(4501)
    x = S.normal((512, 2048), rng)
    logits = S.normal((512, 512), rng)
    _check(oracle, layer, 10, exact, tiles, x, logits, gpu, "512 experts top-10, 512 tokens")


def test_tile_path_leaves_token_major_and_default_bitwise(gpu, qwen_layer):
    """Token-major calls (1, 8, 32 tokens) on a tile-order handle are the
    exact path's bits; switching back to IQ_PATH_AUTO restores the grouped
    path's bits; the call is deterministic."""
    exact, tiles = _pair(qwen_layer, 8, gpu)
    rng = np.random.default_rng(4600)
    for m in (1, 8, 32):
        x = torch.from_numpy(S.normal((m, 2048), rng)).to(gpu)
        lg = torch.from_numpy(S.normal((m, 256), rng)).to(gpu)
        assert_bitexact(tiles.forward(x, lg).hidden.cpu().numpy(), exact.forward(x, lg).hidden.cpu().numpy(),
                        f"token-major m={m}")
    x = torch.from_numpy(S.normal((200, 2048), rng)).to(gpu)
    lg = torch.from_numpy(_dirichlet_logits(200, 256, rng)).to(gpu)
    a = tiles.forward(x, lg).hidden.cpu().numpy()
    assert_bitexact(tiles.forward(x, lg).hidden.cpu().numpy(), a, "tile-order call repeated")
    tiles.set_path(_lib.PATH_AUTO)
    assert_bitexact(tiles.forward(x, lg).hidden.cpu().numpy(), exact.forward(x, lg).hidden.cpu().numpy(),
                    "back on IQ_PATH_AUTO")


def test_tile_path_from_x_with_residual(gpu, qwen_layer):
    """The whole sublayer from x (router on the GPU, residual added last) on
    a tile-order handle: routes equal the default handle's, the output
    within 1e-6 of it, and the residual is added after the combine."""
    rng = np.random.default_rng(4800)
    layer = dict(qwen_layer)
    router = (rng.standard_normal((256, 2048), dtype=np.float32) / np.float32(np.sqrt(2048)))
    t = {k: torch.from_numpy(v).to(gpu) for k, v in layer.items() if isinstance(v, np.ndarray)}
    rt = torch.from_numpy(router).to(gpu)

    def make():
        return MOE.QuantizedMoeLayer(2048, 512, 256, 8, Q4, Q6, t["gate"], t["up"], t["down"], t["shared_gate"],
                                     t["shared_up"], t["shared_down"], t["selector"], router=rt)

    exact, tiles = make(), make()
    tiles.set_path(_lib.PATH_PREFILL_TILES)
    x = torch.from_numpy(S.normal((96, 2048), rng)).to(gpu)
    res = torch.from_numpy(S.normal((96, 2048), rng)).to(gpu)
    a, b = tiles.forward(x, residual=res), exact.forward(x, residual=res)
    assert [r.experts for r in a.routes] == [r.experts for r in b.routes]
    assert_close_normwise(a.hidden.cpu().numpy(), b.hidden.cpu().numpy(), 1e-6, "from x, tiles vs exact")
    plain = tiles.forward(x).hidden
    assert_close_normwise((plain + res).cpu().numpy(), a.hidden.cpu().numpy(), 1e-6, "residual added last")


def test_tile_path_graph_replays_match_eager_calls(gpu, qwen_layer):
    """A tile-order call captured in a HIP graph (after iq_moe_reserve, no
    eager call first) and replayed with fresh inputs and eager work between
    replays gives the eager call's bits each time."""
    _, tiles = _pair(qwen_layer, 8, gpu)
    m = 96
    tiles.reserve(m)
    rng = np.random.default_rng(4900)
    xs = [torch.from_numpy(S.normal((m, 2048), rng)).to(gpu) for _ in range(3)]
    ls = [torch.from_numpy(_dirichlet_logits(m, 256, rng)).to(gpu) for _ in range(3)]
    x_buf, l_buf, o_buf = torch.zeros(m, 2048, device=gpu), torch.zeros(m, 256, device=gpu), \
        torch.empty(m, 2048, device=gpu)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        tiles.forward_into(x_buf, l_buf, o_buf)
    eager = []
    for x, lg in zip(xs, ls):
        o = torch.empty(m, 2048, device=gpu)
        tiles.forward_into(x, lg, o)
        eager.append(o.cpu().numpy())
    for rep in range(2):
        for i in range(3):
            x_buf.copy_(xs[i])
            l_buf.copy_(ls[i])
            graph.replay()
            torch.cuda.synchronize()
            assert_bitexact(o_buf.cpu().numpy(), eager[i], f"replay {rep}.{i}")
            o = torch.empty(m, 2048, device=gpu)
            tiles.forward_into(xs[(i + 1) % 3], ls[(i + 1) % 3], o)
            torch.cuda.synchronize()
            assert_bitexact(o.cpu().numpy(), eager[(i + 1) % 3], "eager between replays")


def test_set_path_refuses_other_paths(gpu, qwen_layer):
    moe, _ = _device_layer(qwen_layer, 8, gpu)
    for path in (_lib.PATH_LANES, _lib.PATH_GEMV, _lib.PATH_LANE_MFMA, 99, -1):
        with pytest.raises(_lib.QgemmError, match="expected IQ_PATH_AUTO or IQ_PATH_PREFILL_TILES"):
            moe.set_path(path)
