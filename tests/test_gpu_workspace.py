"""Workspaces under graph capture, through the C ABI.

A handle that never ran eagerly can be captured at one token (iq_moe_create
sizes its workspace for one token) and, after iq_moe_reserve /
iq_matmul_reserve, at wider calls; a graph captured before a wider eager
call on the same handle or stream stays valid (the outgrown buffer is kept,
not freed); iq_workspace_release frees a stream's workspace and the next
call allocates again.  Every replay is compared bitwise with the eager
result of the same inputs, with eager work between replays.
"""
import numpy as np
import pytest
import torch

from conftest import assert_bitexact
from inferq_amd import moe as MOE
from inferq_amd import qgemm as Q
from inferq_amd import synth as S

pytestmark = pytest.mark.gpu

Q4, Q6 = S.Q4_K, S.Q6_K


@pytest.fixture(scope="module")
def small_qwen_layer():
    """Hidden 2048, intermediate 512 (the one-token kernels' shape), 16
    experts, shared expert."""
    return S.random_moe_layer(2048, 512, 16, Q4, Q6, np.random.default_rng(4040), shared=True)


def _fresh_moe(layer, gpu, top_k=4):
    t = {k: torch.from_numpy(v).to(gpu) for k, v in layer.items() if isinstance(v, np.ndarray)}
    return MOE.QuantizedMoeLayer(layer["hidden"], layer["inter"], layer["n_experts"], top_k, layer["gate_dtype"],
                                 layer["down_dtype"], t["gate"], t["up"], t["down"], t["shared_gate"],
                                 t["shared_up"], t["shared_down"], t["selector"]), t


def _eager(moe, xs, ls, m, gpu):
    res = []
    for x, lg in zip(xs, ls):
        o = torch.empty(m, 2048, device=gpu)
        moe.forward_into(x, lg, o)
        res.append(o.cpu().numpy())
    return res


def _replay_and_check(graph, bufs, xs, ls, expected, between, what):
    x_buf, l_buf, o_buf = bufs
    for rep in range(2):
        for i in range(len(xs)):
            x_buf.copy_(xs[i])
            l_buf.copy_(ls[i])
            graph.replay()
            torch.cuda.synchronize()
            assert_bitexact(o_buf.cpu().numpy(), expected[i], f"{what}: replay {rep}.{i}")
            between()
            torch.cuda.synchronize()


@pytest.mark.parametrize("m,reserve", [(1, 0), (8, 8), (40, 64)])
def test_moe_capture_without_eager_call(gpu, small_qwen_layer, m, reserve):
    """The captured handle has never run: one token needs nothing, wider
    calls an iq_moe_reserve first."""
    rng = np.random.default_rng(500 + m)
    xs = [torch.from_numpy(S.normal((m, 2048), rng)).to(gpu) for _ in range(2)]
    ls = [torch.from_numpy(S.normal((m, 16), rng)).to(gpu) for _ in range(2)]
    ref_moe, _ = _fresh_moe(small_qwen_layer, gpu)
    expected = _eager(ref_moe, xs, ls, m, gpu)
    moe, _ = _fresh_moe(small_qwen_layer, gpu)
    if reserve:
        moe.reserve(reserve)
    bufs = (torch.zeros(m, 2048, device=gpu), torch.zeros(m, 16, device=gpu), torch.empty(m, 2048, device=gpu))
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        moe.forward_into(*bufs)

    def between():
        o = torch.empty(m, 2048, device=gpu)
        ref_moe.forward_into(xs[0], ls[0], o)

    _replay_and_check(graph, bufs, xs, ls, expected, between, f"MoE m={m} captured without an eager call")


def test_moe_capture_of_unreserved_width_is_refused(gpu, small_qwen_layer):
    from inferq_amd import QgemmError

    moe, _ = _fresh_moe(small_qwen_layer, gpu)
    bufs = (torch.zeros(8, 2048, device=gpu), torch.zeros(8, 16, device=gpu), torch.empty(8, 2048, device=gpu))
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(QgemmError, match="iq_moe_reserve"):
        with torch.cuda.graph(graph, stream=stream):
            moe.forward_into(*bufs)
    torch.cuda.synchronize()


def test_moe_graph_survives_a_wider_eager_call(gpu, small_qwen_layer):
    """Capture at one token, then a 64-token eager call grows the handle's
    workspace; the graph (holding the old buffer) still replays correctly."""
    rng = np.random.default_rng(601)
    xs = [torch.from_numpy(S.normal((1, 2048), rng)).to(gpu) for _ in range(2)]
    ls = [torch.from_numpy(S.normal((1, 16), rng)).to(gpu) for _ in range(2)]
    moe, _ = _fresh_moe(small_qwen_layer, gpu)
    expected = _eager(moe, xs, ls, 1, gpu)
    bufs = (torch.zeros(1, 2048, device=gpu), torch.zeros(1, 16, device=gpu), torch.empty(1, 2048, device=gpu))
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        moe.forward_into(*bufs)
    wide_x = torch.from_numpy(S.normal((64, 2048), rng)).to(gpu)
    wide_l = torch.from_numpy(S.normal((64, 16), rng)).to(gpu)
    wide_o = torch.empty(64, 2048, device=gpu)
    moe.forward_into(wide_x, wide_l, wide_o)  # grows the workspace after the capture
    wide_ref = wide_o.cpu().numpy()

    def between():
        o = torch.empty(64, 2048, device=gpu)
        moe.forward_into(wide_x, wide_l, o)
        torch.cuda.synchronize()
        assert_bitexact(o.cpu().numpy(), wide_ref, "wide eager call between replays")

    _replay_and_check(graph, bufs, xs, ls, expected, between, "MoE graph after a wider eager call")


def _matrix(gpu, rng, dtype=Q4, rows=1024, cols=2048):
    w = S.random_matrix(dtype, rows, cols, rng)
    return Q.QuantizedMatrix.upload(w, dtype, rows, cols)


@pytest.mark.parametrize("m", [1, 8, 256])
def test_matmul_reserve_then_capture(gpu, m):
    """iq_matmul_reserve on a fresh stream, then a capture of the product
    (GEMV, lane MFMA and the split-K workspace paths) with no eager call."""
    rng = np.random.default_rng(700 + m)
    mat = _matrix(gpu, rng)
    xs = [torch.from_numpy(S.normal((m, 2048), rng)).to(gpu) for _ in range(2)]
    expected = [mat.forward(x).cpu().numpy() for x in xs]
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        mat.reserve(m)
    x_buf, y_buf = torch.zeros(m, 2048, device=gpu), torch.empty(m, 1024, device=gpu)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        mat.forward_into(x_buf, y_buf)
    for rep in range(2):
        for i, x in enumerate(xs):
            x_buf.copy_(x)
            graph.replay()
            torch.cuda.synchronize()
            assert_bitexact(y_buf.cpu().numpy(), expected[i], f"matmul m={m} replay {rep}.{i}")
            assert_bitexact(mat.forward(xs[1 - i]).cpu().numpy(), expected[1 - i], "eager between replays")


def test_matmul_graph_survives_growth_and_release(gpu):
    """A one-row graph on a stream, then a 256-row eager call on the same
    stream (the workspace grows); the graph still replays correctly.  Then
    the stream's workspace is released and an eager call allocates anew."""
    rng = np.random.default_rng(801)
    mat = _matrix(gpu, rng)
    x1 = torch.from_numpy(S.normal((1, 2048), rng)).to(gpu)
    x256 = torch.from_numpy(S.normal((256, 2048), rng)).to(gpu)
    e1, e256 = mat.forward(x1).cpu().numpy(), mat.forward(x256).cpu().numpy()
    stream = torch.cuda.Stream()
    x_buf, y_buf = x1.clone(), torch.empty(1, 1024, device=gpu)
    with torch.cuda.stream(stream):
        mat.reserve(1)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        mat.forward_into(x_buf, y_buf)
    with torch.cuda.stream(stream):
        y = torch.empty(256, 1024, device=gpu)
        mat.forward_into(x256, y)  # grows this stream's workspace
    torch.cuda.synchronize()
    assert_bitexact(y.cpu().numpy(), e256, "wide call after the capture")
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert_bitexact(y_buf.cpu().numpy(), e1, "one-row graph after the workspace grew")
    del graph
    with torch.cuda.stream(stream):
        Q.release_workspace()
        y = torch.empty(256, 1024, device=gpu)
        mat.forward_into(x256, y)
    torch.cuda.synchronize()
    assert_bitexact(y.cpu().numpy(), e256, "call after the workspace was released")
