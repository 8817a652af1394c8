"""GPU parity of the whole 40-layer decode step as one
HIP graph, through the C ABI.

The model follows the layer mix of the 40-layer Qwen3.6-35B-A3B shape
(src/config.rs:235-246): layers l with (l + 1) % 4 == 0 are full attention
(q/gate [8192 x 2048], k and v [512 x 2048], o [2048 x 4096],
src/qwen/quantized_attention.rs:428-442, 503), the other 30 DeltaNet (qkvz
[12288 x 2048], ba [64 x 2048], out [2048 x 4096],
src/qwen/quantized_deltanet.rs:419-434, 537-563, 699), all Q4_K, each
followed by its MoE layer (256 experts of [512 x 2048] Q4_K gate/up and
[2048 x 512] Q6_K down, top-8 plus the shared expert: about 21 GB resident),
then the LM head [248320 x 2048] Q6_K.  The hidden state runs through the
step: each layer's projections read it, its MoE layer reads it, and the MoE
output is added to it (the residual, src/qwen/quantized_layer.rs:212),
scaled to half the RMS of the hidden state: the synthetic layers have no
normalisation and their MoE outputs grow with the square of their inputs,
so an unscaled residual overflows within a few layers.  The scales are
taken from the eager pass that precedes the capture, which computes the
same values as the replay (same inputs, deterministic kernels).  o and out
read a fresh N(0,1) row in place of the attention or DeltaNet core, which
is outside this path.

Every call of the step (83 launches at M = 1) is captured once in a HIP
graph on one stream and replayed; then each stage is checked against the
oracle on the GPU's own input to that stage: the dense products and the LM
head bitwise, the MoE layers with routes equal and outputs within 1e-4
normwise (exp and the shared expert's selector dot are the two unpinned
orders).  This checks what the two-layer test cannot: 80-odd products in
one graph sharing the stream's workspace and the layers' workspaces.
"""
import os

import numpy as np
import pytest
import torch

from conftest import assert_bitexact, assert_close_normwise
from inferq_amd import moe as M
from inferq_amd import qgemm as Q
from inferq_amd import synth as S

pytestmark = pytest.mark.gpu

Q4, Q6 = S.Q4_K, S.Q6_K
H, I, E, TOPK = 2048, 512, 256, 8
NL = 40
ATTN = (("q_gate", 8192, 2048), ("k", 512, 2048), ("v", 512, 2048), ("o", 2048, 4096))
DELTA = (("qkvz", 12288, 2048), ("ba", 64, 2048), ("out", 2048, 4096))


def _threads():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def _moe_tensors(gpu, seed):
    t = {
        "gate": S.random_matrix_device(Q4, E * I, H, gpu, seed + 1),
        "up": S.random_matrix_device(Q4, E * I, H, gpu, seed + 2),
        "down": S.random_matrix_device(Q6, E * H, I, gpu, seed + 3),
        "shared_gate": S.random_matrix_device(Q4, I, H, gpu, seed + 4),
        "shared_up": S.random_matrix_device(Q4, I, H, gpu, seed + 5),
        "shared_down": S.random_matrix_device(Q6, H, I, gpu, seed + 6),
    }
    g = torch.Generator(device=gpu)
    g.manual_seed(seed + 7)
    t["selector"] = torch.randn(H, device=gpu, generator=g) / float(np.sqrt(H))
    return t


def _host_layer(t):
    host = {k: v.cpu().numpy() for k, v in t.items()}
    host.update(hidden=H, inter=I, n_experts=E, top_k=TOPK, normalize=True, gate_dtype=Q4, down_dtype=Q6,
                shared_gate_dtype=Q4, shared_down_dtype=Q6)
    return host


class _Model:
    def __init__(self, gpu):
        self.is_attn = [(li + 1) % 4 == 0 for li in range(NL)]
        self.dense, self.moe_t, self.moe = [], [], []
        for li in range(NL):
            shapes = ATTN if self.is_attn[li] else DELTA
            mats = []
            for j, (name, r, c) in enumerate(shapes):
                t = S.random_matrix_device(Q4, r, c, gpu, 20000 + 10 * li + j)
                mats.append((name, Q.QuantizedMatrix.view(t, Q4, r, c), t))
            self.dense.append(mats)
            t = _moe_tensors(gpu, 30000 + 10 * li)
            self.moe_t.append(t)
            self.moe.append(M.QuantizedMoeLayer(H, I, E, TOPK, Q4, Q6, t["gate"], t["up"], t["down"],
                                                t["shared_gate"], t["shared_up"], t["shared_down"], t["selector"]))
        self.lm_t = S.random_matrix_device(Q6, 248320, H, gpu, 29999)
        self.lm = Q.QuantizedMatrix.view(self.lm_t, Q6, 248320, H)


class _Step:
    """Buffers and the captured graph of one decode step at m rows."""

    def __init__(self, model, m, gpu, seed):
        g = torch.Generator(device=gpu)
        g.manual_seed(seed)
        self.m = m
        self.hid = [torch.empty(m, H, device=gpu) for _ in range(NL + 1)]
        self.hid[0].copy_(torch.randn(m, H, device=gpu, generator=g))
        self.core = [torch.randn(m, 4096, device=gpu, generator=g) for _ in range(NL)]
        self.logits = [torch.randn(m, E, device=gpu, generator=g) for _ in range(NL)]
        self.ys = [[torch.empty(m, r, device=gpu) for _, r, _ in (ATTN if model.is_attn[li] else DELTA)]
                   for li in range(NL)]
        self.moe_out = [torch.empty(m, H, device=gpu) for _ in range(NL)]
        self.experts = [torch.empty(m, TOPK, dtype=torch.int32, device=gpu) for _ in range(NL)]
        self.ylm = torch.empty(m, 248320, device=gpu)
        self.alpha = [None] * NL
        self.model = model

    def run(self):
        """The step's launches in order; the first (eager) call also fixes
        the residual scales."""
        md = self.model
        for li in range(NL):
            for (name, mat, _), y in zip(md.dense[li], self.ys[li]):
                mat.forward_into(self.core[li] if mat.shape()[1] == 4096 else self.hid[li], y)
            md.moe[li].forward_into(self.hid[li], self.logits[li], self.moe_out[li], experts=self.experts[li])
            if self.alpha[li] is None:
                rms = lambda t: float(t.double().pow(2).mean().sqrt())
                self.alpha[li] = 0.5 * rms(self.hid[li]) / max(rms(self.moe_out[li]), 1e-30)
            torch.add(self.hid[li], self.moe_out[li], alpha=self.alpha[li], out=self.hid[li + 1])
        md.lm.forward_into(self.hid[NL], self.ylm)


@pytest.fixture(scope="module")
def model(gpu):
    md = _Model(gpu)
    yield md
    del md
    torch.cuda.empty_cache()


def test_forty_layer_step_in_one_graph(gpu, oracle, model):
    impl = 1 if oracle.have_avx2() else 0
    nt = _threads()
    stream = torch.cuda.Stream()
    steps = []
    for m, seed in ((1, 41), (8, 48)):
        st = _Step(model, m, gpu, seed)
        # the inputs were drawn on the default stream; the eager pass, which
        # fixes the residual scales, must read them complete
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            st.run()  # sizes the stream's and the layers' workspaces outside the capture
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            st.run()
        for buf in st.ys[0] + [st.moe_out[0], st.ylm] + st.hid[1:]:
            buf.fill_(float("nan"))  # every output the replay must write
        st.experts[0].fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"step m={m}: graph replayed", flush=True)
        steps.append((st, graph))

    for li in range(NL):
        mats = model.dense[li]
        host_w = [(name, mat.shape(), t.cpu().numpy()) for name, mat, t in mats]
        host_moe = _host_layer(model.moe_t[li])
        for st, _ in steps:
            m = st.m
            h = st.hid[li].cpu().numpy()
            for (name, (r, c), w), y in zip(host_w, st.ys[li]):
                x = st.core[li].cpu().numpy() if c == 4096 else h
                expected = oracle.matmul(Q4, w, r, c, x, impl=impl, nthreads=nt)
                assert_bitexact(y.cpu().numpy(), expected, f"layer {li} {name} m={m}")
            logits = st.logits[li].cpu().numpy()
            ref, experts, _ = oracle.moe_forward(host_moe, h, logits, mode=0, impl=impl, nthreads=nt)
            assert st.experts[li].cpu().numpy().tolist() == experts.tolist(), f"layer {li} routes m={m}"
            got = st.moe_out[li].cpu().numpy()
            for r in range(m):
                assert_close_normwise(got[r], ref[r], 1e-4, f"layer {li} MoE row {r} m={m}")
            assert np.isfinite(got).all(), f"layer {li} MoE m={m}"
            assert_close_normwise(st.hid[li + 1].cpu().numpy(), h + st.alpha[li] * got.astype(np.float64), 1e-6,
                                  f"layer {li} residual m={m}")
        del host_w, host_moe
    lm_w = model.lm_t.cpu().numpy()
    for st, _ in steps:
        x = st.hid[NL].cpu().numpy()
        expected = oracle.matmul(Q6, lm_w, 248320, H, x, impl=impl, nthreads=nt)
        assert_bitexact(st.ylm.cpu().numpy(), expected, f"LM head m={st.m}")
