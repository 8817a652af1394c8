"""GPU parity of the whole MoE sublayer from x: the router matmul on the GPU
(src/qwen/quantized_moe.rs:253), routing, experts, shared expert, and the
decoder layer's residual add (src/qwen/quantized_layer.rs:212), through
iq_moe_forward_x.

Tolerance: routes (experts) equal the oracle's exactly, where the oracle's
logits are the router product summed in double; the layer output within
1e-4 normwise of the oracle's layer on those logits.  The router's f32
summation order in the reference (a candle gemm) is not visible, so the
GPU's logits differ from any one order by rounding only -- far below the
gaps between ranked logits at these sizes.  The residual add is checked
bitwise: out = residual + MoE(x) exactly.
"""
import numpy as np
import pytest
import torch

from conftest import assert_bitexact, assert_close_normwise
from inferq_amd import moe as MOE
from inferq_amd import synth as S

pytestmark = pytest.mark.gpu

Q4, Q6 = S.Q4_K, S.Q6_K


@pytest.fixture(scope="module")
def routed_layer(gpu):
    """Config-2 shaped layer (256 experts, top-8, shared expert) with an f32
    router [256 x 2048] ~ N(0,1)/sqrt(2048), so logits are ~ N(0,1)."""
    rng = np.random.default_rng(4040)
    layer = S.random_moe_layer(2048, 512, 256, Q4, Q6, rng, shared=True)
    layer["router"] = (rng.standard_normal((256, 2048), dtype=np.float32) / np.float32(np.sqrt(2048)))
    t = {k: torch.from_numpy(v).to(gpu) for k, v in layer.items() if isinstance(v, np.ndarray)}
    moe = MOE.QuantizedMoeLayer(2048, 512, 256, 8, Q4, Q6, t["gate"], t["up"], t["down"], t["shared_gate"],
                                t["shared_up"], t["shared_down"], t["selector"], router=t["router"])
    host = dict(layer)
    host.update(top_k=8, normalize=True, shared_gate_dtype=Q4, shared_down_dtype=Q6)
    return moe, host, t


@pytest.mark.parametrize("m", [1, 8, 29, 256])
def test_router_layer_matches_oracle(gpu, oracle, routed_layer, m):
    """M = 1 (token-major), 8 (verify), 29 and 256 (grouped MFMA path)."""
    moe, host, _ = routed_layer
    rng = np.random.default_rng(50 + m)
    x = S.normal((m, 2048), rng)
    out = moe.forward(torch.from_numpy(x).to(gpu))
    logits = oracle.router_logits(x, host["router"], order=0)
    ref, ref_e, _ = oracle.moe_forward(host, x, logits, mode=1, impl=1 if oracle.have_avx2() else 0, nthreads=8)
    assert [r.experts for r in out.routes] == ref_e.tolist(), f"routes m={m}"
    got = out.hidden.cpu().numpy()
    for r in range(m):
        assert_close_normwise(got[r], ref[r], 1e-4, f"router layer row {r} m={m}")


@pytest.mark.parametrize("m", [1, 8, 256])
def test_residual_add_is_exact(gpu, routed_layer, m):
    moe, _, _ = routed_layer
    g = torch.Generator(device=gpu).manual_seed(m)
    x = torch.randn(m, 2048, device=gpu, generator=g)
    res = torch.randn(m, 2048, device=gpu, generator=g)
    plain = moe.forward(x).hidden
    fused = moe.forward(x, residual=res).hidden
    assert_bitexact(fused.cpu().numpy(), (res + plain).cpu().numpy(), f"residual m={m}")


def test_given_logits_equal_router_logits(gpu, routed_layer):
    """Logits passed in (iq_moe_forward) and logits from the router
    (iq_moe_forward_x) give the same layer when they are the same logits:
    the router's product is what the layer routes on."""
    moe, host, t = routed_layer
    x = torch.randn(4, 2048, device=gpu, generator=torch.Generator(device=gpu).manual_seed(9))
    # the GPU router's logits, by the same fixed order, recomputed on the host
    xs, r = x.cpu().numpy().astype(np.float64), host["router"].astype(np.float64)
    via_router = moe.forward(x)
    logits = torch.from_numpy((xs @ r.T).astype(np.float32)).to(gpu)
    via_logits = moe.forward(x, logits)
    assert [a.experts for a in via_router.routes] == [b.experts for b in via_logits.routes]
    assert_close_normwise(via_router.hidden.cpu().numpy(), via_logits.hidden.cpu().numpy(), 1e-4, "router vs given")


def test_router_is_required_for_forward_x(gpu):
    rng = np.random.default_rng(3)
    layer = S.random_moe_layer(256, 256, 4, Q4, Q6, rng, shared=False)
    t = {k: torch.from_numpy(v).to(gpu) for k, v in layer.items() if isinstance(v, np.ndarray)}
    moe = MOE.QuantizedMoeLayer(256, 256, 4, 2, Q4, Q6, t["gate"], t["up"], t["down"])
    with pytest.raises(MOE.QgemmError, match="has no router"):
        moe.forward(torch.zeros(1, 256, device=gpu))
