"""GPU kernels against the committed fixtures (tests/golden/qgemm_golden.npz)
through the C ABI: products bit for bit at every fixture row count, the
per-block lane integers, both activation quantisers byte for byte, routes,
and the MoE sublayer (routes exact, output within the 1e-4 normwise f32
bar).  Reads no oracle code: the fixtures alone are the expectation.
"""
import os

import numpy as np
import pytest
import torch

from conftest import assert_bitexact, assert_close_normwise
from inferq_amd import moe as MOE
from inferq_amd import qgemm as Q
from inferq_amd import synth as S

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "qgemm_golden.npz")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


@pytest.mark.parametrize("dtype", [S.Q4_K, S.Q6_K, S.Q8_0])
def test_golden_products(gpu, golden, dtype):
    name = S.NAMES[dtype]
    n, k = (int(v) for v in golden[f"{name}_shape"])
    mat = Q.QuantizedMatrix.upload(golden[f"{name}_w"], dtype, n, k)
    x = torch.from_numpy(golden[f"{name}_x"]).to(gpu)
    for m in (1, 2, 4, 8, 9, 16):
        assert_bitexact(mat.forward(x[:m]).cpu().numpy(), golden[f"{name}_y_m{m}"], f"{name} m={m}")
    y, isum, msum = mat.block_sums(x[:1])
    assert np.array_equal(isum.cpu().numpy()[0], golden[f"{name}_isum_m1"])
    if dtype == S.Q4_K:
        assert np.array_equal(msum.cpu().numpy()[0], golden[f"{name}_msum_m1"])


def test_golden_quantisers(gpu, golden):
    x = torch.from_numpy(golden["quant_x"]).to(gpu)
    assert np.array_equal(Q.quantize_q8k(x).cpu().numpy().reshape(-1), golden["quant_q8k"].reshape(-1))
    assert np.array_equal(Q.quantize_q80(x).cpu().numpy().reshape(-1), golden["quant_q80"].reshape(-1))


def test_golden_moe(gpu, golden):
    t = {k: torch.from_numpy(golden[f"moe_{k}"]).to(gpu)
         for k in ("gate", "up", "down", "shared_gate", "shared_up", "shared_down", "selector")}
    layer = MOE.QuantizedMoeLayer(256, 256, 4, 2, S.Q4_K, S.Q6_K, t["gate"], t["up"], t["down"],
                                  t["shared_gate"], t["shared_up"], t["shared_down"], t["selector"])
    out = layer.forward(torch.from_numpy(golden["moe_x"]).to(gpu), torch.from_numpy(golden["moe_logits"]).to(gpu))
    assert [r.experts for r in out.routes] == golden["moe_experts"].tolist()
    assert_close_normwise(np.array([r.weights for r in out.routes]), golden["moe_weights"], 1e-6, "route weights")
    assert_close_normwise(out.hidden.cpu().numpy(), golden["moe_out"], 1e-4, "MoE output")


def test_golden_routes(gpu, golden):
    """The reference's router case (src/qwen/moe.rs:232-238) is row 0 of the
    route fixture: experts [1, 3] at top-2."""
    logits = golden["route_logits"]
    m, e = logits.shape
    rng = np.random.default_rng(5)
    layer = S.random_moe_layer(256, 256, e, S.Q4_K, S.Q6_K, rng, shared=False)
    t = {k: torch.from_numpy(layer[k]).to(gpu) for k in ("gate", "up", "down")}
    moe = MOE.QuantizedMoeLayer(256, 256, e, 2, S.Q4_K, S.Q6_K, t["gate"], t["up"], t["down"])
    out = moe.forward(torch.zeros(m, 256, device=gpu), torch.from_numpy(logits).to(gpu))
    assert [r.experts for r in out.routes] == golden["route_experts"].tolist()
    assert_close_normwise(np.array([r.weights for r in out.routes]), golden["route_weights"], 1e-6, "weights")
