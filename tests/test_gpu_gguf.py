"""GPU parity of the GGUF residency loader (warm_all_experts,
src/residency.rs:39-131) and of MoE layers assembled from a checkpoint
(QuantizedMoeLayer::load, src/qwen/quantized_moe.rs:141-225).

Bitwise: the resident expert bytes equal the file's bytes.  The layer
built from the file matches the oracle on the bytes the writer produced:
routes exactly, outputs within 1e-4 normwise (the router's f32 order, exp
and the selector dot are the unpinned orders; see test_gpu_moe_router.py).
"""
import ctypes
import os
import sys

import numpy as np
import pytest
import torch

from conftest import assert_bitexact, assert_close_normwise
from inferq_amd import gguf as G
from inferq_amd import synth as S

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import gguf_writer as W  # noqa: E402
import make_gguf  # noqa: E402

FIXTURE = os.path.join(HERE, "golden", "tiny_moe.gguf")


def _device_bytes(ptr, n):
    out = np.empty(n, np.uint8)
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    torch.cuda.synchronize()
    assert hip.hipMemcpy(out.ctypes.data, ptr, n, 2) == 0  # device to host
    return out


def _host_layer(lay, router, top_k):
    d = dict(lay)
    d.update(top_k=top_k, normalize=True, shared_gate_dtype=lay.get("shared_gate_dtype", lay["gate_dtype"]),
             shared_down_dtype=lay.get("shared_down_dtype", lay["down_dtype"]), router=router)
    return d


def _check_layer(oracle, ck, res, li, lay, router, top_k, ms, gpu):
    moe = ck.moe_layer(res, li, top_k)
    host = _host_layer(lay, router, top_k)
    for m in ms:
        x = S.normal((m, lay["hidden"]), np.random.default_rng(100 * li + m))
        out = moe.forward(torch.from_numpy(x).to(gpu))
        logits = oracle.router_logits(x, router, order=0)
        ref, ref_e, _ = oracle.moe_forward(host, x, logits, mode=1, impl=1 if oracle.have_avx2() else 0, nthreads=8)
        assert [r.experts for r in out.routes] == ref_e.tolist(), f"layer {li} m={m}"
        got = out.hidden.cpu().numpy()
        for r in range(m):
            assert_close_normwise(got[r], ref[r], 1e-4, f"layer {li} row {r} m={m}")


def test_resident_bytes_equal_the_file(gpu, tmp_path):
    _, layers = make_gguf.build(str(tmp_path / "t.gguf"))
    ck = G.GgufCheckpoint(FIXTURE)
    res = ck.warm_all_experts(2)
    expected = sum(ck.tensor_info(f"blk.{li}.ffn_{p}_exps.weight").storage_bytes for li in range(2)
                   for p in ("gate", "up", "down"))
    assert res.bytes() == expected
    for li, (lay, _) in enumerate(layers):
        ptr = res.tensor_pointers(li)
        for part, key in (("gate", "gate"), ("up", "up"), ("down", "down")):
            n = ptr["down_bytes"] if part == "down" else ptr["gate_bytes"]
            assert np.array_equal(_device_bytes(ptr[key], n), lay[part]), f"layer {li} {part}"
    mat = ck.load_matrix("blk.0.ffn_down_shexp.weight")
    assert mat.shape() == [256, 256] and mat.dtype() == "Q6K"
    with pytest.raises(G.QgemmError, match="expected a matrix"):
        ck.load_matrix("blk.0.ffn_gate_exps.weight")
    with pytest.raises(G.QgemmError, match="missing expert tensor"):
        ck.warm_all_experts(3)


def test_fixture_layers_match_the_oracle(gpu, oracle, tmp_path):
    _, layers = make_gguf.build(str(tmp_path / "t.gguf"))
    ck = G.GgufCheckpoint(FIXTURE)
    res = ck.warm_all_experts(2)
    for li, (lay, router) in enumerate(layers):
        _check_layer(oracle, ck, res, li, lay, router, 1, (1, 3), gpu)


def test_qwen_shaped_checkpoint(gpu, oracle, tmp_path):
    """Two layers of the config-2 shape with 16 experts (hidden 2048,
    intermediate 512, top-8): the token-major path at M = 1 and 8 and the
    grouped MFMA path at 40 tokens, on experts made resident from a file."""
    rng = np.random.default_rng(7)
    tensors, layers = [], []
    for li in range(2):
        lay = S.random_moe_layer(2048, 512, 16, S.Q4_K, S.Q6_K, rng, shared=True)
        router = rng.standard_normal((16, 2048), dtype=np.float32) / np.float32(np.sqrt(2048))
        layers.append((lay, router))
        tensors += W.moe_layer_tensors(li, lay, router)
    path = str(tmp_path / "qwen.gguf")
    W.write_gguf(path, tensors, {"general.architecture": "qwen3moe"})
    ck = G.GgufCheckpoint(path)
    res = ck.warm_all_experts(2)
    for li, (lay, router) in enumerate(layers):
        _check_layer(oracle, ck, res, li, lay, router, 8, (1, 8, 40), gpu)


def test_reference_mixed_format_checkpoint(gpu, oracle, tmp_path):
    """The file of the reference's MoE GGUF test (src/qwen/quantized_moe.rs:
    490-592): Q4_K gate/up and Q5_K down experts, a Q8_0 shared expert with
    a zero selector, a router favouring expert 1; hidden and intermediate
    256, two experts, top-1.  Loaded through the checkpoint, an input of
    ones routes to expert 1 with a finite output, three tokens equal three
    one-token calls bitwise, and random inputs match the oracle."""
    rng = np.random.default_rng(491)
    lay = S.random_moe_layer(256, 256, 2, S.Q4_K, S.Q5_K, rng, shared=False)
    lay.update({
        "shared_gate_dtype": S.Q8_0, "shared_down_dtype": S.Q8_0,
        "shared_gate": S.random_matrix(S.Q8_0, 256, 256, rng), "shared_up": S.random_matrix(S.Q8_0, 256, 256, rng),
        "shared_down": S.random_matrix(S.Q8_0, 256, 256, rng), "selector": np.zeros(256, np.float32),
    })
    router = np.concatenate([np.zeros(256, np.float32), np.full(256, 0.01, np.float32)]).reshape(2, 256)
    path = str(tmp_path / "moe.gguf")
    W.write_gguf(path, W.moe_layer_tensors(0, lay, router))
    ck = G.GgufCheckpoint(path)
    res = ck.warm_all_experts(1)
    moe = ck.moe_layer(res, 0, 1)
    out = moe.forward(torch.ones(1, 256, device=gpu))
    assert [r.experts for r in out.routes] == [[1]]
    assert np.isfinite(out.hidden.cpu().numpy()).all()
    batch = torch.ones(3, 256, device=gpu)
    singles = np.concatenate([moe.forward(batch[i:i + 1]).hidden.cpu().numpy() for i in range(3)])
    assert_bitexact(moe.forward(batch).hidden.cpu().numpy(), singles, "3 tokens vs one-token calls")
    _check_layer(oracle, ck, res, 0, lay, router, 1, (1, 3), gpu)
