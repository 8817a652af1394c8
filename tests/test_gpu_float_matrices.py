"""GPU parity of unquantised (F32 and BF16) matrices.  The reference's
QuantizedMatrix accepts both dtypes (src/gguf.rs:305-317) and multiplies
them through candle's f32 matmul, having no multi-row kernel for them
(src/gguf.rs:533-535, :599); the router (ffn_gate_inp) and the shared
expert's gate vector are such tensors in the reference's GGUF files.

Checks: (1) bitwise against a host restatement of the library's stated
order (lane l sums x[k] * w[k], product then add, over k = l + 64 j in
turn, then the butterfly xor 32 .. 1), which pins every rounding; (2)
within 1e-5 normwise of the f64 product (the stated tolerance against the
reference, whose candle order is not visible here, is 1e-4); (3) every row
of a wide call bitwise equal to a one-row call; (4) the F32 router matrix
gives the MoE layer's own router logits: iq_moe_forward on them equals
iq_moe_forward_x bit for bit; (5) the reference's errors for paths and
hooks a float matrix has none of.
"""
import numpy as np
import pytest
import torch

from conftest import assert_bitexact, assert_close_normwise
from inferq_amd import moe as MOE
from inferq_amd import qgemm as Q
from inferq_amd import synth as S

pytestmark = pytest.mark.gpu


def to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even bf16 bits of f32 values (finite inputs)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def lane_order_product(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """The library's f32 order, restated with numpy float32 arithmetic
    (IEEE per operation, no fused multiply-add)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    m, k = x.shape
    n = w.shape[0]
    part = np.zeros((m, n, 64), np.float32)
    for j in range((k + 63) // 64):
        lo, hi = 64 * j, min(64 * j + 64, k)
        prod = (x[:, None, lo:hi] * w[None, :, lo:hi]).astype(np.float32)
        part[:, :, : hi - lo] = (part[:, :, : hi - lo] + prod).astype(np.float32)
    lanes = np.arange(64)
    for off in (32, 16, 8, 4, 2, 1):
        part = (part + part[:, :, lanes ^ off]).astype(np.float32)
    return part[:, :, 0]


def _matrix(gpu, dtype, rows, cols, seed):
    rng = np.random.default_rng(seed)
    wf = rng.standard_normal((rows, cols), dtype=np.float32) / np.float32(np.sqrt(cols))
    if dtype == Q.IQ_BF16:
        bits = to_bf16_bits(wf)
        wf = bf16_to_f32(bits)
        raw = bits.view(np.uint8)
    else:
        raw = wf.view(np.uint8)
    mat = Q.QuantizedMatrix.upload(raw.reshape(-1), dtype, rows, cols)
    return mat, wf


@pytest.mark.parametrize("dtype", [Q.IQ_F32, Q.IQ_BF16])
@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 5), (64, 511), (256, 2048), (37, 4096), (2048, 64)])
def test_float_matrix_product(gpu, dtype, rows, cols):
    mat, wf = _matrix(gpu, dtype, rows, cols, rows * 131 + cols)
    assert mat.dtype() == ("F32" if dtype == Q.IQ_F32 else "BF16")
    assert mat.storage_bytes() == rows * cols * (4 if dtype == Q.IQ_F32 else 2)
    m = 11
    x = np.random.default_rng(cols).standard_normal((m, cols), dtype=np.float32)
    got = mat.forward(torch.from_numpy(x).to(gpu)).cpu().numpy()
    assert_bitexact(got, lane_order_product(x, wf), f"{mat.dtype()} [{rows} x {cols}] lane order")
    ref = x.astype(np.float64) @ wf.astype(np.float64).T
    for r in range(m):
        assert_close_normwise(got[r], ref[r], 1e-5, f"{mat.dtype()} [{rows} x {cols}] row {r} vs f64")
    single = np.stack([mat.forward(torch.from_numpy(x[r:r + 1]).to(gpu)).cpu().numpy()[0] for r in range(m)])
    assert_bitexact(got, single, f"{mat.dtype()} [{rows} x {cols}] wide call vs one-row calls")


@pytest.mark.parametrize("m", [1, 8, 9, 64, 300])
def test_float_matrix_row_counts(gpu, m):
    """Tiles of 8 input rows per grid row: ragged last tiles, many tiles."""
    mat, wf = _matrix(gpu, Q.IQ_F32, 512, 2048, 77)
    x = np.random.default_rng(m).standard_normal((m, 2048), dtype=np.float32)
    got = mat.forward(torch.from_numpy(x).to(gpu)).cpu().numpy()
    assert_bitexact(got, lane_order_product(x, wf), f"F32 [512 x 2048] m={m}")


def test_f32_router_matrix_gives_the_layers_logits(gpu):
    """The router as a matrix (QuantizedMatrix F32, as the reference holds
    it) and the MoE layer's own router (iq_moe_forward_x) form the same
    logits: the layer routed on them gives the same bits."""
    rng = np.random.default_rng(4041)
    layer = S.random_moe_layer(2048, 512, 256, S.Q4_K, S.Q6_K, rng, shared=True)
    router = rng.standard_normal((256, 2048), dtype=np.float32) / np.float32(np.sqrt(2048))
    t = {k: torch.from_numpy(v).to(gpu) for k, v in layer.items() if isinstance(v, np.ndarray)}
    tr = torch.from_numpy(router).to(gpu)
    moe = MOE.QuantizedMoeLayer(2048, 512, 256, 8, S.Q4_K, S.Q6_K, t["gate"], t["up"], t["down"], t["shared_gate"],
                                t["shared_up"], t["shared_down"], t["selector"], router=tr)
    rmat = Q.QuantizedMatrix.view(tr.view(torch.uint8).reshape(-1), Q.IQ_F32, 256, 2048)
    for m in (1, 8, 40):
        x = torch.randn(m, 2048, device=gpu, generator=torch.Generator(device=gpu).manual_seed(m))
        logits = rmat.forward(x)
        a, b = moe.forward(x), moe.forward(x, logits)
        assert [r.experts for r in a.routes] == [r.experts for r in b.routes], f"routes m={m}"
        assert_bitexact(a.hidden.cpu().numpy(), b.hidden.cpu().numpy(), f"router matrix vs layer router m={m}")


def test_float_matrix_paths_and_hooks(gpu):
    """No fixed kernel paths and no per-block integers (the reference's
    multi-row paths fail for these dtypes too); the dispatch, the caller's
    workspace, the allocation-free entry, argmax, row concatenation and
    leading rows all work on them."""
    mat, wf = _matrix(gpu, Q.IQ_BF16, 300, 1024, 5)
    x = torch.randn(2, 1024, device=gpu, generator=torch.Generator(device=gpu).manual_seed(2))
    for path in (Q._lib.PATH_LANES, Q._lib.PATH_GEMV, Q._lib.PATH_LANE_MFMA, Q._lib.PATH_PREFILL_TILES):
        with pytest.raises(Q.QgemmError, match="BF16 has no"):
            mat.forward_via(x, path)
    with pytest.raises(Q.QgemmError, match="BF16 has no"):
        mat.block_sums(x)
    want = mat.forward(x).cpu().numpy()
    y = torch.empty(2, 300, device=gpu)
    Q.check(Q.lib().iq_matmul_noalloc(mat.handle, x.data_ptr(), 2, y.data_ptr(), Q._stream()))
    assert_bitexact(y.cpu().numpy(), want, "noalloc")
    idx, val = mat.forward_argmax(x)
    assert idx.cpu().tolist() == [int(np.flatnonzero(r == r.max())[-1]) for r in want]
    both = mat.concatenate_rows(mat)
    assert_bitexact(both.forward(x).cpu().numpy(), np.concatenate([want, want], axis=1), "concatenate_rows")
    head = mat.leading_rows(7)
    assert_bitexact(head.forward(x).cpu().numpy(), want[:, :7], "leading_rows")


def test_gguf_f32_tensor_loads_as_a_matrix(gpu):
    """GgufCheckpoint::load_matrix on an F32 tensor (src/gguf.rs:1234 with
    QuantizedMatrix::new's dtype set): the committed fixture's router
    (blk.0.ffn_gate_inp.weight, [experts x hidden]) as a matrix gives the
    lane-order product of the file's values."""
    import os

    from inferq_amd import gguf as G

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny_moe.gguf")
    with G.GgufCheckpoint.open(path) as ck:
        name = "blk.0.ffn_gate_inp.weight"
        mat = ck.load_matrix(name)
        w = ck.load_f32(name).cpu().numpy()
    assert mat.dtype() == "F32" and mat.shape() == list(w.shape)
    x = np.random.default_rng(8).standard_normal((3, w.shape[1]), dtype=np.float32)
    got = mat.forward(torch.from_numpy(x).to(gpu)).cpu().numpy()
    assert_bitexact(got, lane_order_product(x, w), "GGUF F32 router matrix")
