"""ctypes binding of the parity oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU baseline,
never by the product package.  See iq_oracle.h for what each function restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14

Q4K_BLOCK = np.dtype([("d", "<u2"), ("dmin", "<u2"), ("scales", "u1", 12), ("qs", "u1", 128)])
Q5K_BLOCK = np.dtype([("d", "<u2"), ("dmin", "<u2"), ("scales", "u1", 12), ("qh", "u1", 32), ("qs", "u1", 128)])
Q6K_BLOCK = np.dtype([("ql", "u1", 128), ("qh", "u1", 64), ("scales", "i1", 16), ("d", "<u2")])
Q80_BLOCK = np.dtype([("d", "<u2"), ("qs", "i1", 32)])
Q8K_BLOCK = np.dtype([("d", "<f4"), ("qs", "i1", 256), ("bsums", "<i2", 16)])
assert (Q4K_BLOCK.itemsize, Q5K_BLOCK.itemsize, Q6K_BLOCK.itemsize, Q80_BLOCK.itemsize,
        Q8K_BLOCK.itemsize) == (144, 176, 210, 34, 292)

BLOCK = {Q4_K: Q4K_BLOCK, Q5_K: Q5K_BLOCK, Q6_K: Q6K_BLOCK, Q8_0: Q80_BLOCK}
BLOCK_ELEMS = {Q4_K: 256, Q5_K: 256, Q6_K: 256, Q8_0: 32}

_lib = None


def build() -> None:
    """Compile liboracle.so from the C sources beside this file."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L: ctypes.CDLL) -> None:
    P, S, I, F = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_float
    L.or_f16_to_f32.argtypes, L.or_f16_to_f32.restype = [ctypes.c_uint16], F
    L.or_f32_to_f16.argtypes, L.or_f32_to_f16.restype = [F], ctypes.c_uint16
    for name in ("or_quantize_q8k", "or_quantize_q80"):
        getattr(L, name).argtypes, getattr(L, name).restype = [P, S, P], I
    L.or_router_logits.argtypes, L.or_router_logits.restype = [P, S, S, P, S, P, I], None
    L.or_q4k_block_lanes.argtypes = [P, P, P, P]
    L.or_q5k_block_lanes.argtypes = [P, P, P, P]
    L.or_q5k_block_textbook.argtypes = [P, P, P, P]
    L.or_q6k_block_lanes.argtypes = [P, P, P]
    L.or_q80_block_lanes.argtypes = [P, P, P]
    L.or_q4k_block_textbook.argtypes = [P, P, P, P]
    L.or_q6k_block_textbook.argtypes = [P, P, P]
    L.or_q80_block_textbook.argtypes = [P, P, P]
    for name in ("or_q4k_q8k_row_lanes", "or_q5k_q8k_row_lanes", "or_q6k_q8k_row_lanes", "or_q80_q80_row_lanes"):
        getattr(L, name).argtypes, getattr(L, name).restype = [P, S, P, S, P], None
    for name in ("or_q4k_q8k_row_avx2", "or_q6k_q8k_row_avx2", "or_q80_q80_row_avx2"):
        getattr(L, name).argtypes, getattr(L, name).restype = [P, S, P, S, P], I
    L.or_have_avx2.argtypes, L.or_have_avx2.restype = [], I
    L.or_pool_pin.argtypes, L.or_pool_pin.restype = [P, I], None
    L.or_dequantize.argtypes, L.or_dequantize.restype = [I, P, S, S, P], I
    for name in ("or_matmul", "or_matmul_tiled"):
        getattr(L, name).argtypes, getattr(L, name).restype = [I, P, S, S, P, S, P, I, I], I
    L.or_top_k_routes.argtypes, L.or_top_k_routes.restype = [P, S, S, S, I, P, P], I
    L.or_moe_forward.argtypes, L.or_moe_forward.restype = [P, P, P, S, P, P, P, I, I, I], I
    L.or_silu_mul.argtypes, L.or_silu_mul.restype = [F, F], F
    L.or_sigmoid.argtypes, L.or_sigmoid.restype = [F], F


def _p(a: np.ndarray) -> int:
    assert a.flags.c_contiguous
    return a.ctypes.data


def pool_pin(cpus) -> None:
    """Pin the oracle's row-spread pool: worker t >= 1 on cpus[t % len]."""
    arr = np.ascontiguousarray(cpus, dtype=np.int32)
    lib().or_pool_pin(_p(arr) if arr.size else None, int(arr.size))


def have_avx2() -> bool:
    return bool(lib().or_have_avx2())


def f16_to_f32(h: int) -> float:
    return lib().or_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return lib().or_f32_to_f16(f)


def quantize_q8k(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 256, dtype=Q8K_BLOCK)
    if lib().or_quantize_q8k(_p(x), x.size, _p(out)):
        raise ValueError("Q8K quantisation needs a multiple of 256 values")
    return out


def quantize_q80(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 32, dtype=Q80_BLOCK)
    if lib().or_quantize_q80(_p(x), x.size, _p(out)):
        raise ValueError("Q8_0 quantisation needs a multiple of 32 values")
    return out


def block_lanes(dtype: int, wblock: np.ndarray, xblock: np.ndarray):
    """Per-block lane integers (isum[8], msum[4] for Q4_K and Q5_K)."""
    isum = np.zeros(8, np.int32)
    msum = np.zeros(4, np.int32)
    w = np.ascontiguousarray(wblock)
    x = np.ascontiguousarray(xblock)
    if dtype in (Q4_K, Q5_K):
        fn = lib().or_q4k_block_lanes if dtype == Q4_K else lib().or_q5k_block_lanes
        fn(_p(w), _p(x), _p(isum), _p(msum))
        return isum, msum
    if dtype == Q6_K:
        lib().or_q6k_block_lanes(_p(w), _p(x), _p(isum))
    else:
        lib().or_q80_block_lanes(_p(w), _p(x), _p(isum))
    return isum, None


def block_textbook(dtype: int, wblock: np.ndarray, xblock: np.ndarray):
    isum = np.zeros(1, np.int64)
    msum = np.zeros(1, np.int64)
    w = np.ascontiguousarray(wblock)
    x = np.ascontiguousarray(xblock)
    if dtype in (Q4_K, Q5_K):
        fn = lib().or_q4k_block_textbook if dtype == Q4_K else lib().or_q5k_block_textbook
        fn(_p(w), _p(x), _p(isum), _p(msum))
        return int(isum[0]), int(msum[0])
    if dtype == Q6_K:
        lib().or_q6k_block_textbook(_p(w), _p(x), _p(isum))
    else:
        lib().or_q80_block_textbook(_p(w), _p(x), _p(isum))
    return int(isum[0]), None


def row_kernel(dtype: int, wrow: np.ndarray, inputs_block_major: np.ndarray, rows: int, impl: str = "lanes"):
    """One weight row against `rows` block-major inputs (q*_row entry)."""
    out = np.zeros(rows, np.float32)
    w = np.ascontiguousarray(wrow)
    x = np.ascontiguousarray(inputs_block_major)
    name = {Q4_K: "q4k_q8k", Q5_K: "q5k_q8k", Q6_K: "q6k_q8k", Q8_0: "q80_q80"}[dtype]
    fn = getattr(lib(), f"or_{name}_row_{impl}")
    rc = fn(_p(w), w.size, _p(x), rows, _p(out))
    if impl == "avx2" and rc:
        raise RuntimeError("oracle built without AVX2")
    return out


def dequantize(dtype: int, wbytes: np.ndarray, rows: int, cols: int) -> np.ndarray:
    out = np.zeros((rows, cols), np.float32)
    w = np.ascontiguousarray(wbytes)
    if lib().or_dequantize(dtype, _p(w), rows, cols, _p(out)):
        raise ValueError("bad dtype or width")
    return out


def matmul(dtype: int, wbytes: np.ndarray, rows: int, cols: int, x: np.ndarray, impl: int = 0,
           nthreads: int = 1, tiled: bool = False) -> np.ndarray:
    """fused_forward: y[m x rows] for x[m x cols] (impl 0 lanes, 1 AVX2)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, cols)
    m = x.shape[0]
    y = np.zeros((m, rows), np.float32)
    w = np.ascontiguousarray(wbytes)
    fn = lib().or_matmul_tiled if tiled else lib().or_matmul
    rc = fn(dtype, _p(w), rows, cols, _p(x), m, _p(y), impl, nthreads)
    if rc:
        raise RuntimeError(f"or_matmul failed ({rc})")
    return y


def top_k_routes(logits: np.ndarray, k: int, normalize: bool = True):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    m, e = logits.shape
    experts = np.zeros((m, k), np.int32)
    weights = np.zeros((m, k), np.float32)
    if lib().or_top_k_routes(_p(logits), m, e, k, int(normalize), _p(experts), _p(weights)):
        raise ValueError(f"invalid router top-k {k} for {e} experts")
    return experts, weights


class _MoeLayer(ctypes.Structure):
    _fields_ = [
        ("hidden", ctypes.c_size_t), ("inter", ctypes.c_size_t), ("n_experts", ctypes.c_size_t),
        ("top_k", ctypes.c_size_t), ("normalize", ctypes.c_int),
        ("gate_dtype", ctypes.c_int), ("down_dtype", ctypes.c_int),
        ("shared_gate_dtype", ctypes.c_int), ("shared_down_dtype", ctypes.c_int),
        ("gate", ctypes.c_void_p), ("up", ctypes.c_void_p), ("down", ctypes.c_void_p),
        ("shared_gate", ctypes.c_void_p), ("shared_up", ctypes.c_void_p), ("shared_down", ctypes.c_void_p),
        ("selector", ctypes.c_void_p),
    ]


def moe_forward(layer: dict, x: np.ndarray, logits: np.ndarray, mode: int = 0, impl: int = 0, nthreads: int = 1):
    """QuantizedMoeLayer::forward.  `layer` holds numpy byte arrays and shapes:
    hidden, inter, n_experts, top_k, normalize, gate_dtype, down_dtype,
    gate, up, down, and optionally shared_gate/shared_up/shared_down/selector
    with shared_gate_dtype/shared_down_dtype."""
    H = layer["hidden"]
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, H)
    logits = np.ascontiguousarray(logits, dtype=np.float32).reshape(x.shape[0], -1)
    m = x.shape[0]
    k = layer["top_k"]
    keep = {name: np.ascontiguousarray(layer[name]) for name in
            ("gate", "up", "down", "shared_gate", "shared_up", "shared_down", "selector") if layer.get(name) is not None}
    if "selector" in keep:
        keep["selector"] = np.ascontiguousarray(keep["selector"], dtype=np.float32)
    desc = _MoeLayer(
        H, layer["inter"], layer["n_experts"], k, int(layer.get("normalize", True)),
        layer["gate_dtype"], layer["down_dtype"],
        layer.get("shared_gate_dtype", layer["gate_dtype"]), layer.get("shared_down_dtype", layer["down_dtype"]),
        *(keep[n].ctypes.data if n in keep else None
          for n in ("gate", "up", "down", "shared_gate", "shared_up", "shared_down", "selector")),
    )
    out = np.zeros((m, H), np.float32)
    experts = np.zeros((m, k), np.int32)
    weights = np.zeros((m, k), np.float32)
    rc = lib().or_moe_forward(ctypes.byref(desc), _p(x), _p(logits), m, _p(out), _p(experts), _p(weights),
                              mode, impl, nthreads)
    if rc:
        raise RuntimeError(f"or_moe_forward failed ({rc})")
    return out, experts, weights


def router_logits(x: np.ndarray, router: np.ndarray, order: int = 0) -> np.ndarray:
    """or_router_logits: x [m x h] . router [e x h]^T (order 0: double, 1:
    sequential f32)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    router = np.ascontiguousarray(router, dtype=np.float32)
    h = router.shape[-1]
    x = x.reshape(-1, h)
    e = router.size // h
    out = np.zeros((x.shape[0], e), np.float32)
    lib().or_router_logits(_p(x), x.shape[0], h, _p(router), e, _p(out), order)
    return out


def silu_mul(g: float, u: float) -> float:
    return lib().or_silu_mul(g, u)


def sigmoid(v: float) -> float:
    return lib().or_sigmoid(v)
