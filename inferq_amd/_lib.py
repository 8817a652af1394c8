"""ctypes binding of libiq_qgemm.so (the C ABI in include/iq_qgemm.h).

There is no fallback: if the library is missing or fails to load, every
entry point raises.  Build it with `python -m inferq_amd._build`.
"""
from __future__ import annotations

import ctypes
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libiq_qgemm.so")

IQ_Q8_0, IQ_Q4_K, IQ_Q5_K, IQ_Q6_K = 8, 12, 13, 14
IQ_F32, IQ_BF16 = 0, 30  # unquantised matrices (the reference's F32 / BF16 QuantizedMatrix)
# enum iq_path (the reference's MultiRowPath, src/gguf.rs:43-62)
PATH_AUTO, PATH_LANES, PATH_GEMV, PATH_LANE_MFMA, PATH_PREFILL_TILES = 0, 1, 2, 3, 4
IQ_OK = 0
IQ_ERR_INVALID, IQ_ERR_SHAPE, IQ_ERR_DTYPE, IQ_ERR_OOM, IQ_ERR_HIP, IQ_ERR_RANGE = -1, -2, -3, -4, -5, -6
STATUS_NAMES = {
    IQ_ERR_INVALID: "IQ_ERR_INVALID", IQ_ERR_SHAPE: "IQ_ERR_SHAPE", IQ_ERR_DTYPE: "IQ_ERR_DTYPE",
    IQ_ERR_OOM: "IQ_ERR_OOM", IQ_ERR_HIP: "IQ_ERR_HIP", IQ_ERR_RANGE: "IQ_ERR_RANGE",
}


class QgemmError(RuntimeError):
    """A C-ABI call returned an error status; `status` holds the code."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{message} [{STATUS_NAMES.get(status, status)}]")
        self.status = status


_lib = None

P, I64, SZ, INT = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t, ctypes.c_int
_SIGNATURES = {
    "iq_version": ([], ctypes.c_char_p),
    "iq_last_error": ([], ctypes.c_char_p),
    "iq_init": ([INT], INT),
    "iq_weights_upload": ([P, SZ, INT, I64, I64, ctypes.POINTER(P)], INT),
    "iq_weights_view": ([P, SZ, INT, I64, I64, ctypes.POINTER(P)], INT),
    "iq_weights_free": ([P], INT),
    "iq_weights_info": ([P, ctypes.POINTER(INT), ctypes.POINTER(I64), ctypes.POINTER(I64), ctypes.POINTER(SZ),
                         ctypes.POINTER(P)], INT),
    "iq_weights_concat_rows": ([P, P, ctypes.POINTER(P)], INT),
    "iq_weights_leading_rows": ([P, I64, ctypes.POINTER(P)], INT),
    "iq_matmul": ([P, P, I64, P, P], INT),
    "iq_matmul_via": ([P, P, I64, P, INT, P], INT),
    "iq_matmul_noalloc": ([P, P, I64, P, P], INT),
    "iq_matmul_noalloc_max_bytes": ([], SZ),
    "iq_matmul_workspace_size": ([P, I64], SZ),
    "iq_matmul_reserve": ([P, I64, P], INT),
    "iq_workspace_release": ([P], INT),
    "iq_matmul_ws": ([P, P, I64, P, P, SZ, P], INT),
    "iq_matmul_host": ([P, P, I64, P], INT),
    "iq_argmax_rows": ([P, I64, I64, P, P, P], INT),
    "iq_q4k_q8k_row": ([P, SZ, P, SZ, SZ, P, SZ], INT),
    "iq_q6k_q8k_row": ([P, SZ, P, SZ, SZ, P, SZ], INT),
    "iq_q80_q80_row": ([P, SZ, P, SZ, SZ, P, SZ], INT),
    "iq_matmul_argmax": ([P, P, I64, P, P, P], INT),
    "iq_quantize_q8k": ([P, I64, I64, P, P], INT),
    "iq_quantize_q80": ([P, I64, I64, P, P], INT),
    "iq_block_sums": ([P, P, I64, P, P, P, P], INT),
    "iq_prefill_block_sums": ([P, P, I64, P, P, P, P], INT),
    "iq_gguf_open": ([ctypes.c_char_p, ctypes.POINTER(P)], INT),
    "iq_gguf_close": ([P], INT),
    "iq_gguf_tensor_count": ([P], I64),
    "iq_gguf_tensor_name": ([P, I64], ctypes.c_char_p),
    "iq_gguf_tensor_info": ([P, ctypes.c_char_p, ctypes.POINTER(INT), ctypes.POINTER(INT),
                             ctypes.POINTER(I64), ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)],
                            INT),
    "iq_gguf_meta_int": ([P, ctypes.c_char_p, ctypes.POINTER(I64)], INT),
    "iq_gguf_meta_str": ([P, ctypes.c_char_p], ctypes.c_char_p),
    "iq_gguf_load_matrix": ([P, ctypes.c_char_p, ctypes.POINTER(P)], INT),
    "iq_gguf_upload_tensor": ([P, ctypes.c_char_p, P, SZ, P], INT),
    "iq_gguf_load_experts": ([P, I64, ctypes.POINTER(P)], INT),
    "iq_experts_free": ([P], INT),
    "iq_experts_bytes": ([P], SZ),
    "iq_experts_layer": ([P, I64, P], INT),
    "iq_moe_create": ([P, ctypes.POINTER(P)], INT),
    "iq_moe_destroy": ([P], INT),
    "iq_moe_reserve": ([P, I64, P], INT),
    "iq_moe_slice_tokens": ([P], I64),
    "iq_moe_set_path": ([P, INT], INT),
    "iq_moe_forward": ([P, P, P, I64, P, P, P, P], INT),
    "iq_moe_forward_x": ([P, P, I64, P, P, P, P, P], INT),
    "iq_moe_forward_timed": ([P, P, P, I64, P, P, P, ctypes.POINTER(P), P], INT),
    "iq_moe_forward_stage": ([P, INT, P], INT),
}


class MoeDesc(ctypes.Structure):
    """iq_moe_desc (include/iq_qgemm.h)."""

    _fields_ = [
        ("hidden", ctypes.c_int64), ("inter", ctypes.c_int64), ("n_experts", ctypes.c_int64),
        ("top_k", ctypes.c_int64), ("normalize", ctypes.c_int),
        ("gate_dtype", ctypes.c_int), ("down_dtype", ctypes.c_int),
        ("gate", ctypes.c_void_p), ("up", ctypes.c_void_p), ("down", ctypes.c_void_p),
        ("gate_bytes", ctypes.c_size_t), ("up_bytes", ctypes.c_size_t), ("down_bytes", ctypes.c_size_t),
        ("shared_gate_dtype", ctypes.c_int), ("shared_down_dtype", ctypes.c_int),
        ("shared_gate", ctypes.c_void_p), ("shared_up", ctypes.c_void_p), ("shared_down", ctypes.c_void_p),
        ("selector", ctypes.c_void_p), ("router", ctypes.c_void_p),
    ]


def lib() -> ctypes.CDLL:
    """Load the HIP library (raises OSError when it is missing)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise OSError(f"{LIB_PATH} is missing: build it with `python -m inferq_amd._build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(L, name, None)
            if fn is None:
                continue
            fn.argtypes, fn.restype = args, res
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != IQ_OK:
        raise QgemmError(status, lib().iq_last_error().decode(errors="replace"))


def declared_symbols() -> list[str]:
    """Function names declared in include/*.h (the exported C ABI)."""
    import glob
    import re

    names = []
    for header in sorted(glob.glob(os.path.join(os.path.dirname(PKG), "include", "*.h"))):
        text = open(header).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"\b(iq_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))
