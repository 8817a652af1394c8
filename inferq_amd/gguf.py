"""Host-side mirror of the reference's GGUF checkpoint and expert residency.

`GgufCheckpoint` keeps the interface of inferq's GgufCheckpoint
(src/gguf.rs:790-1460) for this path: tensor listing and lookup, matrices
streamed into HBM, and `warm_all_experts` (src/residency.rs:39-131), which
makes every routed expert resident in file order.  `moe_layer` assembles a
QuantizedMoeLayer from a resident layer the way QuantizedMoeLayer::load does
(src/qwen/quantized_moe.rs:141-225).  Parsing and uploads run in the C ABI
(iq_gguf_*, include/iq_qgemm.h); there is no Python fallback.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

from . import _lib
from ._lib import MoeDesc, QgemmError, check, lib
from .qgemm import QuantizedMatrix, _ensure_init, _stream

GGML_TYPE_NAMES = {0: "F32", 1: "F16", 8: "Q8_0", 12: "Q4K", 13: "Q5K", 14: "Q6K", 30: "BF16"}


@dataclass
class GgufTensorInfo:
    """src/gguf.rs:1204-1232: name, dtype, shape (outermost first), absolute
    file offset and storage bytes."""

    name: str
    dtype: str
    ggml_dtype: int
    shape: list
    offset: int
    storage_bytes: int


class GgufCheckpoint:
    """An open GGUF file (host parse only; no device work until a load)."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        check(lib().iq_gguf_open(str(path).encode(), ctypes.byref(h)))
        self._h = h
        self.path = str(path)

    @classmethod
    def open(cls, path: str) -> "GgufCheckpoint":
        return cls(path)

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and _lib._lib is not None:
            _lib._lib.iq_gguf_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- listing -------------------------------------------------------
    def tensor_info(self, name: str) -> GgufTensorInfo | None:
        dt, nd = ctypes.c_int(), ctypes.c_int()
        dims = (ctypes.c_int64 * 4)()
        off, nb = ctypes.c_uint64(), ctypes.c_uint64()
        rc = lib().iq_gguf_tensor_info(self._h, name.encode(), ctypes.byref(dt), ctypes.byref(nd), dims,
                                       ctypes.byref(off), ctypes.byref(nb))
        if rc == _lib.IQ_ERR_RANGE:
            return None
        check(rc)
        return GgufTensorInfo(name, GGML_TYPE_NAMES.get(dt.value, f"type{dt.value}"), dt.value,
                              [dims[i] for i in range(nd.value)], off.value, nb.value)

    def tensor_infos(self) -> list:
        n = lib().iq_gguf_tensor_count(self._h)
        names = [lib().iq_gguf_tensor_name(self._h, i).decode() for i in range(n)]
        return sorted((self.tensor_info(nm) for nm in names), key=lambda t: t.name)

    def meta_int(self, key: str) -> int:
        v = ctypes.c_int64()
        check(lib().iq_gguf_meta_int(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def meta_str(self, key: str) -> str | None:
        s = lib().iq_gguf_meta_str(self._h, key.encode())
        return None if s is None else s.decode()

    # ---- loads ---------------------------------------------------------
    def load_matrix(self, name: str) -> QuantizedMatrix:
        """src/gguf.rs:1234: a 2-D quantised tensor, resident in HBM."""
        _ensure_init()
        h = ctypes.c_void_p()
        check(lib().iq_gguf_load_matrix(self._h, name.encode(), ctypes.byref(h)))
        return QuantizedMatrix(h)

    def load_f32(self, name: str):
        """An F32 tensor (router, shared-expert selector) as a device tensor
        of the shape the reference reads (outermost first)."""
        import torch

        _ensure_init()
        info = self.tensor_info(name)
        if info is None:
            raise QgemmError(_lib.IQ_ERR_RANGE, f"GGUF is missing tensor {name!r}")
        if info.ggml_dtype != 0:
            raise QgemmError(_lib.IQ_ERR_DTYPE, f"GGUF tensor {name!r} is {info.dtype}, expected F32")
        t = torch.empty(info.shape, dtype=torch.float32, device=torch.device("cuda", torch.cuda.current_device()))
        check(lib().iq_gguf_upload_tensor(self._h, name.encode(), t.data_ptr(), t.numel() * 4, _stream()))
        return t

    def warm_all_experts(self, n_layers: int) -> "ExpertResidency":
        """src/residency.rs:39-131 with a pinned cache: every routed expert of
        layers [0, n_layers) resident in HBM, read in file order, gate/up
        paired."""
        _ensure_init()
        h = ctypes.c_void_p()
        check(lib().iq_gguf_load_experts(self._h, n_layers, ctypes.byref(h)))
        return ExpertResidency(h, n_layers)

    def moe_layer(self, residency: "ExpertResidency", layer: int, experts_per_token: int,
                  normalize_top_k: bool = True, with_router: bool = True):
        """QuantizedMoeLayer::load (src/qwen/quantized_moe.rs:141-225) over
        resident experts: the router, the shared expert and its selector are
        loaded from the checkpoint; routed experts are the resident ones."""
        from .moe import QuantizedMoeLayer

        prefix = f"blk.{layer}"
        desc = residency.desc(layer)
        router = self.load_f32(f"{prefix}.ffn_gate_inp.weight") if with_router else None
        if router is not None and list(router.shape) != [desc.n_experts, desc.hidden]:
            raise QgemmError(_lib.IQ_ERR_SHAPE, f"router shape {list(router.shape)} does not match "
                                                f"[{desc.n_experts}, {desc.hidden}]")
        shared = [self.load_matrix(f"{prefix}.ffn_{p}_shexp.weight") for p in ("gate", "up", "down")]
        selector = self.load_f32(f"{prefix}.ffn_gate_inp_shexp.weight").reshape(-1)
        return QuantizedMoeLayer.from_desc(desc, experts_per_token, normalize_top_k, shared, selector, router,
                                           keepalive=[residency, shared, selector, router])


class ExpertResidency:
    """Owner of the resident expert tensors (iq_experts_t)."""

    def __init__(self, handle: ctypes.c_void_p, n_layers: int):
        self._h = handle
        self.n_layers = n_layers

    def __del__(self):
        if getattr(self, "_h", None) is not None and _lib._lib is not None:
            _lib._lib.iq_experts_free(self._h)
            self._h = None

    def bytes(self) -> int:
        return lib().iq_experts_bytes(self._h)

    def desc(self, layer: int) -> MoeDesc:
        d = MoeDesc()
        check(lib().iq_experts_layer(self._h, layer, ctypes.byref(d)))
        return d

    def tensor_pointers(self, layer: int) -> dict:
        d = self.desc(layer)
        return {"gate": d.gate, "up": d.up, "down": d.down, "gate_bytes": d.gate_bytes, "down_bytes": d.down_bytes}
