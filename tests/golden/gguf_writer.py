"""Test-side GGUF v3 writer (little endian), from the public GGUF layout:
magic "GGUF", version, tensor count, metadata count, metadata key/values,
tensor infos (name, dimension count, dimensions innermost first, GGML type,
offset from the data start), padding to the alignment, tensor data with each
tensor at an aligned offset.  Used to write the fixtures the GGUF reader is
tested on; the reference writes its own test checkpoints the same way
(candle gguf_file::write in src/qwen/quantized_moe.rs:536-548).
"""
from __future__ import annotations

import struct

import numpy as np

GGML_F32, GGML_Q8_0, GGML_Q4_K, GGML_Q5_K, GGML_Q6_K = 0, 8, 12, 13, 14

_META_TYPES = {"u32": 4, "i32": 5, "f32": 6, "bool": 7, "str": 8, "u64": 10}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _meta(key: str, value) -> bytes:
    if isinstance(value, bool):
        return _str(key) + struct.pack("<IB", _META_TYPES["bool"], int(value))
    if isinstance(value, int):
        return _str(key) + struct.pack("<II", _META_TYPES["u32"], value)
    if isinstance(value, float):
        return _str(key) + struct.pack("<If", _META_TYPES["f32"], value)
    if isinstance(value, str):
        return _str(key) + struct.pack("<I", _META_TYPES["str"]) + _str(value)
    if isinstance(value, list):  # array of u32
        return _str(key) + struct.pack("<IIQ", 9, _META_TYPES["u32"], len(value)) + struct.pack(
            f"<{len(value)}I", *value)
    raise TypeError(f"unsupported metadata value {value!r}")


def write_gguf(path: str, tensors, metadata: dict | None = None, alignment: int = 32, version: int = 3) -> dict:
    """tensors: iterable of (name, ggml_type, shape outermost first, bytes).
    Tensor data is laid out in the given order.  Returns {name: absolute
    file offset} of the tensor data."""
    metadata = dict(metadata or {})
    if alignment != 32:
        metadata["general.alignment"] = alignment
    tensors = [(n, t, list(shape), np.ascontiguousarray(b).view(np.uint8).reshape(-1)) for n, t, shape, b in tensors]
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(metadata))
    head += b"".join(_meta(k, v) for k, v in metadata.items())
    rel, offsets = 0, []
    infos = b""
    for name, ttype, shape, data in tensors:
        offsets.append(rel)
        infos += _str(name) + struct.pack("<I", len(shape)) + struct.pack(f"<{len(shape)}Q", *reversed(shape))
        infos += struct.pack("<IQ", ttype, rel)
        rel += (data.size + alignment - 1) // alignment * alignment
    head += infos
    data_start = (len(head) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * (data_start - len(head)))
        for (name, _, _, data), off in zip(tensors, offsets):
            f.seek(data_start + off)
            f.write(data.tobytes())
        end = data_start + rel
        f.truncate(end)
    return {name: data_start + off for (name, _, _, _), off in zip(tensors, offsets)}


def moe_layer_tensors(layer: int, lay: dict, router: np.ndarray):
    """The tensors QuantizedMoeLayer::load reads for one layer
    (src/qwen/quantized_moe.rs:148-200), from a synth.random_moe_layer dict."""
    E, H, I = lay["n_experts"], lay["hidden"], lay["inter"]
    p = f"blk.{layer}"
    return [
        (f"{p}.ffn_gate_inp.weight", GGML_F32, [E, H], router.astype(np.float32)),
        (f"{p}.ffn_gate_exps.weight", lay["gate_dtype"], [E, I, H], lay["gate"]),
        (f"{p}.ffn_up_exps.weight", lay["gate_dtype"], [E, I, H], lay["up"]),
        (f"{p}.ffn_down_exps.weight", lay["down_dtype"], [E, H, I], lay["down"]),
        (f"{p}.ffn_gate_shexp.weight", lay.get("shared_gate_dtype", lay["gate_dtype"]), [I, H], lay["shared_gate"]),
        (f"{p}.ffn_up_shexp.weight", lay.get("shared_gate_dtype", lay["gate_dtype"]), [I, H], lay["shared_up"]),
        (f"{p}.ffn_down_shexp.weight", lay.get("shared_down_dtype", lay["down_dtype"]), [H, I], lay["shared_down"]),
        (f"{p}.ffn_gate_inp_shexp.weight", GGML_F32, [H], lay["selector"].astype(np.float32)),
    ]
