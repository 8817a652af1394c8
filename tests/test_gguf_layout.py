"""The GGUF reader against a file assembled byte by byte in this test from
the published GGUF layout, independent of the fixture writer
(tests/golden/gguf_writer.py), so that one reading of the format is not on
both sides of the check.

Layout (little endian, GGUF v2 and v3 alike):
  u32 magic "GGUF" | u32 version | u64 tensor count | u64 metadata count
  metadata: u64 key length, key bytes, u32 value type, value
    (type 8 string: u64 length + bytes; type 9 array: u32 element type,
    u64 count, elements)
  tensor infos: u64 name length, name, u32 n_dims, n_dims x u64 dims
    (innermost first), u32 GGML type, u64 offset from the data start
  padding to general.alignment, then the tensor data.
The reader must report dims outermost first (the reference's shapes,
src/gguf.rs:1204-1262) and absolute offsets.
"""
import struct

import numpy as np
import pytest

from inferq_amd import gguf as G

ALIGN = 64
F32, Q4_K, Q6_K = 0, 12, 14


def u32(v):
    return struct.pack("<I", v)


def u64(v):
    return struct.pack("<Q", v)


def gstr(s):
    b = s.encode()
    return u64(len(b)) + b


def _file(version, rng, pad_key=""):
    """Bytes of a checkpoint with three tensors and mixed metadata, and the
    expectations the reader must meet; pad_key adds one more string entry
    (to move where the header ends)."""
    meta = b""
    meta += gstr("general.architecture") + u32(8) + gstr("qwen3moe")
    meta += gstr("general.alignment") + u32(4) + u32(ALIGN)
    meta += gstr("tokenizer.ggml.tokens") + u32(9) + u32(8) + u64(3) + gstr("<s>") + gstr("hello") + gstr("")
    meta += gstr("qwen3moe.expert_count") + u32(10) + u64(2)  # u64
    meta += gstr("tiny.i8") + u32(1) + struct.pack("<b", -5)
    meta += gstr("tiny.f64") + u32(12) + struct.pack("<d", 7.75)
    meta += gstr("tiny.flag") + u32(7) + bytes([1])
    meta += gstr("tiny.i16_list") + u32(9) + u32(3) + u64(4) + struct.pack("<4h", 1, -2, 3, -4)
    n_kv = 8
    if pad_key:
        meta += gstr(pad_key) + u32(8) + gstr("x")
        n_kv += 1
    # tensors: a 3-D expert tensor [experts 2, rows 3, cols 512] Q4_K, a 2-D
    # Q6_K [rows 5, cols 256], a 1-D F32 [7]; data offsets chosen here,
    # aligned to 64 and not packed tightly
    exp = rng.integers(0, 256, 2 * 3 * 2 * 144, dtype=np.uint8).tobytes()
    q6 = rng.integers(0, 256, 5 * 210, dtype=np.uint8).tobytes()
    vec = rng.standard_normal(7).astype(np.float32).tobytes()
    rel = {"blk.0.ffn_gate_exps.weight": 0, "output.weight": 1792, "blk.0.ffn_gate_inp_shexp.weight": 3072}
    assert all(v % ALIGN == 0 for v in rel.values())
    assert rel["output.weight"] >= len(exp) and rel["blk.0.ffn_gate_inp_shexp.weight"] >= 1792 + len(q6)
    infos = b""
    infos += gstr("blk.0.ffn_gate_exps.weight") + u32(3) + u64(512) + u64(3) + u64(2) + u32(Q4_K) + u64(rel[
        "blk.0.ffn_gate_exps.weight"])
    infos += gstr("output.weight") + u32(2) + u64(256) + u64(5) + u32(Q6_K) + u64(rel["output.weight"])
    infos += gstr("blk.0.ffn_gate_inp_shexp.weight") + u32(1) + u64(7) + u32(F32) + u64(
        rel["blk.0.ffn_gate_inp_shexp.weight"])
    head = b"GGUF" + u32(version) + u64(3) + u64(n_kv) + meta + infos
    data_start = -(-len(head) // ALIGN) * ALIGN
    data = bytearray(b"\xee" * (rel["blk.0.ffn_gate_inp_shexp.weight"] + len(vec)))  # 0xee: padding bytes
    for name, blob in (("blk.0.ffn_gate_exps.weight", exp), ("output.weight", q6),
                       ("blk.0.ffn_gate_inp_shexp.weight", vec)):
        data[rel[name]:rel[name] + len(blob)] = blob
    raw = head + b"\xcd" * (data_start - len(head)) + bytes(data)
    expect = {
        "blk.0.ffn_gate_exps.weight": (Q4_K, [2, 3, 512], data_start + rel["blk.0.ffn_gate_exps.weight"], exp),
        "output.weight": (Q6_K, [5, 256], data_start + rel["output.weight"], q6),
        "blk.0.ffn_gate_inp_shexp.weight": (F32, [7], data_start + rel["blk.0.ffn_gate_inp_shexp.weight"], vec),
    }
    return raw, expect


@pytest.mark.parametrize("version", [2, 3])
def test_hand_assembled_file(tmp_path, version):
    raw, expect = _file(version, np.random.default_rng(version))
    path = tmp_path / f"v{version}.gguf"
    path.write_bytes(raw)
    ck = G.GgufCheckpoint(str(path))
    infos = ck.tensor_infos()
    assert sorted(t.name for t in infos) == sorted(expect)
    for name, (dtype, shape, offset, blob) in expect.items():
        t = ck.tensor_info(name)
        assert (t.ggml_dtype, t.shape, t.offset, t.storage_bytes) == (dtype, shape, offset, len(blob)), name
        assert raw[t.offset:t.offset + t.storage_bytes] == blob, name
        assert t.offset % ALIGN == 0
    assert ck.meta_str("general.architecture") == "qwen3moe"
    assert ck.meta_int("general.alignment") == ALIGN
    assert ck.meta_int("tokenizer.ggml.tokens") == 3  # arrays report their length
    assert ck.meta_int("qwen3moe.expert_count") == 2
    assert ck.meta_int("tiny.i8") == -5
    assert ck.meta_int("tiny.f64") == 7
    assert ck.meta_int("tiny.flag") == 1
    assert ck.meta_int("tiny.i16_list") == 4
    assert ck.meta_str("tiny.i8") is None


def test_hand_assembled_alignment_is_honoured(tmp_path):
    """A header whose end rounds to different starts at 32 and at 64 bytes:
    the reader must take the file's general.alignment (64)."""
    for n in range(1, 64):
        raw, expect = _file(3, np.random.default_rng(9), pad_key="k" * n)
        head_end = raw.index(b"\xcd" * 8) if b"\xcd" * 8 in raw else None
        if head_end is not None and -(-head_end // 32) * 32 != -(-head_end // 64) * 64:
            break
    else:
        raise AssertionError("no key length gives distinct 32- and 64-byte data starts")
    path = tmp_path / "a.gguf"
    path.write_bytes(raw)
    ck = G.GgufCheckpoint(str(path))
    for name, (dtype, shape, offset, blob) in expect.items():
        t = ck.tensor_info(name)
        assert t.offset == offset and offset == -(-head_end // 64) * 64 + (offset - expect[
            "blk.0.ffn_gate_exps.weight"][2])
        assert raw[t.offset:t.offset + t.storage_bytes] == blob
