"""The GGUF reader on the host (no GPU): the C ABI parses the committed
fixture (tests/golden/tiny_moe.gguf, written by tests/golden/make_gguf.py)
and files written here, and refuses malformed ones with an error.

Pinned by the writer: every tensor's name, GGML type, shape (outermost
first, as the reference reads it, src/gguf.rs:1204-1232), absolute offset
and byte size must equal what the writer laid out, and the bytes at each
offset must be the bytes it wrote.
"""
import os
import struct
import sys

import numpy as np
import pytest

from inferq_amd import _lib
from inferq_amd import gguf as G
from inferq_amd import synth as S

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import gguf_writer as W  # noqa: E402
import make_gguf  # noqa: E402

FIXTURE = os.path.join(HERE, "golden", "tiny_moe.gguf")


def test_fixture_is_reproducible(tmp_path):
    path = tmp_path / "again.gguf"
    make_gguf.build(str(path))
    assert open(path, "rb").read() == open(FIXTURE, "rb").read()


def test_fixture_listing_matches_the_writer(tmp_path):
    offsets, layers = make_gguf.build(str(tmp_path / "t.gguf"))
    ck = G.GgufCheckpoint(FIXTURE)
    infos = ck.tensor_infos()
    assert [t.name for t in infos] == sorted(offsets)
    raw = np.fromfile(FIXTURE, np.uint8)
    for li, (lay, router) in enumerate(layers):
        for name, ttype, shape, data in W.moe_layer_tensors(li, lay, router):
            t = ck.tensor_info(name)
            data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
            assert (t.ggml_dtype, t.shape, t.offset, t.storage_bytes) == (ttype, shape, offsets[name], data.size)
            assert np.array_equal(raw[t.offset:t.offset + t.storage_bytes], data), name
    assert ck.tensor_info("blk.9.ffn_gate_exps.weight") is None
    assert ck.meta_str("general.architecture") == "qwen3moe"
    assert ck.meta_int("qwen3moe.expert_count") == 2
    assert ck.meta_str("qwen3moe.expert_count") is None
    with pytest.raises(_lib.QgemmError, match="no metadata key"):
        ck.meta_int("missing.key")
    # layer 1 was written first: file order is not layer order
    assert ck.tensor_info("blk.1.ffn_gate_exps.weight").offset < ck.tensor_info("blk.0.ffn_gate_exps.weight").offset


def test_alignment_arrays_and_f32(tmp_path):
    rng = np.random.default_rng(3)
    q8 = S.random_matrix(S.Q8_0, 3, 64, rng)
    vec = rng.standard_normal(5).astype(np.float32)
    path = str(tmp_path / "a.gguf")
    offs = W.write_gguf(path, [("a", W.GGML_Q8_0, [3, 64], q8), ("v", W.GGML_F32, [5], vec)],
                        {"general.alignment": 64, "list": [1, 2, 3], "flag": True, "pi": 3.25}, alignment=64)
    ck = G.GgufCheckpoint(path)
    assert all(o % 64 == 0 for o in offs.values())
    assert ck.tensor_info("a").shape == [3, 64] and ck.tensor_info("a").storage_bytes == q8.size
    assert ck.tensor_info("v").shape == [5] and ck.tensor_info("v").offset == offs["v"]
    assert ck.meta_int("general.alignment") == 64 and ck.meta_int("list") == 3 and ck.meta_int("flag") == 1
    assert ck.meta_int("pi") == 3


def _expect_refused(path, text):
    with pytest.raises(_lib.QgemmError, match=text):
        G.GgufCheckpoint(str(path))


def test_malformed_files_are_refused(tmp_path):
    good = open(FIXTURE, "rb").read()
    _expect_refused(tmp_path / "missing.gguf", "cannot open")
    (tmp_path / "magic.gguf").write_bytes(b"GGML" + good[4:])
    _expect_refused(tmp_path / "magic.gguf", "bad magic")
    (tmp_path / "v1.gguf").write_bytes(good[:4] + struct.pack("<I", 1) + good[8:])
    _expect_refused(tmp_path / "v1.gguf", "unsupported GGUF version 1")
    for cut in (3, 10, 30, 200, 1500, len(good) - 1000):
        (tmp_path / "cut.gguf").write_bytes(good[:cut])
        with pytest.raises(_lib.QgemmError):
            G.GgufCheckpoint(str(tmp_path / "cut.gguf"))
    rng = np.random.default_rng(4)
    blocks = S.random_matrix(S.Q4_K, 2, 256, rng)
    p = str(tmp_path / "dup.gguf")
    W.write_gguf(p, [("t", W.GGML_Q4_K, [2, 256], blocks), ("t", W.GGML_Q4_K, [2, 256], blocks)])
    _expect_refused(p, "appears twice")
    p = str(tmp_path / "ragged.gguf")
    W.write_gguf(p, [("t", W.GGML_Q4_K, [2, 256], blocks)])
    raw = bytearray(open(p, "rb").read())
    i = raw.index(struct.pack("<QQ", 256, 2))  # dims innermost first
    raw[i:i + 8] = struct.pack("<Q", 200)  # width not a whole number of blocks
    open(p, "wb").write(bytes(raw))
    _expect_refused(p, "whole number of blocks")
    raw[i:i + 8] = struct.pack("<Q", 256 * 64)  # tensor runs past the end of the file
    open(p, "wb").write(bytes(raw))
    _expect_refused(p, "past the end of the file")
    raw[i:i + 8] = struct.pack("<Q", 256)
    # an aligned offset that wraps past 2^64 onto the header once the data
    # start is added: refused, not read as tensor bytes
    data_start = W.write_gguf(p, [("t", W.GGML_Q4_K, [2, 256], blocks)])["t"]
    raw[i + 20:i + 28] = struct.pack("<Q", (1 << 64) - data_start)  # after the u32 type: the u64 offset
    open(p, "wb").write(bytes(raw))
    _expect_refused(p, "offset overflows")


def test_library_exports_the_gguf_entries():
    L = _lib.lib()
    for name in ("iq_gguf_open", "iq_gguf_load_experts", "iq_experts_layer", "iq_gguf_upload_tensor"):
        assert hasattr(L, name)
