"""The C-ABI library (inferq_amd/libiq_qgemm.so) on the CPU: it loads,
exports exactly what include/*.h declares, and rejects malformed calls with
the reference's error categories before any device work (no GPU needed).
"""
import ctypes
import subprocess

import numpy as np
import pytest

import inferq_amd
from inferq_amd import _lib
from inferq_amd import synth as S


@pytest.fixture(scope="module")
def L():
    return inferq_amd.lib()


def _exported(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], check=True, capture_output=True, text=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_library_exports_every_declared_symbol(L):
    declared = _lib.declared_symbols()
    assert len(declared) >= 20
    for name in declared:
        assert hasattr(L, name), name
    iq = {s for s in _exported(_lib.LIB_PATH) if s.startswith("iq_")}
    assert iq == set(declared), f"exported but undeclared: {iq - set(declared)}"


def test_every_declared_symbol_has_a_ctypes_signature():
    assert set(_lib.declared_symbols()) == set(_lib._SIGNATURES)


def test_version_string(L):
    assert b"gfx950" in L.iq_version()


def _err(L, rc, status, text=None):
    assert rc == status, (rc, L.iq_last_error())
    if text:
        assert text in L.iq_last_error().decode()


def test_upload_rejects_malformed_matrices(L):
    h = ctypes.c_void_p()
    buf = np.zeros(4096, np.uint8)
    p = buf.ctypes.data
    _err(L, L.iq_weights_upload(p, 144, 2, 1, 256, ctypes.byref(h)), _lib.IQ_ERR_DTYPE,
         "unsupported executable GGUF matrix dtype 2")
    # src/gguf.rs:1729-1739: a 300-column K-quant matrix is not representable
    _err(L, L.iq_weights_upload(p, 144, _lib.IQ_Q4_K, 1, 300, ctypes.byref(h)), _lib.IQ_ERR_SHAPE,
         "not divisible by Q4K block size 256")
    _err(L, L.iq_weights_upload(p, 143, _lib.IQ_Q4_K, 1, 256, ctypes.byref(h)), _lib.IQ_ERR_SHAPE,
         "quantized matrix has 143 bytes, expected 144")
    _err(L, L.iq_weights_upload(p, 70, _lib.IQ_Q8_0, 2, 32, ctypes.byref(h)), _lib.IQ_ERR_SHAPE, "expected 68")
    _err(L, L.iq_weights_upload(p, 0, _lib.IQ_Q6_K, 0, 256, ctypes.byref(h)), _lib.IQ_ERR_SHAPE, "invalid matrix shape")
    _err(L, L.iq_weights_upload(None, 144, _lib.IQ_Q4_K, 1, 256, ctypes.byref(h)), _lib.IQ_ERR_INVALID)
    _err(L, L.iq_weights_view(p + 4, 144, _lib.IQ_Q4_K, 1, 256, ctypes.byref(h)), _lib.IQ_ERR_INVALID,
         "16-byte aligned")
    # F32 and BF16 are executable matrix dtypes (src/gguf.rs:305-317) with
    # one element per "block"; F16 is not
    _err(L, L.iq_weights_upload(p, 10, _lib.IQ_F32, 2, 3, ctypes.byref(h)), _lib.IQ_ERR_SHAPE,
         "quantized matrix has 10 bytes, expected 24")
    _err(L, L.iq_weights_upload(p, 10, _lib.IQ_BF16, 2, 3, ctypes.byref(h)), _lib.IQ_ERR_SHAPE, "expected 12")
    _err(L, L.iq_weights_upload(p, 12, 1, 2, 3, ctypes.byref(h)), _lib.IQ_ERR_DTYPE,
         "expected Q4_K, Q5_K, Q6_K, Q8_0, F32, or BF16")


def test_null_handles_are_rejected(L):
    x = np.zeros(256, np.float32).ctypes.data
    _err(L, L.iq_matmul(None, x, 1, x, None), _lib.IQ_ERR_INVALID, "null quantized matrix handle")
    _err(L, L.iq_matmul_host(None, x, 1, x), _lib.IQ_ERR_INVALID)
    _err(L, L.iq_moe_forward(None, x, x, 1, x, None, None, None), _lib.IQ_ERR_INVALID, "null MoE handle")
    _err(L, L.iq_moe_forward_stage(None, 1, None), _lib.IQ_ERR_INVALID)
    # releasing a null handle is a no-op, as free(NULL) is
    assert L.iq_weights_free(None) == _lib.IQ_OK and L.iq_moe_destroy(None) == _lib.IQ_OK
    assert L.iq_matmul_workspace_size(None, 1) == 0


def _desc(**kw):
    d = _lib.MoeDesc(hidden=256, inter=256, n_experts=4, top_k=2, normalize=1,
                     gate_dtype=_lib.IQ_Q4_K, down_dtype=_lib.IQ_Q6_K)
    fake = 1 << 20  # aligned non-null addresses; creation never dereferences them
    d.gate, d.up, d.down = fake, fake, fake
    d.gate_bytes = d.up_bytes = S.matrix_bytes(S.Q4_K, 4 * 256, 256)
    d.down_bytes = S.matrix_bytes(S.Q6_K, 4 * 256, 256)
    for k, v in kw.items():
        setattr(d, k, v)
    return d


@pytest.mark.parametrize("kw,status,text", [
    (dict(top_k=0), _lib.IQ_ERR_SHAPE, "invalid top-k 0 for 4 experts"),
    (dict(top_k=5), _lib.IQ_ERR_SHAPE, "invalid top-k 5 for 4 experts"),
    (dict(gate_dtype=2), _lib.IQ_ERR_DTYPE, "unsupported expert dtypes"),
    (dict(hidden=300), _lib.IQ_ERR_SHAPE, "do not fit"),
    (dict(up_bytes=144), _lib.IQ_ERR_SHAPE, "up expert shape"),
    (dict(down_bytes=210), _lib.IQ_ERR_SHAPE, "invalid down expert shape"),
    (dict(up=0), _lib.IQ_ERR_INVALID, "null expert tensor"),
    (dict(down=(1 << 20) + 8), _lib.IQ_ERR_INVALID, "16-byte aligned"),
    (dict(shared_gate=1 << 20), _lib.IQ_ERR_INVALID, "shared expert needs gate, up and down"),
    (dict(shared_gate=1 << 20, shared_up=1 << 20, shared_down=1 << 20, shared_gate_dtype=_lib.IQ_Q4_K,
          shared_down_dtype=_lib.IQ_Q6_K), _lib.IQ_ERR_INVALID, "selector"),
    (dict(n_experts=1024, top_k=2, gate_bytes=S.matrix_bytes(S.Q4_K, 1024 * 256, 256)), _lib.IQ_ERR_RANGE,
     "at most 512 experts"),
])
def test_moe_create_rejects_malformed_layers(L, kw, status, text):
    """Load-time checks of QuantizedMoeLayer::load (src/qwen/quantized_moe.rs:141-225)."""
    h = ctypes.c_void_p()
    d = _desc(**kw)
    _err(L, L.iq_moe_create(ctypes.byref(d), ctypes.byref(h)), status, text)
    assert not h.value


def test_product_path_has_no_cpu_fallback(monkeypatch, tmp_path):
    """With the library missing the package raises instead of computing."""
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "libiq_qgemm.so"))
    with pytest.raises(OSError, match="missing"):
        _lib.lib()


def test_moe_rejects_host_tensors():
    """Host (CPU) tensors never reach the C ABI: their addresses would be
    dereferenced by the kernels as device addresses."""
    import torch

    from inferq_amd import moe

    cpu = torch.zeros(4, dtype=torch.uint8)
    with pytest.raises(_lib.QgemmError, match="resident in HBM"):
        moe.QuantizedMoeLayer(256, 256, 4, 2, S.Q4_K, S.Q6_K, cpu, cpu, cpu)
    layer = object.__new__(moe.QuantizedMoeLayer)
    layer.hidden, layer.n_experts, layer.top_k, layer.device = 256, 4, 2, 0
    x = torch.zeros(1, 256)
    for call in (lambda: layer.forward_into(x, torch.zeros(1, 4), torch.zeros(1, 256)),
                 lambda: layer.forward(x, torch.zeros(1, 4)),
                 lambda: layer.forward_timed(x, torch.zeros(1, 4), torch.zeros(1, 256), [None] * 4)):
        with pytest.raises(_lib.QgemmError, match="must be a tensor on cuda:0"):
            call()


def test_row_entries_check_the_reference_preconditions(L):
    """q4k_q8k_row's debug asserts (src/qgemm.rs:450-451) become status
    codes, checked before any device work."""
    L = _lib.lib()
    w = np.zeros(144 * 2, np.uint8)
    x = np.zeros(292 * 6, np.uint8)
    out = np.zeros(3, np.float32)
    _err(L, L.iq_q4k_q8k_row(w.ctypes.data, 2, x.ctypes.data, 6, 3, out.ctypes.data, 2), _lib.IQ_ERR_SHAPE,
         "out.len() 2 != rows 3")
    _err(L, L.iq_q6k_q8k_row(w.ctypes.data, 2, x.ctypes.data, 5, 3, out.ctypes.data, 3), _lib.IQ_ERR_SHAPE,
         "inputs.len() 5 != rows 3 x weight.len() 2")
    _err(L, L.iq_q80_q80_row(None, 2, x.ctypes.data, 6, 3, out.ctypes.data, 3), _lib.IQ_ERR_INVALID, "null slice")


def test_rust_binding_declares_every_entry():
    """The FFI crate (inferq_amd/rust/inferq-amd-sys) binds every entry
    include/*.h declares, and nothing else."""
    import os
    import re

    src = os.path.join(os.path.dirname(inferq_amd.__file__), "rust", "inferq-amd-sys", "src", "lib.rs")
    text = open(src).read()
    block = text[text.index('extern "C" {'):]
    block = block[:block.index("\n}\n")]
    bound = set(re.findall(r"pub fn (iq_[a-z0-9_]+)\(", block))
    assert bound == set(_lib.declared_symbols())
