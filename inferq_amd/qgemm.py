"""Host-side mirror of the reference's executable quantised matrix.

`QuantizedMatrix` keeps the interface of inferq's QuantizedMatrix
(src/gguf.rs:163-690): the same method names, argument meaning and error
behaviour, with the packed GGUF blocks resident in HBM and every product run
by the gfx950 kernels through the C ABI (include/iq_qgemm.h).  PyTorch is
used only for device memory and the current stream.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import IQ_BF16, IQ_F32, IQ_Q4_K, IQ_Q5_K, IQ_Q6_K, IQ_Q8_0, QgemmError, check, lib

DTYPE_NAMES = {IQ_Q4_K: "Q4K", IQ_Q5_K: "Q5K", IQ_Q6_K: "Q6K", IQ_Q8_0: "Q8_0", IQ_F32: "F32", IQ_BF16: "BF16"}
BLOCK_ELEMS = {IQ_Q4_K: 256, IQ_Q5_K: 256, IQ_Q6_K: 256, IQ_Q8_0: 32, IQ_F32: 1, IQ_BF16: 1}
BLOCK_BYTES = {IQ_Q4_K: 144, IQ_Q5_K: 176, IQ_Q6_K: 210, IQ_Q8_0: 34, IQ_F32: 4, IQ_BF16: 2}

_initialised = set()


def init(device: int = 0) -> None:
    """Bind the calling thread to `device` (a gfx950 GPU)."""
    import torch

    torch.cuda.set_device(device)
    check(lib().iq_init(device))
    _initialised.add(device)


def _ensure_init():
    import torch

    dev = torch.cuda.current_device()
    if dev not in _initialised:
        init(dev)


def _stream():
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class QuantizedMatrix:
    """A [rows x cols] GGUF matrix (Q4_K, Q6_K or Q8_0) resident in HBM."""

    def __init__(self, handle: ctypes.c_void_p, keepalive=None):
        self._h = handle
        self._keepalive = keepalive  # device buffer a view borrows
        dt, r, c, nb = ctypes.c_int(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_size_t()
        check(lib().iq_weights_info(self._h, ctypes.byref(dt), ctypes.byref(r), ctypes.byref(c), ctypes.byref(nb),
                                    None))
        self._dtype, self._rows, self._cols, self._bytes = dt.value, r.value, c.value, nb.value

    # ---- construction --------------------------------------------------
    @classmethod
    def upload(cls, data, dtype: int, rows: int, cols: int) -> "QuantizedMatrix":
        """Copy host GGUF block bytes (bytes / numpy uint8) to HBM."""
        _ensure_init()
        arr = np.ascontiguousarray(np.frombuffer(data, dtype=np.uint8) if isinstance(data, (bytes, bytearray))
                                   else np.asarray(data).view(np.uint8).reshape(-1))
        h = ctypes.c_void_p()
        check(lib().iq_weights_upload(arr.ctypes.data, arr.nbytes, dtype, rows, cols, ctypes.byref(h)))
        return cls(h)

    @classmethod
    def view(cls, device_tensor, dtype: int, rows: int, cols: int, offset: int = 0,
             nbytes: int | None = None) -> "QuantizedMatrix":
        """Wrap bytes already in HBM (a CUDA uint8 tensor) without copying."""
        _ensure_init()
        if nbytes is None:
            nbytes = rows * (cols // BLOCK_ELEMS.get(dtype, 1)) * BLOCK_BYTES.get(dtype, 0)
        h = ctypes.c_void_p()
        check(lib().iq_weights_view(device_tensor.data_ptr() + offset, nbytes, dtype, rows, cols, ctypes.byref(h)))
        return cls(h, keepalive=device_tensor)

    def __del__(self):
        h = getattr(self, "_h", None)
        L = getattr(_lib, "_lib", None) if _lib is not None else None  # module globals are gone at interpreter exit
        if h is not None and L is not None:
            L.iq_weights_free(h)
            self._h = None

    # ---- reference accessors (src/gguf.rs:322-332) --------------------
    def dtype(self) -> str:
        return DTYPE_NAMES[self._dtype]

    @property
    def ggml_dtype(self) -> int:
        return self._dtype

    def shape(self) -> list[int]:
        return [self._rows, self._cols]

    def storage_bytes(self) -> int:
        return self._bytes

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def device_ptr(self) -> int:
        p = ctypes.c_void_p()
        check(lib().iq_weights_info(self._h, None, None, None, None, ctypes.byref(p)))
        return p.value

    # ---- derived matrices ----------------------------------------------
    def concatenate_rows(self, other: "QuantizedMatrix") -> "QuantizedMatrix":
        """src/gguf.rs:379-404: this matrix's rows, then `other`'s."""
        h = ctypes.c_void_p()
        check(lib().iq_weights_concat_rows(self._h, other._h, ctypes.byref(h)))
        return QuantizedMatrix(h)

    def leading_rows(self, rows: int) -> "QuantizedMatrix":
        """src/gguf.rs:352-377: the first `rows` output rows."""
        h = ctypes.c_void_p()
        check(lib().iq_weights_leading_rows(self._h, rows, ctypes.byref(h)))
        return QuantizedMatrix(h)

    # ---- products --------------------------------------------------------
    def _validated_input(self, xs):
        """src/gguf.rs:692-708: rank >= 2, last dim == cols, converted to f32."""
        import torch

        if xs.dim() < 2:
            raise QgemmError(_lib.IQ_ERR_SHAPE, "quantized matrix input must have rank at least two")
        if xs.shape[-1] != self._cols:
            raise QgemmError(_lib.IQ_ERR_SHAPE, f"quantized matrix input has final dimension {xs.shape[-1]}, "
                                                f"expected {self._cols}")
        if not xs.is_cuda:
            raise QgemmError(_lib.IQ_ERR_INVALID, "quantized matrix input must be a device (HBM) tensor")
        return xs.to(torch.float32).contiguous()

    def forward(self, xs):
        """src/gguf.rs:406: y[..., rows] = xs[..., cols] . W^T."""
        import torch

        xs = self._validated_input(xs)
        m = xs.numel() // self._cols
        y = torch.empty(*xs.shape[:-1], self._rows, dtype=torch.float32, device=xs.device)
        check(lib().iq_matmul(self._h, xs.data_ptr(), m, y.data_ptr(), _stream()))
        return y

    def forward_via(self, xs, path: int):
        """src/gguf.rs:522-556: run one chosen kernel (an `iq_path` value,
        e.g. `_lib.PATH_PREFILL_TILES`), bypassing the dispatch."""
        import torch

        xs = self._validated_input(xs)
        m = xs.numel() // self._cols
        y = torch.empty(*xs.shape[:-1], self._rows, dtype=torch.float32, device=xs.device)
        check(lib().iq_matmul_via(self._h, xs.data_ptr(), m, y.data_ptr(), path, _stream()))
        return y

    def forward_argmax(self, xs):
        """Greedy token selection on the product (iq_matmul_argmax): per
        input row the last index of the largest finite logit and that
        logit (src/qwen/quantized_model.rs:737-743 + src/sampling.rs:
        104-110), without materialising the logits.  Index -1: the row had
        no finite logit."""
        import torch

        xs = self._validated_input(xs)
        m = xs.numel() // self._cols
        idx = torch.empty(*xs.shape[:-1], dtype=torch.int32, device=xs.device)
        val = torch.empty(*xs.shape[:-1], dtype=torch.float32, device=xs.device)
        check(lib().iq_matmul_argmax(self._h, xs.data_ptr(), m, idx.data_ptr(), val.data_ptr(), _stream()))
        return idx, val

    def reserve(self, input_rows: int) -> None:
        """Size the current stream's library workspace for products of up to
        `input_rows` rows of this matrix (iq_matmul_reserve), so that they
        can be captured into a graph without an eager call first."""
        _ensure_init()
        check(lib().iq_matmul_reserve(self._h, int(input_rows), _stream()))

    def forward_into(self, x, y, path: int = 0) -> None:
        """Raw call: contiguous device f32 x [m, cols] into y [m, rows]
        (`path` as forward_via; 0 = the dispatch)."""
        m = x.numel() // self._cols
        check(lib().iq_matmul_via(self._h, x.data_ptr(), m, y.data_ptr(), path, _stream()))

    # Where the output rows are computed never changes the result
    # (RowSpread, src/gguf.rs:64-80); on the GPU there is one spread.
    def forward_spread(self, xs, spread=None):
        return self.forward(xs)

    def forward_rows(self, values, input_rows: int):
        """src/gguf.rs:433-456: `input_rows` contiguous rows of a flat f32
        device tensor, result flat row-major [input_rows x rows]."""
        import torch

        if values.numel() != input_rows * self._cols:
            raise QgemmError(_lib.IQ_ERR_SHAPE, f"expected {input_rows * self._cols} input values for {input_rows} "
                                                f"rows of {self._cols} columns, got {values.numel()}")
        x = values.reshape(input_rows, self._cols)
        return self.forward(x).reshape(-1) if input_rows else torch.empty(0, device=values.device)

    def forward_host(self, x: np.ndarray) -> np.ndarray:
        """Host f32 [m x cols] in, host f32 [m x rows] out (iq_matmul_host)."""
        _ensure_init()
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim < 2 or x.shape[-1] != self._cols:
            raise QgemmError(_lib.IQ_ERR_SHAPE, f"quantized matrix input has final dimension {x.shape[-1]}, "
                                                f"expected {self._cols}")
        m = x.size // self._cols
        y = np.empty((*x.shape[:-1], self._rows), np.float32)
        check(lib().iq_matmul_host(self._h, x.ctypes.data, m, y.ctypes.data))
        return y

    def block_sums(self, xs):
        """Per-block lane integers of xs . W^T (see iq_block_sums)."""
        import torch

        xs = self._validated_input(xs)
        m = xs.numel() // self._cols
        nb = self._cols // BLOCK_ELEMS[self._dtype]
        y = torch.empty(m, self._rows, dtype=torch.float32, device=xs.device)
        isum = torch.empty(m, self._rows, nb, 8, dtype=torch.int32, device=xs.device)
        msum = torch.empty(m, self._rows, nb, 4, dtype=torch.int32, device=xs.device)
        check(lib().iq_block_sums(self._h, xs.data_ptr(), m, y.data_ptr(), isum.data_ptr(), msum.data_ptr(),
                                  _stream()))
        return y, isum, (msum if self._dtype in (IQ_Q4_K, IQ_Q5_K) else None)

    def prefill_block_sums(self, xs):
        """Product and per-block integer totals of the int8-MFMA path (Q4_K,
        64+ rows; see iq_prefill_block_sums): y, isum, msum [m, rows, blocks]."""
        import torch

        xs = self._validated_input(xs)
        m = xs.numel() // self._cols
        nb = self._cols // 256
        y = torch.empty(m, self._rows, dtype=torch.float32, device=xs.device)
        isum = torch.empty(m, self._rows, nb, dtype=torch.int32, device=xs.device)
        msum = torch.empty(m, self._rows, nb, dtype=torch.int32, device=xs.device)
        check(lib().iq_prefill_block_sums(self._h, xs.data_ptr(), m, y.data_ptr(), isum.data_ptr(), msum.data_ptr(),
                                          _stream()))
        return y, isum, msum


def row_kernel(dtype: int, weight_row, inputs_block_major, rows: int) -> np.ndarray:
    """The reference's per-row entry (q4k_q8k_row / q6k_q8k_row / q80_q80_row,
    src/qgemm.rs:447-468) on host arrays: one weight row of GGUF blocks
    against `rows` quantised input rows stored block-major."""
    _ensure_init()
    fn = {IQ_Q4_K: "iq_q4k_q8k_row", IQ_Q6_K: "iq_q6k_q8k_row", IQ_Q8_0: "iq_q80_q80_row"}.get(dtype)
    if fn is None:
        raise QgemmError(_lib.IQ_ERR_DTYPE, f"no per-row kernel for dtype {dtype}")
    w = np.ascontiguousarray(weight_row).view(np.uint8).reshape(-1)
    x = np.ascontiguousarray(inputs_block_major).view(np.uint8).reshape(-1)
    out = np.empty(rows, np.float32)
    ib = 34 if dtype == IQ_Q8_0 else 292
    check(getattr(lib(), fn)(w.ctypes.data, w.size // BLOCK_BYTES[dtype], x.ctypes.data, x.size // ib, rows,
                             out.ctypes.data, rows))
    return out


def release_workspace() -> None:
    """Free the current stream's library workspace (iq_workspace_release)."""
    _ensure_init()
    check(lib().iq_workspace_release(_stream()))


def argmax(logits):
    """sampling::argmax (src/sampling.rs:104-110) over the last dimension of
    device f32 logits: (index, value) per row, index -1 when a row has no
    finite value."""
    import torch

    _ensure_init()
    if not logits.is_cuda:
        raise QgemmError(_lib.IQ_ERR_INVALID, "argmax logits must be a device (HBM) tensor")
    y = logits.to(torch.float32).contiguous()
    n = y.shape[-1]
    m = y.numel() // n if n else 0
    idx = torch.empty(y.shape[:-1], dtype=torch.int32, device=y.device)
    val = torch.empty(y.shape[:-1], dtype=torch.float32, device=y.device)
    check(lib().iq_argmax_rows(y.data_ptr(), m, n, idx.data_ptr(), val.data_ptr(), _stream()))
    return idx, val


def quantize_q8k(xs):
    """Q8K blocks (292 B each) of device f32 rows xs[m x k], k % 256 == 0."""
    import torch

    _ensure_init()
    xs = xs.to(torch.float32).contiguous()
    k = xs.shape[-1]
    m = xs.numel() // k
    out = torch.empty(m * (k // 256) * 292, dtype=torch.uint8, device=xs.device)
    check(lib().iq_quantize_q8k(xs.data_ptr(), m, k, out.data_ptr(), _stream()))
    return out


def quantize_q80(xs):
    """Q8_0 blocks (34 B each) of device f32 rows xs[m x k], k % 32 == 0."""
    import torch

    _ensure_init()
    xs = xs.to(torch.float32).contiguous()
    k = xs.shape[-1]
    m = xs.numel() // k
    out = torch.empty(m * (k // 32) * 34, dtype=torch.uint8, device=xs.device)
    check(lib().iq_quantize_q80(xs.data_ptr(), m, k, out.data_ptr(), _stream()))
    return out
