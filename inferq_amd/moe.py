"""Host-side mirror of the reference's quantised MoE sublayer.

`QuantizedMoeLayer` keeps the interface of inferq's QuantizedMoeLayer
(src/qwen/quantized_moe.rs:105-460) with the routed experts resident in HBM
as the GGUF expert tensors and the whole layer (router matmul when the
layer has a router, routing, grouped experts, SwiGLU, ordered combine,
shared expert, optionally the decoder layer's residual add) run by the
gfx950 kernels through the C ABI.  Router logits may also be given.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

from . import _lib
from ._lib import MoeDesc, QgemmError, check, lib
from .qgemm import BLOCK_BYTES, BLOCK_ELEMS, _ensure_init, _stream


@dataclass
class Route:
    """src/qwen/moe.rs:14-19 (without the logits echo)."""

    experts: list
    weights: list


@dataclass
class QuantizedMoeOutput:
    hidden: object  # torch.Tensor [..., hidden]
    routes: list


def _rows_bytes(dtype: int, rows: int, cols: int) -> int:
    return rows * (cols // BLOCK_ELEMS[dtype]) * BLOCK_BYTES[dtype]


class QuantizedMoeLayer:
    """One MoE sublayer over device tensors (uint8 GGUF bytes, f32 selector)."""

    def __init__(self, hidden: int, inter: int, n_experts: int, top_k: int, gate_dtype: int, down_dtype: int,
                 gate, up, down, shared_gate=None, shared_up=None, shared_down=None, selector=None,
                 normalize: bool = True, shared_gate_dtype: int | None = None,
                 shared_down_dtype: int | None = None, router=None):
        import torch

        named = (("gate", gate), ("up", up), ("down", down), ("shared_gate", shared_gate),
                 ("shared_up", shared_up), ("shared_down", shared_down), ("selector", selector),
                 ("router", router))
        for name, t in named:  # before any device call: a host tensor is a caller error, not a missing GPU
            if t is not None and not t.is_cuda:
                raise QgemmError(_lib.IQ_ERR_INVALID, f"MoE {name} tensor must be resident in HBM (got {t.device})")
        _ensure_init()
        self.hidden, self.inter, self.n_experts, self.top_k = hidden, inter, n_experts, top_k
        self.device = torch.cuda.current_device()
        self._check_device(**dict(named))
        self._keep = [t for t in (gate, up, down, shared_gate, shared_up, shared_down, selector, router)
                      if t is not None]
        self.has_router = router is not None

        def ptr(t):
            return None if t is None else t.data_ptr()

        def nbytes(t):
            return 0 if t is None else t.numel() * t.element_size()

        desc = MoeDesc(
            hidden, inter, n_experts, top_k, int(normalize), gate_dtype, down_dtype,
            ptr(gate), ptr(up), ptr(down), nbytes(gate), nbytes(up), nbytes(down),
            shared_gate_dtype if shared_gate_dtype is not None else gate_dtype,
            shared_down_dtype if shared_down_dtype is not None else down_dtype,
            ptr(shared_gate), ptr(shared_up), ptr(shared_down), ptr(selector), ptr(router),
        )
        h = ctypes.c_void_p()
        check(lib().iq_moe_create(ctypes.byref(desc), ctypes.byref(h)))
        self._h = h

    @classmethod
    def from_desc(cls, routed, top_k: int, normalize: bool, shared, selector, router, keepalive) -> "QuantizedMoeLayer":
        """A layer over routed experts already resident (an iq_moe_desc with
        the routed fields filled, e.g. from ExpertResidency.desc), plus the
        shared expert's three QuantizedMatrix objects, its f32 selector and
        the optional f32 router (device tensors).  `keepalive` holds
        whatever owns those device bytes."""
        import torch

        _ensure_init()
        obj = object.__new__(cls)
        obj.hidden, obj.inter, obj.n_experts, obj.top_k = routed.hidden, routed.inter, routed.n_experts, top_k
        obj.device = torch.cuda.current_device()
        obj._check_device(selector=selector, router=router)
        obj._keep = keepalive
        obj.has_router = router is not None
        d = MoeDesc.from_buffer_copy(routed)
        d.top_k, d.normalize = top_k, int(normalize)
        if shared:
            d.shared_gate_dtype, d.shared_down_dtype = shared[0].ggml_dtype, shared[2].ggml_dtype
            d.shared_gate, d.shared_up, d.shared_down = (m.device_ptr() for m in shared)
            d.selector = selector.data_ptr()
        d.router = None if router is None else router.data_ptr()
        h = ctypes.c_void_p()
        check(lib().iq_moe_create(ctypes.byref(d), ctypes.byref(h)))
        obj._h = h
        return obj

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and _lib._lib is not None:
            _lib._lib.iq_moe_destroy(h)
            self._h = None

    def _check_device(self, **tensors) -> None:
        """Every tensor handed to the C ABI must live in this layer's HBM:
        a host pointer would reach the kernels as a device address."""
        for name, t in tensors.items():
            if t is None:
                continue
            if not t.is_cuda or t.device.index != self.device:
                raise QgemmError(_lib.IQ_ERR_INVALID, f"MoE {name} must be a tensor on cuda:{self.device} "
                                                      f"(got {t.device})")

    def reserve(self, max_tokens: int) -> None:
        """Size the layer's workspace for calls of up to max_tokens tokens
        (iq_moe_reserve): such calls can then be captured into a graph
        without an eager call first."""
        check(lib().iq_moe_reserve(self._h, int(max_tokens), _stream()))

    def slice_tokens(self) -> int:
        """Tokens one set of the layer's launches serves (iq_moe_slice_tokens);
        wider calls run as consecutive slices."""
        return int(lib().iq_moe_slice_tokens(self._h))

    def set_path(self, path: int) -> None:
        """How grouped calls form the down products (iq_moe_set_path):
        _lib.PATH_AUTO keeps the reference's bits, _lib.PATH_PREFILL_TILES
        takes tile order (within 1e-4, not bitwise)."""
        check(lib().iq_moe_set_path(self._h, int(path)))

    def forward_into(self, xs, router_logits, out, experts=None, weights=None) -> None:
        """Raw call: device f32 xs [m, hidden], logits [m, n_experts], out [m, hidden]."""
        self._check_device(xs=xs, router_logits=router_logits, out=out, experts=experts, weights=weights)
        m = xs.numel() // self.hidden
        check(lib().iq_moe_forward(self._h, xs.data_ptr(), router_logits.data_ptr(), m, out.data_ptr(),
                                   None if experts is None else experts.data_ptr(),
                                   None if weights is None else weights.data_ptr(), _stream()))

    def forward_x_into(self, xs, out, residual=None, experts=None, weights=None) -> None:
        """Raw call of the whole sublayer from x (iq_moe_forward_x): the
        layer's router gives the logits; out = residual + MoE(xs) when a
        residual is given."""
        self._check_device(xs=xs, out=out, residual=residual, experts=experts, weights=weights)
        m = xs.numel() // self.hidden
        check(lib().iq_moe_forward_x(self._h, xs.data_ptr(), m, None if residual is None else residual.data_ptr(),
                                     out.data_ptr(), None if experts is None else experts.data_ptr(),
                                     None if weights is None else weights.data_ptr(), _stream()))

    def forward_timed(self, xs, router_logits, out, events) -> None:
        """forward_into recording 4 hipEvent_t handles around the routing,
        gate/up and down launches (iq_moe_forward_timed)."""
        self._check_device(xs=xs, router_logits=router_logits, out=out)
        m = xs.numel() // self.hidden
        ev = (ctypes.c_void_p * 4)(*events)
        check(lib().iq_moe_forward_timed(self._h, xs.data_ptr(), router_logits.data_ptr(), m, out.data_ptr(),
                                         None, None, ev, _stream()))

    def forward_stage(self, stage: int) -> None:
        """Re-launch one stage of the last call (iq_moe_forward_stage)."""
        check(lib().iq_moe_forward_stage(self._h, stage, _stream()))

    def forward(self, xs, router_logits=None, residual=None) -> QuantizedMoeOutput:
        """src/qwen/quantized_moe.rs:227: the layer output and the routes.
        Without router_logits the layer's router computes them
        (src/qwen/quantized_moe.rs:253); with a residual the output is
        residual + MoE(xs) (src/qwen/quantized_layer.rs:212)."""
        import torch

        if xs.numel() % self.hidden:
            raise QgemmError(_lib.IQ_ERR_SHAPE,
                             f"MoE input element count is not divisible by hidden size {self.hidden}")
        self._check_device(xs=xs, router_logits=router_logits, residual=residual)
        flat = xs.to(torch.float32).reshape(-1, self.hidden).contiguous()
        m = flat.shape[0]
        out = torch.empty_like(flat)
        experts = torch.empty(m, self.top_k, dtype=torch.int32, device=flat.device)
        weights = torch.empty(m, self.top_k, dtype=torch.float32, device=flat.device)
        if router_logits is None:
            res = None if residual is None else residual.to(torch.float32).reshape(m, self.hidden).contiguous()
            self.forward_x_into(flat, out, res, experts, weights)
        else:
            if residual is not None:
                raise QgemmError(_lib.IQ_ERR_INVALID, "a residual goes with the layer's own router (forward_x)")
            logits = router_logits.to(torch.float32).reshape(m, self.n_experts).contiguous()
            self.forward_into(flat, logits, out, experts, weights)
        e, w = experts.cpu().tolist(), weights.cpu().tolist()
        return QuantizedMoeOutput(out.reshape(xs.shape), [Route(a, b) for a, b in zip(e, w)])
