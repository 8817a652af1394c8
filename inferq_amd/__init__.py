"""inferq_amd -- MI355X (gfx950) quantised-matmul hot path of inferq.

GGUF Q8_0 / Q4_K / Q6_K matrices stay resident in HBM in their native block
layout; hand-written HIP kernels compute the dense projections, the grouped
MoE experts and the LM head with the reference CPU kernels' exact
arithmetic.  The product is libiq_qgemm.so and its C ABI
(include/iq_qgemm.h); this package is its Python host mirror.
"""
from ._lib import IQ_Q4_K, IQ_Q6_K, IQ_Q8_0, QgemmError, lib  # noqa: F401

__all__ = ["IQ_Q4_K", "IQ_Q6_K", "IQ_Q8_0", "QgemmError", "lib"]
