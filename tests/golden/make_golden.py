"""Write tests/golden/qgemm_golden.npz: small seeded fixtures of the quantised
matmul path (weights, inputs, quantised activations, products, per-block lane
integers, routes, one MoE sublayer).

source = the oracle (oracle/, a restatement of the reference read as text);
the reference itself commits no golden vectors and needs Rust + candle, which
this image lacks, so these are regression fixtures for both the oracle and
the GPU kernels, not an independent pin.  Run from the repository root:

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from inferq_amd import synth  # noqa: E402
from oracle import oracle as O  # noqa: E402

OUT = os.path.join(HERE, "qgemm_golden.npz")
ROWS = (1, 2, 4, 8, 9, 16)
SHAPES = {O.Q4_K: (32, 1024), O.Q6_K: (32, 512), O.Q8_0: (64, 512)}


def quant_rows(k: int, rng: np.random.Generator) -> np.ndarray:
    """Activation rows that exercise from_float's edge cases."""
    rows = [
        np.zeros(k, np.float32),
        rng.standard_normal(k, dtype=np.float32),
        np.where(np.arange(k) == 3, np.float32(-2.5), np.float32(0.0)),
        np.tile(np.float32([0.75, -0.75]), k // 2),
        (np.arange(k, dtype=np.float32) - k / 2) / 64,
    ]
    return np.stack(rows).astype(np.float32)


def main() -> None:
    rng = np.random.default_rng(8080)
    data = {"source": np.array("oracle restatement (no reference import)")}
    for dt, (n, k) in SHAPES.items():
        name = synth.NAMES[dt]
        w = synth.random_matrix(dt, n, k, rng)
        x = synth.normal((max(ROWS), k), rng)
        data[f"{name}_w"] = w
        data[f"{name}_x"] = x
        data[f"{name}_shape"] = np.array([n, k])
        for m in ROWS:
            data[f"{name}_y_m{m}"] = O.matmul(dt, w, n, k, x[:m])
        q = O.quantize_q80(x[0]) if dt == O.Q8_0 else O.quantize_q8k(x[0])
        wb = w.view(O.BLOCK[dt]).reshape(n, -1)
        isum = np.zeros((n, wb.shape[1], 8), np.int32)
        msum = np.zeros((n, wb.shape[1], 4), np.int32)
        for r in range(n):
            for b in range(wb.shape[1]):
                i, mm = O.block_lanes(dt, wb[r, b], q[b])
                isum[r, b] = i
                if mm is not None:
                    msum[r, b] = mm
        data[f"{name}_isum_m1"] = isum
        if dt == O.Q4_K:
            data[f"{name}_msum_m1"] = msum
    qx = quant_rows(512, rng)
    data["quant_x"] = qx
    data["quant_q8k"] = np.concatenate([O.quantize_q8k(r) for r in qx]).view(np.uint8)
    data["quant_q80"] = np.concatenate([O.quantize_q80(r) for r in qx]).view(np.uint8)
    logits = np.concatenate([np.float32([[1, 4, 2, 3, 0, 0, 0, 0]]), synth.normal((3, 8), rng)])
    e, wts = O.top_k_routes(logits, 2, True)
    data["route_logits"], data["route_experts"], data["route_weights"] = logits, e, wts
    layer = synth.random_moe_layer(256, 256, 4, O.Q4_K, O.Q6_K, rng, shared=True)
    for key in ("gate", "up", "down", "shared_gate", "shared_up", "shared_down", "selector"):
        data[f"moe_{key}"] = layer[key]
    layer.update(top_k=2, normalize=True)
    mx = synth.normal((3, 256), rng)
    ml = synth.normal((3, 4), rng)
    out, me, mw = O.moe_forward(layer, mx, ml, mode=1)
    data.update(moe_x=mx, moe_logits=ml, moe_out=out, moe_experts=me, moe_weights=mw)
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
