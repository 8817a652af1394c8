"""Seeded synthetic GGUF block data and activations.

Weights are random bytes in the native GGUF block layouts, drawn so that
every block is a valid, finite block:
  * Q4_K (144 B): fp16 d and dmin ~ U[0, 2^-6); 12 scale bytes and 128 quant
    bytes uniform u8.
  * Q5_K (176 B): as Q4_K, plus 32 high-bit bytes uniform u8.
  * Q6_K (210 B): ql, qh uniform u8; 16 scales uniform i8; fp16 d ~ U[0, 2^-6).
  * Q8_0 (34 B): fp16 d = |N(0,1)| * 0.02; 32 quants uniform in [-127, 127].
Activations and router logits are f32 ~ N(0, 1).
"""
from __future__ import annotations

import numpy as np

Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14
BLOCK_BYTES = {Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_0: 34}
BLOCK_ELEMS = {Q4_K: 256, Q5_K: 256, Q6_K: 256, Q8_0: 32}
NAMES = {Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", Q8_0: "Q8_0"}


def row_bytes(dtype: int, cols: int) -> int:
    if cols % BLOCK_ELEMS[dtype]:
        raise ValueError(f"{NAMES[dtype]} needs a width divisible by {BLOCK_ELEMS[dtype]}, got {cols}")
    return cols // BLOCK_ELEMS[dtype] * BLOCK_BYTES[dtype]


def matrix_bytes(dtype: int, rows: int, cols: int) -> int:
    return rows * row_bytes(dtype, cols)


def _f16_bits(values: np.ndarray) -> np.ndarray:
    return values.astype(np.float16).view(np.uint16)


def random_blocks(dtype: int, n_blocks: int, rng: np.random.Generator) -> np.ndarray:
    """n_blocks random blocks as a flat uint8 array."""
    bb = BLOCK_BYTES[dtype]
    raw = rng.integers(0, 256, size=(n_blocks, bb), dtype=np.uint8)
    if dtype in (Q4_K, Q5_K):
        d = _f16_bits(rng.random(n_blocks, dtype=np.float32) * np.float32(2.0 ** -6))
        dmin = _f16_bits(rng.random(n_blocks, dtype=np.float32) * np.float32(2.0 ** -6))
        raw[:, 0:2] = d.view(np.uint8).reshape(n_blocks, 2)
        raw[:, 2:4] = dmin.view(np.uint8).reshape(n_blocks, 2)
    elif dtype == Q6_K:
        d = _f16_bits(rng.random(n_blocks, dtype=np.float32) * np.float32(2.0 ** -6))
        raw[:, 208:210] = d.view(np.uint8).reshape(n_blocks, 2)
    elif dtype == Q8_0:
        d = _f16_bits(np.abs(rng.standard_normal(n_blocks, dtype=np.float32)) * np.float32(0.02))
        raw[:, 0:2] = d.view(np.uint8).reshape(n_blocks, 2)
        raw[:, 2:34] = rng.integers(-127, 128, size=(n_blocks, 32), dtype=np.int8).view(np.uint8)
    else:
        raise ValueError(f"unsupported dtype {dtype}")
    return raw.reshape(-1)


def random_matrix(dtype: int, rows: int, cols: int, rng: np.random.Generator) -> np.ndarray:
    """A [rows x cols] matrix of random GGUF blocks (flat uint8)."""
    return random_blocks(dtype, rows * (cols // BLOCK_ELEMS[dtype]), rng)


def normal(shape, rng: np.random.Generator) -> np.ndarray:
    return rng.standard_normal(shape, dtype=np.float32)


def random_moe_layer(hidden: int, inter: int, n_experts: int, gate_dtype: int, down_dtype: int,
                     rng: np.random.Generator, shared: bool = True) -> dict:
    """Byte arrays of one MoE sublayer in GGUF expert-tensor layout:
    gate/up [E, inter, hidden], down [E, hidden, inter], the shared expert
    (gate/up [inter, hidden], down [hidden, inter]) and the f32 selector
    ~ N(0,1)/sqrt(hidden)."""
    layer = {
        "hidden": hidden, "inter": inter, "n_experts": n_experts,
        "gate_dtype": gate_dtype, "down_dtype": down_dtype,
        "gate": random_matrix(gate_dtype, n_experts * inter, hidden, rng),
        "up": random_matrix(gate_dtype, n_experts * inter, hidden, rng),
        "down": random_matrix(down_dtype, n_experts * hidden, inter, rng),
    }
    if shared:
        layer.update({
            "shared_gate_dtype": gate_dtype, "shared_down_dtype": down_dtype,
            "shared_gate": random_matrix(gate_dtype, inter, hidden, rng),
            "shared_up": random_matrix(gate_dtype, inter, hidden, rng),
            "shared_down": random_matrix(down_dtype, hidden, inter, rng),
            "selector": (rng.standard_normal(hidden, dtype=np.float32) / np.float32(np.sqrt(hidden))),
        })
    return layer


def random_blocks_device(dtype: int, n_blocks: int, device, seed: int):
    """random_blocks drawn on the GPU (same distributions, different stream
    of numbers): a flat CUDA uint8 tensor of n_blocks blocks."""
    import torch

    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    bb = BLOCK_BYTES[dtype]
    raw = torch.randint(0, 256, (n_blocks, bb), dtype=torch.uint8, device=device, generator=gen)

    def f16_bytes(values):
        return values.to(torch.float16).view(torch.uint8).reshape(n_blocks, 2)

    if dtype in (Q4_K, Q5_K):
        raw[:, 0:2] = f16_bytes(torch.rand(n_blocks, device=device, generator=gen) * 2.0 ** -6)
        raw[:, 2:4] = f16_bytes(torch.rand(n_blocks, device=device, generator=gen) * 2.0 ** -6)
    elif dtype == Q6_K:
        raw[:, 208:210] = f16_bytes(torch.rand(n_blocks, device=device, generator=gen) * 2.0 ** -6)
    elif dtype == Q8_0:
        raw[:, 0:2] = f16_bytes(torch.randn(n_blocks, device=device, generator=gen).abs() * 0.02)
        q = torch.randint(-127, 128, (n_blocks, 32), dtype=torch.int8, device=device, generator=gen)
        raw[:, 2:34] = q.view(torch.uint8)
    else:
        raise ValueError(f"unsupported dtype {dtype}")
    return raw.reshape(-1)


def random_matrix_device(dtype: int, rows: int, cols: int, device, seed: int):
    return random_blocks_device(dtype, rows * (cols // BLOCK_ELEMS[dtype]), device, seed)
