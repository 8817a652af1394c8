"""Writes tests/golden/tiny_moe.gguf: two MoE layers (2 experts, hidden 256,
intermediate 256; Q4_K gate/up, Q6_K down, shared expert, F32 router and
selector) from seeded synthetic blocks, with layer 1's tensors stored before
layer 0's so that file order differs from layer order.

Run from the repository root: python tests/golden/make_gguf.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, HERE]

from gguf_writer import moe_layer_tensors, write_gguf  # noqa: E402
from inferq_amd import synth as S  # noqa: E402

SEED = 20261202


def build(path):
    rng = np.random.default_rng(SEED)
    layers = []
    for _ in range(2):
        lay = S.random_moe_layer(256, 256, 2, S.Q4_K, S.Q6_K, rng, shared=True)
        router = rng.standard_normal((2, 256), dtype=np.float32) / np.float32(16)
        layers.append((lay, router))
    tensors = moe_layer_tensors(1, *layers[1]) + moe_layer_tensors(0, *layers[0])
    meta = {"general.architecture": "qwen3moe", "qwen3moe.block_count": 2, "qwen3moe.expert_count": 2,
            "qwen3moe.expert_used_count": 1, "qwen3moe.embedding_length": 256,
            "qwen3moe.expert_feed_forward_length": 256, "general.name": "inferq-amd tiny MoE fixture"}
    return write_gguf(path, tensors, meta), layers


if __name__ == "__main__":
    out = os.path.join(HERE, "tiny_moe.gguf")
    build(out)
    print(out, os.path.getsize(out))
