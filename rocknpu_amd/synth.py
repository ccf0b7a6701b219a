"""Deterministic synthetic GGUF K-quant weights and activations.

Every tensor comes from numpy's PCG64 seeded with (SEED_BASE, tensor index),
so the same index gives the same bytes on every machine. Distributions follow
the benchmark configurations: Q4_K blocks carry fp16 d and dmin ~ |N(0, 0.01)|,
eight 6-bit scales and eight 6-bit mins uniform in [0, 63] and 4-bit quants
uniform in [0, 15]; Q6_K blocks carry 6-bit quants uniform in [0, 63], sixteen
int8 scales uniform in [-63, 63] and fp16 d ~ |N(0, 0.01)|; Q5_K adds a uniform
fifth bit to the Q4_K layout; activations are f32 N(0, 1).
"""
from __future__ import annotations

import numpy as np

SEED_BASE = 0x524F434B4E5055  # "ROCKNPU"
QK = 256
BLOCK_BYTES = {4: 144, 5: 176, 6: 210}
Q8K_BYTES = 292

# TinyLlama-1.1B projection shapes (name, k, n, kind): ggml weight [n rows x k].
TINYLLAMA_LAYER = (
    ("q", 2048, 2048, 4),
    ("k", 2048, 256, 4),
    ("v", 2048, 256, 4),
    ("o", 2048, 2048, 4),
    ("gate", 2048, 5632, 4),
    ("up", 2048, 5632, 4),
    ("down", 5632, 2048, 6),
)
TINYLLAMA_LAYERS = 22


def rng(index: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64([SEED_BASE, index]))


def _f16_bytes(values: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(values.astype(np.float16)).view(np.uint8).reshape(-1, 2)


def pack_scales_k4(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """Pack eight 6-bit scales and mins per block into the 12-byte K-quant field."""
    sc = sc.astype(np.uint8)
    mn = mn.astype(np.uint8)
    out = np.empty((sc.shape[0], 12), np.uint8)
    out[:, 0:4] = (sc[:, :4] & 63) | ((sc[:, 4:] >> 4) << 6)
    out[:, 4:8] = (mn[:, :4] & 63) | ((mn[:, 4:] >> 4) << 6)
    out[:, 8:12] = (sc[:, 4:] & 0xF) | ((mn[:, 4:] & 0xF) << 4)
    return out


def q4_k(n: int, k: int, index: int) -> np.ndarray:
    """n rows of k values as Q4_K blocks, flat uint8 of n*(k/256)*144 bytes."""
    assert k % QK == 0
    nbt = n * (k // QK)
    g = rng(index)
    blk = np.empty((nbt, 144), np.uint8)
    blk[:, 0:2] = _f16_bytes(np.abs(g.normal(0.0, 0.01, nbt)))
    blk[:, 2:4] = _f16_bytes(np.abs(g.normal(0.0, 0.01, nbt)))
    blk[:, 4:16] = pack_scales_k4(g.integers(0, 64, (nbt, 8)), g.integers(0, 64, (nbt, 8)))
    blk[:, 16:] = g.integers(0, 256, (nbt, 128), dtype=np.uint8)
    return blk.reshape(-1)


def q5_k(n: int, k: int, index: int) -> np.ndarray:
    assert k % QK == 0
    nbt = n * (k // QK)
    g = rng(index)
    blk = np.empty((nbt, 176), np.uint8)
    blk[:, 0:2] = _f16_bytes(np.abs(g.normal(0.0, 0.01, nbt)))
    blk[:, 2:4] = _f16_bytes(np.abs(g.normal(0.0, 0.01, nbt)))
    blk[:, 4:16] = pack_scales_k4(g.integers(0, 64, (nbt, 8)), g.integers(0, 64, (nbt, 8)))
    blk[:, 16:] = g.integers(0, 256, (nbt, 160), dtype=np.uint8)
    return blk.reshape(-1)


def q6_k(n: int, k: int, index: int) -> np.ndarray:
    assert k % QK == 0
    nbt = n * (k // QK)
    g = rng(index)
    blk = np.empty((nbt, 210), np.uint8)
    blk[:, 0:192] = g.integers(0, 256, (nbt, 192), dtype=np.uint8)
    blk[:, 192:208] = g.integers(-63, 64, (nbt, 16)).astype(np.int8).view(np.uint8)
    blk[:, 208:210] = _f16_bytes(np.abs(g.normal(0.0, 0.01, nbt)))
    return blk.reshape(-1)


def kquant(kind: int, n: int, k: int, index: int) -> np.ndarray:
    return {4: q4_k, 5: q5_k, 6: q6_k}[kind](n, k, index)


def activations(m: int, k: int, index: int) -> np.ndarray:
    return rng(index).standard_normal((m, k), dtype=np.float32)
