"""Seeded synthetic inputs: numpy PCG64 normals drawn in f64, scaled, rounded
to f32 (RNE); bf16 inputs are the RNE rounding of those f32 values."""
from __future__ import annotations

import numpy as np

# seed per workload: 0 round trip, 1 INT8 GEMV, 2 INT4 GEMV, 3 W8A8, 4 MLP
SEEDS = {"roundtrip": 0, "gemv_w8": 1, "gemv_w4": 2, "w8a8": 3, "mlp": 4}


def normal_f32(seed: int, shape, std: float = 1.0, stream: int = 0) -> np.ndarray:
    """N(0, std^2) as float32; `stream` separates independent tensors of one seed."""
    rng = np.random.Generator(np.random.PCG64([seed, stream]))
    n = int(np.prod(shape))
    return (rng.standard_normal(n) * std).astype(np.float32).reshape(shape)


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """IEEE round-to-nearest-even f32 -> bf16, as uint16 bit patterns."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
