"""bf16 helpers for the oracle (test infrastructure only).

bf16 values are carried as uint16 bit patterns.  f32 -> bf16 is
round-to-nearest-even, NaN kept quiet, exactly as the device helper
`f32_to_bf16_bits`.  Pinned by tests/test_oracle_core.py against
torch.Tensor.to(torch.bfloat16) on the CPU (an independent implementation)
over random, tie and special values.
"""

from __future__ import annotations

import numpy as np


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 array -> uint16 bf16 bits (round to nearest even)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    is_nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x007FFFFF) != 0)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    r = np.where(is_nan, (u >> 16) | 0x40, r)
    return (r & 0xFFFF).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    """uint16 bf16 bits -> float32."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 value, returned as float32."""
    return bf16_to_f32(f32_to_bf16(x))


def normal_bf16(rng: np.random.Generator, shape, std: float = 1.0) -> np.ndarray:
    """N(0, std^2) samples rounded to bf16, as uint16 bits."""
    return f32_to_bf16((rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32))
