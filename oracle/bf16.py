"""bfloat16 helpers for the CPU oracle (test infrastructure only).

bf16 values are carried as ``uint16`` bit patterns in numpy.  Conversion from
float32 is round-to-nearest-even with NaN mapped to 0x7FC0, which is what torch's
CPU ``BFloat16`` conversion does (c10/util/BFloat16.h ``round_to_nearest_even``);
``tests/test_oracle_bf16.py`` pins it against torch on every float32 class.
"""

from __future__ import annotations

import numpy as np


def to_f32(bits: np.ndarray) -> np.ndarray:
    """uint16 bf16 bits -> float32 (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def from_f32(x: np.ndarray) -> np.ndarray:
    """float32 -> uint16 bf16 bits, round to nearest even, NaN -> 0x7FC0."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded[nan] = 0x7FC0
    return rounded


def round_f32(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bf16 precision, returned as float32."""
    return to_f32(from_f32(x))
