"""float32 <-> bfloat16 in numpy, round to nearest even.

The reference obtains bfloat16 from ml_dtypes (reference
autotune/src/autotune/runner/types.py:17-30), which rounds to nearest even.
ml_dtypes is absent here, so this restates the rounding on the bit pattern:
add 0x7FFF plus the lowest kept bit, truncate the low 16 bits; every NaN
becomes the canonical quiet NaN 0x7FC0.
"""

from __future__ import annotations

import numpy as np


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """bfloat16 bit patterns (uint16) of float32 ``x``, RNE."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        rounded = np.where(nan, np.uint16(0x7FC0), rounded)
    return rounded


def from_bf16_bits(b: np.ndarray) -> np.ndarray:
    """float32 values of bfloat16 bit patterns."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """``x`` rounded to the nearest bfloat16, returned as float32."""
    return from_bf16_bits(to_bf16_bits(x))
