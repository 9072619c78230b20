"""bfloat16 <-> float32 conversions used by the oracle (test infrastructure).

bf16 values are carried as ``uint16`` arrays holding the upper 16 bits of an
IEEE float32.  Rounding float32 -> bf16 is round-to-nearest-even with NaNs
kept quiet, the same rule MLX and torch apply when an array is cast with
``astype(bfloat16)`` (the reference casts at ``mlx_ops.py:146-147`` and
``backends/cpu_reference.py:371-384``).
"""
from __future__ import annotations

import numpy as np


def f32_to_bf16_bits(x) -> np.ndarray:
    """Round float32 values to bf16 (RNE); return their uint16 bit patterns."""
    f = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    rounding = ((u >> 16) & 1) + 0x7FFF
    out = ((u + rounding) >> 16).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        out = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), out)
    return out


def bf16_bits_to_f32(b) -> np.ndarray:
    """Widen bf16 bit patterns (uint16) to float32 exactly."""
    b = np.ascontiguousarray(np.asarray(b, dtype=np.uint16))
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(x) -> np.ndarray:
    """float32 -> bf16 -> float32 (the value a bf16 tensor would hold)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))
