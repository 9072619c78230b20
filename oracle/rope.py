"""RoPE oracle (test infrastructure).

Restates ``MLXRotaryEmbedding`` (``src/ollm/llama_mlx.py:95-146``) and
``apply_rotary_pos_emb_mlx``/``rotate_half`` (``llama_mlx.py:149-182``;
compiled twin ``metal_optimizations.py:70-118``): non-interleaved
"rotate-half" RoPE, ``inv_freq[i] = 1/theta^(2i/D)``, ``emb = [f, f]``.

Numerical contract shared bit-for-bit with the HIP kernels:

* ``inv_freq`` and ``cos``/``sin`` are evaluated in float64 and rounded once
  to float32 (the angle itself is ``fp32(fp32(pos) * inv_freq)``, a single
  float32 product as in ``mx.outer``);
* ``out = fp32(x*cos) + fp32(rot*sin)`` with each product and the sum rounded
  to float32 separately (no fused multiply-add), as ``(q * cos) +
  (rotate_half(q) * sin)`` evaluates in MLX.
"""
from __future__ import annotations

import numpy as np


def inv_freq(dim: int, theta: float) -> np.ndarray:
    i = np.arange(0, dim, 2, dtype=np.float64)
    return (1.0 / np.power(np.float64(theta), i / dim)).astype(np.float32)


def cos_sin(positions: np.ndarray, dim: int, theta: float):
    """cos/sin ``float32 [B, L, D]`` for integer positions ``[B, L]``."""
    pos = np.asarray(positions).astype(np.float32)
    inv = inv_freq(dim, theta)
    ang = (pos[..., None] * inv).astype(np.float32)           # [B, L, D/2]
    c = np.cos(ang.astype(np.float64)).astype(np.float32)
    s = np.sin(ang.astype(np.float64)).astype(np.float32)
    return np.concatenate([c, c], axis=-1), np.concatenate([s, s], axis=-1)


def rotate_half(x: np.ndarray) -> np.ndarray:
    x1, x2 = np.split(x, 2, axis=-1)
    return np.concatenate([-x2, x1], axis=-1)


def apply(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Rotate ``x [B, H, L, D]`` (float32) with cos/sin ``[B, L, D]``."""
    x = np.asarray(x, dtype=np.float32)
    c = cos[:, None, :, :].astype(np.float32)
    s = sin[:, None, :, :].astype(np.float32)
    a = (x * c).astype(np.float32)
    b = (rotate_half(x) * s).astype(np.float32)
    return (a + b).astype(np.float32)
