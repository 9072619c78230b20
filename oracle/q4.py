"""Group-wise affine 4-bit quantization oracle (test infrastructure).

Format (MLX "affine" mode, bits=4, as consumed by ``mx.quantized_matmul`` at
``src/ollm/llama_mlx.py:53-74`` with ``transpose=True``; tensor names
``.scales``/``.biases`` at ``llama_mlx.py:484-495``, ``U32`` dtype at
``mlx_loader.py:289,298``):

* ``w``      uint32 ``[N, K/8]``: element ``k`` of row ``n`` is nibble ``k % 8``
  of word ``k // 8``, lowest bits first;
* ``scales`` bf16 ``[N, K/G]`` and ``biases`` bf16 ``[N, K/G]``;
* ``W[n, k] = scales[n, k//G] * q + biases[n, k//G]`` with ``q`` in 0..15;
* ``y = x @ W.T`` accumulated in fp32 (here: float64, then rounded), result in
  the dtype of ``x`` (bf16 -> round-to-nearest-even).
"""
from __future__ import annotations

import numpy as np

from .bf16 import bf16_bits_to_f32, f32_to_bf16_bits

BITS = 4
PER_WORD = 32 // BITS  # 8 nibbles per uint32


def pack(codes: np.ndarray) -> np.ndarray:
    """Pack 4-bit codes ``uint8 [N, K]`` (values 0..15) into ``uint32 [N, K/8]``."""
    codes = np.asarray(codes)
    n, k = codes.shape
    if k % PER_WORD:
        raise ValueError("K must be a multiple of 8 for 4-bit packing")
    if codes.min(initial=0) < 0 or codes.max(initial=0) > 15:
        raise ValueError("4-bit codes must lie in 0..15")
    c = codes.astype(np.uint32).reshape(n, k // PER_WORD, PER_WORD)
    shifts = (np.arange(PER_WORD, dtype=np.uint32) * BITS)[None, None, :]
    return np.bitwise_or.reduce(c << shifts, axis=2).astype(np.uint32)


def unpack(w: np.ndarray) -> np.ndarray:
    """Unpack ``uint32 [N, K/8]`` to codes ``uint8 [N, K]`` (nibble k%8 of word k//8)."""
    w = np.asarray(w, dtype=np.uint32)
    n, kw = w.shape
    shifts = (np.arange(PER_WORD, dtype=np.uint32) * BITS)[None, None, :]
    return ((w[:, :, None] >> shifts) & 0xF).astype(np.uint8).reshape(n, kw * PER_WORD)


def quantize(weight: np.ndarray, group_size: int = 64):
    """Quantize ``float [N, K]`` to (packed u32, scales bf16-bits, biases bf16-bits).

    The build's own fixture quantizer (the reference only consumes
    pre-quantized checkpoints; ``mx.quantize`` is used only in
    ``tests/test_mlx_generation.py:180``).  Per group: ``scale=(max-min)/15``,
    ``bias=min``, both rounded to bf16 first, then
    ``q = clip(rint((w - bias) / scale), 0, 15)``.  Matmul parity is defined on
    the packed triple, so this rounding choice does not affect it.
    """
    w = np.asarray(weight, dtype=np.float32)
    n, k = w.shape
    if k % group_size:
        raise ValueError("K must be divisible by group_size")
    g = w.reshape(n, k // group_size, group_size)
    wmin = g.min(axis=2)
    wmax = g.max(axis=2)
    scale = np.maximum((wmax - wmin) / 15.0, 1e-8).astype(np.float32)
    s_bits = f32_to_bf16_bits(scale)
    b_bits = f32_to_bf16_bits(wmin)
    s = bf16_bits_to_f32(s_bits)
    b = bf16_bits_to_f32(b_bits)
    q = np.rint((g - b[:, :, None]) / s[:, :, None])
    q = np.clip(q, 0, 15).astype(np.uint8).reshape(n, k)
    return pack(q), s_bits, b_bits


def dequantize(w: np.ndarray, scales_bits: np.ndarray, biases_bits: np.ndarray,
               group_size: int = 64) -> np.ndarray:
    """``W[n,k] = s*q + b`` in float64 (exact for bf16 s, b and 4-bit q)."""
    q = unpack(w).astype(np.float64)
    n, k = q.shape
    s = bf16_bits_to_f32(scales_bits).astype(np.float64)
    b = bf16_bits_to_f32(biases_bits).astype(np.float64)
    if s.shape != (n, k // group_size) or b.shape != s.shape:
        raise ValueError("scales/biases must have shape [N, K/group_size]")
    return (q.reshape(n, k // group_size, group_size) * s[:, :, None]
            + b[:, :, None]).reshape(n, k)


def quantized_matmul(x: np.ndarray, w: np.ndarray, scales_bits: np.ndarray,
                     biases_bits: np.ndarray, group_size: int = 64,
                     bits: int = 4, mode: str = "affine") -> np.ndarray:
    """``y = x @ dequant(W).T`` (restates ``llama_mlx.py:53-74``).

    ``x`` is float32 (bf16 inputs are passed already widened).  Returns the
    float32 result of a float64 accumulation; callers round to bf16 when the
    activation dtype is bf16.
    """
    if bits != 4 or mode != "affine":
        raise ValueError("only 4-bit affine quantization is supported")
    x = np.asarray(x, dtype=np.float64)
    wd = dequantize(w, scales_bits, biases_bits, group_size)
    if x.shape[-1] != wd.shape[1]:
        raise ValueError("x last dim must equal K")
    return (x @ wd.T).astype(np.float32)


def linear_bytes(n: int, k: int, group_size: int = 64, m: int = 1) -> int:
    """Algorithmic HBM bytes of one q4 linear at batch m with bf16 activations."""
    return n * k // 2 + 2 * (n * (k // group_size)) * 2 + 2 * k * m + 2 * n * m
