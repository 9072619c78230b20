"""Pins the oracle's bf16 rounding and q4 format/matmul (CPU only)."""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import q4
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16

ROOT = Path(__file__).resolve().parent.parent


def test_bf16_rounding_matches_torch_cast():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.normal(0, 1, 10000), rng.normal(0, 1e30, 100), rng.normal(0, 1e-30, 100),
                        [0.0, -0.0, np.inf, -np.inf, 1.0 + 2**-8, 1.0 + 3 * 2**-8, 65504.0]]).astype(np.float32)
    ours = f32_to_bf16_bits(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    assert np.isnan(round_bf16(np.array([np.nan], np.float32)))[0]


def test_pack_unpack_brute_force_and_roundtrip():
    # closed-form rule on a tiny case: element k of row n is nibble k%8 of word k//8
    codes = np.array([[1, 2, 3, 4, 5, 6, 7, 8, 15, 0, 0, 0, 0, 0, 0, 9]], dtype=np.uint8)
    w = q4.pack(codes)
    assert w.dtype == np.uint32 and w.shape == (1, 2)
    assert w[0, 0] == 0x87654321 and w[0, 1] == 0x9000000F
    rng = np.random.default_rng(2)
    words = rng.integers(0, 2**32, size=(7, 16), dtype=np.uint64).astype(np.uint32)
    assert np.array_equal(q4.pack(q4.unpack(words)), words)
    un = q4.unpack(words)
    for n in range(7):
        for k in range(128):
            assert un[n, k] == (int(words[n, k // 8]) >> (4 * (k % 8))) & 15


def _dense_scalar(w, s, b, G):
    """Scalar-loop dequantization (independent of q4.dequantize's vectorization)."""
    n, kw = w.shape
    out = np.zeros((n, kw * 8))
    sf, bf = bf16_bits_to_f32(s), bf16_bits_to_f32(b)
    for i in range(n):
        for k in range(kw * 8):
            q = (int(w[i, k // 8]) >> (4 * (k % 8))) & 15
            out[i, k] = float(sf[i, k // G]) * q + float(bf[i, k // G])
    return out


def test_quantized_matmul_matches_torch_float64_of_scalar_dequant():
    rng = np.random.default_rng(3)
    N, K, G = 12, 128, 64
    w, s, b = q4.quantize(rng.normal(0, 0.02, (N, K)).astype(np.float32), G)
    x = rng.normal(0, 1, (3, K)).astype(np.float32)
    dense = _dense_scalar(w, s, b, G)
    ref = (torch.from_numpy(x).double() @ torch.from_numpy(dense).T).numpy()
    got = q4.quantized_matmul(x, w, s, b, G)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-7)


def test_quantized_matmul_invariants():
    rng = np.random.default_rng(4)
    N, K, G = 8, 256, 64
    zero = np.zeros((N, K // 8), np.uint32)
    s = f32_to_bf16_bits(rng.uniform(0.01, 0.1, (N, K // G)).astype(np.float32))
    b = f32_to_bf16_bits(rng.normal(0, 0.1, (N, K // G)).astype(np.float32))
    x = rng.normal(0, 1, (2, K)).astype(np.float32)
    # all-zero codes: y = sum_g bias_g * sum_{k in g} x_k
    expect = np.einsum("mgk,ng->mn", x.reshape(2, K // G, G).astype(np.float64),
                       bf16_bits_to_f32(b).astype(np.float64))
    np.testing.assert_allclose(q4.quantized_matmul(x, zero, s, b, G), expect, rtol=1e-6, atol=1e-6)
    # one-hot x picks column k: y[n] = s*q[n,k] + b
    w = rng.integers(0, 2**32, size=(N, K // 8), dtype=np.uint64).astype(np.uint32)
    k = 77
    onehot = np.zeros((1, K), np.float32)
    onehot[0, k] = 1.0
    col = q4.unpack(w)[:, k] * bf16_bits_to_f32(s)[:, k // G] + bf16_bits_to_f32(b)[:, k // G]
    np.testing.assert_allclose(q4.quantized_matmul(onehot, w, s, b, G)[0], col, rtol=1e-6)
    # linearity in x
    x2 = rng.normal(0, 1, (2, K)).astype(np.float32)
    lhs = q4.quantized_matmul(2 * x - 3 * x2, w, s, b, G)
    rhs = 2 * q4.quantized_matmul(x, w, s, b, G) - 3 * q4.quantized_matmul(x2, w, s, b, G)
    np.testing.assert_allclose(lhs, rhs, rtol=1e-4, atol=1e-4)


def test_quantizer_reconstruction_error_bounded():
    rng = np.random.default_rng(5)
    wf = rng.normal(0, 0.02, (16, 512)).astype(np.float32)
    w, s, b = q4.quantize(wf, 64)
    deq = q4.dequantize(w, s, b, 64)
    step = bf16_bits_to_f32(s).repeat(64, axis=1)
    assert np.all(np.abs(deq - wf) <= 0.5 * step * 1.02 + 2e-4)


def test_rejects_bad_quantization_parameters():
    w = np.zeros((1, 8), np.uint32)
    s = np.zeros((1, 1), np.uint16)
    with pytest.raises(ValueError):
        q4.quantized_matmul(np.zeros((1, 64), np.float32), w, s, s, 64, bits=8)
    with pytest.raises(ValueError):
        q4.quantize(np.zeros((2, 65), np.float32), 64)


def test_c_oracle_matches_numpy_oracle():
    so = ROOT / "oracle" / "libstrata_oracle.so"
    if not so.exists():
        pytest.skip("C oracle not built (make -C oracle/c)")
    lib = C.CDLL(str(so))
    rng = np.random.default_rng(6)
    N, K, M = 40, 256, 2
    w, s, b = q4.quantize(rng.normal(0, 0.02, (N, K)).astype(np.float32), 64)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    y = np.zeros((M, N), np.float32)
    P = C.c_void_p
    lib.oracle_q4_matmul(x.ctypes.data_as(P), C.c_int64(M), C.c_int64(K), w.ctypes.data_as(P),
                         s.ctypes.data_as(P), b.ctypes.data_as(P), C.c_int64(N), C.c_int(64),
                         y.ctypes.data_as(P))
    np.testing.assert_allclose(y, q4.quantized_matmul(x, w, s, b), rtol=1e-4, atol=1e-4)
