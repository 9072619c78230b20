"""Pins the oracle functions that no reference fixture covers (CPU only).

Each check is independent of the oracle's own formula: torch's fp32 kernels,
float64 closed forms, brute force, or the float64 softmax attention.  Each
is chosen so that a plausible slip fails it: a dropped eps, sum instead of
mean, sqrt for rsqrt, the weight left out, sigmoid(-g), a transposed head
mapping, a missing 1/sqrt(D), a wrong nibble order or a wrong group index.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import llama as oll
from oracle import q4 as oq
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

ROOT = Path(__file__).resolve().parents[1]
P = C.c_void_p


def _bf16(x):
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(x, np.float32)))


def _ulps_bf16(a, b):
    """Distance in bf16 units in the last place between two bf16-valued arrays."""
    ia = f32_to_bf16_bits(a).astype(np.int32)
    ib = f32_to_bf16_bits(b).astype(np.int32)
    # map the sign-magnitude bit patterns onto a monotone integer line
    ia = np.where(ia & 0x8000, 0x8000 - ia, ia)
    ib = np.where(ib & 0x8000, 0x8000 - ib, ib)
    return np.abs(ia - ib)


# ---------------------------------------------------------------- RMSNorm
@pytest.mark.parametrize("H,eps", [(64, 1e-6), (3072, 1e-5), (4096, 1e-5)])
def test_rms_norm_against_torch_and_float64(H, eps):
    """llama_mlx.py:77-92 / metal_optimizations.py:76-96: w * x * rsqrt(mean(x^2) + eps)."""
    rng = np.random.default_rng(H)
    x = _bf16(rng.normal(0, 1.5, (5, H)))
    x[0] *= 40.0  # large dynamic range row
    x[1, : H // 2] = 0.0
    w_bits = f32_to_bf16_bits(rng.normal(1.0, 0.3, H).astype(np.float32))
    w = bf16_bits_to_f32(w_bits)
    got = oll.rms_norm(x, w_bits, eps)

    # (1) torch's own fp32 rms_norm, rounded once to bf16
    tt = torch.nn.functional.rms_norm(torch.from_numpy(x), (H,), torch.from_numpy(w), eps)
    ref_t = tt.to(torch.bfloat16).float().numpy()
    assert _ulps_bf16(got, ref_t).max() <= 1
    assert (got != ref_t).mean() < 0.01

    # (2) float64 closed form in the reference's operand order (w*x)*rsqrt(var+eps)
    x64 = x.astype(np.float64)
    ref64 = (w.astype(np.float64) * x64) / np.sqrt(np.mean(x64 * x64, -1, keepdims=True) + eps)
    assert _ulps_bf16(got, ref64.astype(np.float32)).max() <= 1

    # (3) eps is inside the root: an all-zero row gives 0, a tiny row is not blown up to 1
    z = np.zeros((1, H), np.float32)
    assert np.all(oll.rms_norm(z, w_bits, eps) == 0)
    tv = float(_bf16([1e-4])[0])
    tiny = oll.rms_norm(np.full((1, H), tv, np.float32), w_bits, eps)
    expect = _bf16(w * tv / np.sqrt(tv * tv + eps))[None]
    np.testing.assert_allclose(tiny, expect, rtol=8e-3)


def test_rms_norm_unit_rms_row_is_weight():
    H = 256
    x = np.where(np.arange(H) % 2 == 0, 1.0, -1.0).astype(np.float32)[None]
    w_bits = f32_to_bf16_bits(np.linspace(-2, 2, H).astype(np.float32))
    got = oll.rms_norm(x, w_bits, 0.0)
    np.testing.assert_array_equal(got[0], bf16_bits_to_f32(w_bits) * x[0])


# ---------------------------------------------------------------- SiLU * up
def test_silu_mul_against_torch_and_closed_forms():
    """llama_mlx.py:399-407: gate * sigmoid(gate) * up."""
    rng = np.random.default_rng(11)
    g = _bf16(np.concatenate([rng.normal(0, 3, 4000), [-1000, -100, -20, 0, 20, 100, 1000]]))
    u = _bf16(rng.normal(0, 2, g.shape))
    got = oll.silu_mul(g, u)
    ref = (torch.nn.functional.silu(torch.from_numpy(g)) * torch.from_numpy(u)).to(
        torch.bfloat16).float().numpy()
    assert _ulps_bf16(got, ref).max() <= 1
    assert (got != ref).mean() < 0.01
    # closed forms: silu(0) = 0, silu(g) -> g for large g, -> 0 for very negative g
    i0 = np.where(g == 0)[0][0]
    assert got[i0] == 0
    big = g >= 20
    np.testing.assert_allclose(got[big], _bf16(g[big] * u[big]), rtol=1e-2)
    assert np.all(np.abs(got[g <= -100]) < 1e-30)
    # silu is not odd: silu(-2) = -2*sigmoid(-2) ~ -0.2384
    assert abs(float(oll.silu_mul(np.array([-2.0], np.float32), np.ones(1, np.float32))[0])
               + 0.2384) < 2e-3


# ---------------------------------------------------------------- C oracle
@pytest.fixture(scope="module")
def clib():
    so = ROOT / "oracle" / "libstrata_oracle.so"
    if not so.exists():
        pytest.skip("oracle/libstrata_oracle.so not built (make -C oracle/c)")
    return C.CDLL(str(so))


@pytest.mark.parametrize("B,Hq,Hkv,L", [(1, 12, 4, 1), (2, 8, 2, 37), (1, 24, 8, 1024),
                                         (2, 16, 4, 513), (1, 4, 1, 8192)])
def test_c_decode_attention_against_float64_softmax(clib, B, Hq, Hkv, L):
    """oracle_decode_attn (C) against tests/test_mlx_attention.py:17-40's dense softmax."""
    D = 128
    rng = np.random.default_rng(B * 1000 + L)
    q = rng.normal(0, 1, (B, Hq, D)).astype(np.float32)
    kb = f32_to_bf16_bits(rng.normal(0, 1, (B, Hkv, L, D)).astype(np.float32))
    vb = f32_to_bf16_bits(rng.normal(0, 1, (B, Hkv, L, D)).astype(np.float32))
    out = np.zeros((B, Hq, D), np.float32)
    clib.oracle_decode_attn(q.ctypes.data_as(P), kb.ctypes.data_as(P), vb.ctypes.data_as(P),
                            B, Hq, Hkv, L, D, out.ctypes.data_as(P))
    ref = oatt.naive_gqa(q[:, :, None, :], bf16_bits_to_f32(kb), bf16_bits_to_f32(vb))[:, :, 0]
    err = np.abs(out - ref).max() / max(np.abs(ref).max(), 1e-6)
    assert err < 1e-4, err
    # and against torch's fp64 SDPA with GQA head expansion
    G = Hq // Hkv
    kt = torch.from_numpy(bf16_bits_to_f32(kb)).double().repeat_interleave(G, 1)
    vt = torch.from_numpy(bf16_bits_to_f32(vb)).double().repeat_interleave(G, 1)
    sd = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q).double()[:, :, None], kt, vt)[:, :, 0].numpy()
    assert np.abs(out - sd).max() / np.abs(sd).max() < 1e-4


def _q4_case(N, K, seed):
    rng = np.random.default_rng(seed)
    pw, s, b = oq.quantize(rng.normal(0, 0.02, (N, K)).astype(np.float32))
    x = f32_to_bf16_bits(rng.normal(0, 1, K).astype(np.float32))
    return x, pw, s, b


@pytest.mark.parametrize("N,K", [(8, 64), (33, 512), (256, 4096), (64, 14336)])
def test_c_q4_gemv_bf16_against_float64(clib, N, K):
    x, pw, s, b = _q4_case(N, K, N + K)
    y = np.zeros(N, np.uint16)
    clib.oracle_q4_gemv_bf16(x.ctypes.data_as(P), C.c_int64(K), pw.ctypes.data_as(P),
                             s.ctypes.data_as(P), b.ctypes.data_as(P), C.c_int64(N), 64,
                             y.ctypes.data_as(P))
    # brute-force dequant: nibble k%8 of word k/8, LSB first; group k//64
    codes = (pw[:, np.arange(K) // 8] >> (4 * (np.arange(K) % 8)).astype(np.uint32)) & 15
    W = (bf16_bits_to_f32(s)[:, np.arange(K) // 64].astype(np.float64) * codes
         + bf16_bits_to_f32(b)[:, np.arange(K) // 64])
    ref = W @ bf16_bits_to_f32(x).astype(np.float64)
    got = bf16_bits_to_f32(y)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 2e-2
    assert _ulps_bf16(got, ref.astype(np.float32)).max() <= 2
    # agrees with the NumPy oracle
    np.testing.assert_allclose(got, oq.quantized_matmul(bf16_bits_to_f32(x)[None], pw, s, b)[0],
                               rtol=1e-2, atol=1e-2 * np.abs(ref).max())


def test_c_bf16_gemv_against_float64(clib):
    rng = np.random.default_rng(5)
    N, K = 300, 4096
    w = f32_to_bf16_bits(rng.normal(0, 0.02, (N, K)).astype(np.float32))
    x = f32_to_bf16_bits(rng.normal(0, 1, K).astype(np.float32))
    y = np.zeros(N, np.float32)
    clib.oracle_bf16_gemv(x.ctypes.data_as(P), C.c_int64(K), w.ctypes.data_as(P), C.c_int64(N),
                          y.ctypes.data_as(P))
    ref = bf16_bits_to_f32(w).astype(np.float64) @ bf16_bits_to_f32(x).astype(np.float64)
    assert np.abs(y - ref).max() / np.abs(ref).max() < 1e-4
    # W·e_j picks column j
    e = np.zeros(K, np.float32)
    e[123] = 1.0
    eb = f32_to_bf16_bits(e)
    clib.oracle_bf16_gemv(eb.ctypes.data_as(P), C.c_int64(K), w.ctypes.data_as(P), C.c_int64(N),
                          y.ctypes.data_as(P))
    np.testing.assert_array_equal(y, bf16_bits_to_f32(w[:, 123]))
