"""Decode GEMV over the load-time layout (matrix-core kernel) vs the oracle."""
import numpy as np
import pytest
import torch

from oracle import q4
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits
from tests.gpu_util import rel_err, to_dev, to_np_f32

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2   # rel-err bound for bf16 outputs
TOL_F32 = 1e-3    # rel-err bound for fp32 outputs


def _weights(rng, N, K, std=0.02):
    return q4.quantize(rng.normal(0, std, (N, K)).astype(np.float32), 64)


def _x(rng, M, K):
    return f32_to_bf16_bits(rng.normal(0, 1, (M, K)).astype(np.float32))


def _layout(dev, probs):
    from lokahi_amd import ops
    return ops.Q4Layout([tuple(to_dev(a, dev) for a in p) for p in probs])


@pytest.mark.parametrize("shapes,K", [([(4096,), (1024,), (1024,)], 4096),  # q/k/v
                                      ([(14336,), (14336,)], 4096),          # gate/up
                                      ([(4096,)], 14336)])                   # down
def test_layout_gemv_8b_shapes(dev, shapes, K):
    rng = np.random.default_rng(K + len(shapes))
    probs = [_weights(rng, n, K) for (n,) in shapes]
    lay = _layout(dev, probs)
    x = _x(rng, 1, K)
    tx = to_dev(x, dev)
    y32 = lay(tx, out_dtype=torch.float32)
    y16 = lay(tx)
    for (w, s, b), a, c in zip(probs, y32, y16):
        ref = q4.quantized_matmul(bf16_bits_to_f32(x), w, s, b)
        assert rel_err(to_np_f32(a), ref) < TOL_F32
        assert rel_err(to_np_f32(c), ref) < TOL_BF16
        # the bf16 output is the RNE rounding of (nearly) the fp32 result
        assert np.mean(f32_to_bf16_bits(to_np_f32(a)) == f32_to_bf16_bits(to_np_f32(c))) > 0.999


@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_layout_gemv_batches_ragged_rows_padded_k(dev, M):
    # N not a multiple of the 16-row block, K not a multiple of the 1024-code task
    rng = np.random.default_rng(30 + M)
    K = 1088
    probs = [_weights(rng, n, K) for n in (100, 36, 17)]
    lay = _layout(dev, probs)
    x = _x(rng, M, K)
    ys = lay(to_dev(x, dev), out_dtype=torch.float32)
    for (w, s, b), y in zip(probs, ys):
        assert y.shape == (M, w.shape[0])
        assert rel_err(to_np_f32(y), q4.quantized_matmul(bf16_bits_to_f32(x), w, s, b)) < TOL_F32


@pytest.mark.parametrize("M,K", [(5, 1088), (8, 3072), (6, 4096), (7, 8192), (8, 4096),
                                 (8, 1024), (5, 14336), (8, 14336), (6, 16384)])
def test_layout_gemv_eight_rows_equal_two_four_row_calls(dev, M, K):
    """5..8 rows run in one launch: two 4-row workgroups per row block share
    the grid.  Every row is bit-identical to the same row in a 4-row call,
    and within the fp32 tolerance of the oracle."""
    rng = np.random.default_rng(50 + M + K)
    probs = [_weights(rng, n, K) for n in (100, 36, 17)]
    lay = _layout(dev, probs)
    x = _x(rng, M, K)
    tx = to_dev(x, dev)
    ys = lay(tx, out_dtype=torch.float32)
    lo = lay(tx[:4].contiguous(), out_dtype=torch.float32)
    # rows M-4 .. M-1 (a 4-row call: a single row would take the 1-row kernel)
    hi = lay(tx[M - 4:].contiguous(), out_dtype=torch.float32)
    ys16 = lay(tx)
    for (w, s, b), y, a, c, y16 in zip(probs, ys, lo, hi, ys16):
        assert y.shape == (M, w.shape[0])
        assert torch.equal(y[:4], a) and torch.equal(y[4:], c[8 - M:])
        ref = q4.quantized_matmul(bf16_bits_to_f32(x), w, s, b)
        assert rel_err(to_np_f32(y), ref) < TOL_F32
        assert rel_err(to_np_f32(y16), ref) < TOL_BF16


def test_layout_gemv_rejects_more_than_eight_rows(dev):
    rng = np.random.default_rng(58)
    lay = _layout(dev, [_weights(rng, 32, 2048)])
    with pytest.raises(ValueError, match="outside"):
        lay(to_dev(_x(rng, 9, 2048), dev))
    assert lay(to_dev(_x(rng, 8, 2048), dev))[0].shape == (8, 32)


def test_layout_gemv_matches_mlx_layout_gemv(dev):
    from lokahi_amd import ops
    rng = np.random.default_rng(41)
    K = 3072
    w, s, b = _weights(rng, 1024, K)
    x = _x(rng, 1, K)
    tx = to_dev(x, dev)
    y_lay = to_np_f32(_layout(dev, [(w, s, b)])(tx, out_dtype=torch.float32)[0])
    y_mlx = to_np_f32(ops.linear(tx, *(to_dev(a, dev) for a in (w, s, b)), out_dtype=torch.float32))
    ref = q4.quantized_matmul(bf16_bits_to_f32(x), w, s, b)
    # both accumulate exact bf16 x code products in fp32; only the order differs
    assert rel_err(y_lay, y_mlx) < 1e-5
    assert rel_err(y_lay, ref) < 1e-5


def test_layout_gemv_closed_forms(dev):
    rng = np.random.default_rng(42)
    K = 2048
    # all-zero codes: y = sum_g b_g * sum(x over group g)
    N = 48
    zw = np.zeros((N, K // 8), np.uint32)
    s = f32_to_bf16_bits(np.full((N, K // 64), 0.25, np.float32))
    bb = f32_to_bf16_bits(rng.normal(0, 1, (N, K // 64)).astype(np.float32))
    x = _x(rng, 1, K)
    y = to_np_f32(_layout(dev, [(zw, s, bb)])(to_dev(x, dev), out_dtype=torch.float32)[0])
    xs = bf16_bits_to_f32(x).reshape(1, K // 64, 64).sum(-1, dtype=np.float64)
    ref = xs @ bf16_bits_to_f32(bb).astype(np.float64).T
    assert rel_err(y, ref) < 1e-5
    # one-hot x picks column k exactly: y[n] = s[n, k/64] * q[n, k] + b[n, k/64]
    w, s, b = _weights(rng, N, K)
    for k in (0, 63, 64, 1023, 1024, K - 1):
        xo = np.zeros((1, K), np.float32)
        xo[0, k] = 1.0
        y = to_np_f32(_layout(dev, [(w, s, b)])(to_dev(f32_to_bf16_bits(xo), dev),
                                                 out_dtype=torch.float32)[0])
        q = (w[:, k // 8] >> np.uint32(4 * (k % 8))) & np.uint32(15)
        sk = bf16_bits_to_f32(s[:, k // 64]).astype(np.float64)
        bk = bf16_bits_to_f32(b[:, k // 64]).astype(np.float64)
        exact = sk * q + bk
        # the kernel forms s (128 + q) + (b - 128 s): a few fp32 roundings of
        # terms of magnitude 128 |s| + |b|
        bound = 4 * np.finfo(np.float32).eps * (128 * np.abs(sk) + np.abs(bk))
        assert np.all(np.abs(y[0] - exact) <= bound), k


def test_layout_gemv_linearity_and_edges(dev):
    rng = np.random.default_rng(43)
    for N, K in [(1, 64), (5, 192), (33, 1024), (16, 16384)]:
        w, s, b = _weights(rng, N, K)
        lay = _layout(dev, [(w, s, b)])
        x = _x(rng, 1, K)
        y = to_np_f32(lay(to_dev(x, dev), out_dtype=torch.float32)[0])
        assert rel_err(y, q4.quantized_matmul(bf16_bits_to_f32(x), w, s, b)) < TOL_F32, (N, K)
        # y(2x) == 2 y(x) exactly (a power-of-two scale commutes with every rounding)
        x2 = f32_to_bf16_bits(2 * bf16_bits_to_f32(x))
        y2 = to_np_f32(lay(to_dev(x2, dev), out_dtype=torch.float32)[0])
        assert np.array_equal(y2, 2 * y), (N, K)
