"""q4 linear (GEMV / MFMA GEMM), bf16 linear and the quantizer vs the oracle."""
import numpy as np
import pytest
import torch

from oracle import q4
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16
from tests.gpu_util import bf16_dev, rel_err, to_dev, to_np_f32

pytestmark = pytest.mark.gpu

# Llama-3-8B decode linears (north_star config 2): (N, K)
SHAPES_8B = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]
TOL_BF16 = 2e-2   # rel-err bound for bf16 outputs
TOL_F32 = 1e-3    # rel-err bound for fp32 outputs


def _problem(rng, N, K, M=1):
    w, s, b = q4.quantize(rng.normal(0, 0.02, (N, K)).astype(np.float32), 64)
    x = f32_to_bf16_bits(rng.normal(0, 1, (M, K)).astype(np.float32))
    return w, s, b, x


@pytest.mark.parametrize("N,K", SHAPES_8B)
def test_gemv_decode_shapes_match_oracle(dev, N, K):
    from lokahi_amd import ops
    rng = np.random.default_rng(N + K)
    w, s, b, x = _problem(rng, N, K)
    ref = q4.quantized_matmul(bf16_bits_to_f32(x), w, s, b)
    tw, ts, tb, tx = (to_dev(a, dev) for a in (w, s, b, x))
    y32 = to_np_f32(ops.linear(tx, tw, ts, tb, out_dtype=torch.float32))
    assert rel_err(y32, ref) < TOL_F32
    y16 = to_np_f32(ops.linear(tx, tw, ts, tb))
    assert rel_err(y16, ref) < TOL_BF16
    # bf16 output is the RNE rounding of (nearly) the fp32 result
    assert np.mean(f32_to_bf16_bits(y32) == f32_to_bf16_bits(y16)) > 0.999


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
def test_gemv_small_batches_and_fp32_activations(dev, M):
    from lokahi_amd import ops
    rng = np.random.default_rng(M)
    N, K = 384, 1024
    w, s, b, x = _problem(rng, N, K, M)
    ref = q4.quantized_matmul(bf16_bits_to_f32(x), w, s, b)
    tw, ts, tb = (to_dev(a, dev) for a in (w, s, b))
    y = to_np_f32(ops.linear(to_dev(x, dev), tw, ts, tb, out_dtype=torch.float32))
    assert rel_err(y, ref) < TOL_F32
    xf = rng.normal(0, 1, (M, K)).astype(np.float32)  # reference dtype flow: fp32 activations
    y = to_np_f32(ops.linear(torch.from_numpy(xf).to(dev), tw, ts, tb))
    assert rel_err(y, q4.quantized_matmul(xf, w, s, b)) < TOL_F32


def test_gemv_multi_problem_one_launch(dev):
    from lokahi_amd import ops
    rng = np.random.default_rng(9)
    K = 2048
    probs = [_problem(rng, n, K)[:3] for n in (512, 128, 128)]  # q / k / v-like
    x = f32_to_bf16_bits(rng.normal(0, 1, (1, K)).astype(np.float32))
    outs = ops.linear_multi(to_dev(x, dev), [tuple(to_dev(a, dev) for a in p) for p in probs],
                            out_dtype=torch.float32)
    for (w, s, b), y in zip(probs, outs):
        assert rel_err(to_np_f32(y), q4.quantized_matmul(bf16_bits_to_f32(x), w, s, b)) < TOL_F32


def test_gemv_edge_shapes(dev):
    from lokahi_amd import ops
    rng = np.random.default_rng(10)
    for N, K in [(1, 64), (3, 64), (17, 192), (1000, 320)]:
        w, s, b, x = _problem(rng, N, K)
        y = to_np_f32(ops.linear(to_dev(x, dev), *(to_dev(a, dev) for a in (w, s, b)),
                                 out_dtype=torch.float32))
        assert rel_err(y, q4.quantized_matmul(bf16_bits_to_f32(x), w, s, b)) < TOL_F32, (N, K)
    # all-zero codes: closed form y = sum_g b_g * sum x_g
    K = 256
    zw = np.zeros((4, K // 8), np.uint32)
    s = f32_to_bf16_bits(np.full((4, K // 64), 0.5, np.float32))
    bb = f32_to_bf16_bits(rng.normal(0, 1, (4, K // 64)).astype(np.float32))
    x = f32_to_bf16_bits(rng.normal(0, 1, (1, K)).astype(np.float32))
    y = to_np_f32(ops.linear(to_dev(x, dev), to_dev(zw, dev), to_dev(s, dev), to_dev(bb, dev),
                             out_dtype=torch.float32))
    expect = bf16_bits_to_f32(x).reshape(K // 64, 64).sum(1).astype(np.float64) @ bf16_bits_to_f32(bb).T
    np.testing.assert_allclose(y[0], expect, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("M,N,K", [(64, 256, 512), (200, 1000, 1024), (1000, 384, 4096),
                                   (9, 128, 64), (2048, 4096, 4096)])
def test_gemm_prefill_matches_oracle(dev, M, N, K):
    from lokahi_amd import ops
    rng = np.random.default_rng(M * 7 + N)
    w, s, b, x = _problem(rng, N, K, M)
    y = to_np_f32(ops.linear(to_dev(x, dev), *(to_dev(a, dev) for a in (w, s, b)),
                             out_dtype=torch.float32))
    ref = q4.quantized_matmul(bf16_bits_to_f32(x), w, s, b)
    # weights are dequantized to bf16 in LDS (as MLX's qmm does): bf16 tolerance
    # against the exact product, fp32 tolerance against x @ bf16(dequant(W)).T
    assert rel_err(y, ref) < TOL_BF16
    wq = round_bf16(q4.dequantize(w, s, b, 64).astype(np.float32)).astype(np.float64)
    ref_b = bf16_bits_to_f32(x).astype(np.float64) @ wq.T
    assert rel_err(y, ref_b) < TOL_F32


@pytest.mark.parametrize("M,N,K", [(300, 1000, 1024), (512, 4096, 4096), (257, 96, 64)])
def test_gemm_prefill_rows_match_oracle(dev, M, N, K):
    """Prefill rows run the fused-dequant kernels (MFMA, or the 128 x 128 tile
    kernel for N not a multiple of 256): the bf16-staged product within fp32
    tolerance, the exact product within bf16 tolerance."""
    from lokahi_amd import ops
    rng = np.random.default_rng(M + N + K)
    w, s, b, x = _problem(rng, N, K, M)
    tw, ts, tb = (to_dev(a, dev) for a in (w, s, b))
    ref = q4.quantized_matmul(bf16_bits_to_f32(x), w, s, b)
    wq = round_bf16(q4.dequantize(w, s, b, 64).astype(np.float32)).astype(np.float64)
    ref_b = bf16_bits_to_f32(x).astype(np.float64) @ wq.T
    y32 = to_np_f32(ops.linear(to_dev(x, dev), tw, ts, tb, out_dtype=torch.float32))
    y16 = to_np_f32(ops.linear(to_dev(x, dev), tw, ts, tb))
    assert rel_err(y32, ref_b) < TOL_F32
    assert rel_err(y16, ref) < TOL_BF16


def test_linear_rejects_bad_parameters(dev):
    from lokahi_amd import ops
    w = torch.zeros((4, 8), dtype=torch.uint32, device=dev)
    s = torch.zeros((4, 1), dtype=torch.bfloat16, device=dev)
    x = torch.zeros((1, 64), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        ops.linear(x, w, s, s, bits=8)
    with pytest.raises(ValueError):
        ops.linear(torch.zeros((1, 96), dtype=torch.bfloat16, device=dev), w, s, s)


def test_bf16_dense_linear(dev):
    from lokahi_amd import ops
    rng = np.random.default_rng(12)
    # K = 4096 takes the x-ahead-of-weights kernels (batch tiles 1, 2, 4;
    # M = 5 leaves three zeroed rows in its second tile)
    for M, N, K in [(1, 1000, 512), (3, 333, 256), (1, 777, 4096), (2, 500, 4096),
                    (4, 300, 4096), (5, 130, 4096)]:
        W = f32_to_bf16_bits(rng.normal(0, 0.02, (N, K)).astype(np.float32))
        x = f32_to_bf16_bits(rng.normal(0, 1, (M, K)).astype(np.float32))
        y = to_np_f32(ops.linear(to_dev(x, dev), to_dev(W, dev), None, None, out_dtype=torch.float32))
        ref = bf16_bits_to_f32(x).astype(np.float64) @ bf16_bits_to_f32(W).T.astype(np.float64)
        assert rel_err(y, ref) < TOL_F32


def test_quantizer_is_bit_exact_with_oracle(dev):
    from lokahi_amd import ops
    rng = np.random.default_rng(13)
    wf = rng.normal(0, 0.02, (300, 512)).astype(np.float32)
    pw, sc, bi = ops.quantize(torch.from_numpy(wf).to(dev))
    ew, es, eb = q4.quantize(wf, 64)
    assert np.array_equal(pw.cpu().view(torch.int32).numpy().view(np.uint32), ew)
    assert np.array_equal(sc.cpu().view(torch.int16).numpy().view(np.uint16), es)
    assert np.array_equal(bi.cpu().view(torch.int16).numpy().view(np.uint16), eb)


def test_gemm_many_prompt_lengths(dev):
    """Prefill M is the prompt length: a run of distinct lengths through the
    per-call re-layout and split-K routing stays correct."""
    from lokahi_amd import ops
    rng = np.random.default_rng(260)
    N, K = 256, 128
    w, s, b, x = _problem(rng, N, K, 600)
    tw, ts, tb, tx = (to_dev(a, dev) for a in (w, s, b, x))
    wq = round_bf16(q4.dequantize(w, s, b, 64).astype(np.float32)).astype(np.float64)
    for M in range(300, 560, 7):
        y = ops.linear(tx[:M], tw, ts, tb, out_dtype=torch.float32)
        ref = bf16_bits_to_f32(x[:M]).astype(np.float64) @ wq.T
        assert rel_err(to_np_f32(y), ref) < TOL_F32, M


@pytest.mark.parametrize("M,K", [(9, 1024), (16, 3584), (17, 1024), (40, 2048), (64, 1024),
                                 (65, 1024), (150, 512), (300, 1024)])
def test_gemm_few_rows_skinny_kernel(dev, M, K):
    """Up to 39 rows the skinny kernel runs: 16 or 64 output columns per
    workgroup, the K quarters of each column block summed in LDS (from 40
    rows, linears whose N is a multiple of 256 take the MFMA kernel, whose
    own test follows).  q/k/v-like linears in one launch, bf16 and fp32
    outputs, against x @ bf16(dequant(W)).T in float64, and bit-identical to
    separate launches of each linear."""
    from lokahi_amd import ops
    rng = np.random.default_rng(M * 7 + K)
    ns = (1024, 256, 256) if M != 16 else (16384, 16, 48)  # 64- and 16-column blocks
    probs = [_problem(rng, n, K)[:3] for n in ns]
    x = f32_to_bf16_bits(rng.normal(0, 1, (M, K)).astype(np.float32))
    dprobs = [tuple(to_dev(a, dev) for a in p) for p in probs]
    xd = to_dev(x, dev)
    y32 = ops.linear_multi(xd, dprobs, out_dtype=torch.float32)
    y16 = ops.linear_multi(xd, dprobs)
    for (w, s, b), a32, a16, dp in zip(probs, y32, y16, dprobs):
        wq = round_bf16(q4.dequantize(w, s, b, 64).astype(np.float32)).astype(np.float64)
        ref_b = bf16_bits_to_f32(x).astype(np.float64) @ wq.T
        assert rel_err(to_np_f32(a32), ref_b) < TOL_F32
        assert rel_err(to_np_f32(a16), q4.quantized_matmul(bf16_bits_to_f32(x), w, s, b)) < TOL_BF16
        alone = ops.linear(xd, *dp, out_dtype=torch.float32)
        assert torch.equal(alone, a32)


@pytest.mark.parametrize("M,K,ns", [(65, 4096, (4096, 1024, 1024)), (100, 1024, (1024, 256, 256)),
                                    (128, 4096, (14336,)), (200, 14336, (4096,)),
                                    (255, 2048, (512, 1536)), (300, 1024, (1024, 256, 256)),
                                    (777, 4096, (4096,)), (128, 4096, (14336, 4096)),
                                    (40, 512, (256,)), (1000, 64, (256, 512))])
def test_gemm_mid_rows_split_k(dev, M, K, ns):
    """40 rows and up, N a multiple of 256: the 256-column MFMA
    kernel over all rows (a partial last row tile), each linear whose tiles
    leave CUs idle split over K slices whose fp32 partial sums are added in
    slice order.  Against x @ bf16(dequant(W)).T in float64 and the oracle's
    q4 matmul; a linear gives the same bits in a fused launch as alone (the
    split depends on its own M, K and N only).  Includes a call whose
    linears get different slice counts (two launches), K = 64 (one group,
    no split) and exactly 40 rows at a short K."""
    from lokahi_amd import ops
    rng = np.random.default_rng(M * 11 + K)
    probs = [_problem(rng, n, K)[:3] for n in ns]
    x = f32_to_bf16_bits(rng.normal(0, 1, (M, K)).astype(np.float32))
    dprobs = [tuple(to_dev(a, dev) for a in p) for p in probs]
    xd = to_dev(x, dev)
    y32 = ops.linear_multi(xd, dprobs, out_dtype=torch.float32)
    y16 = ops.linear_multi(xd, dprobs)
    xf = bf16_bits_to_f32(x)
    for (w, s, b), a32, a16, dp in zip(probs, y32, y16, dprobs):
        wq = round_bf16(q4.dequantize(w, s, b, 64).astype(np.float32)).astype(np.float64)
        ref_b = xf.astype(np.float64) @ wq.T
        assert rel_err(to_np_f32(a32), ref_b) < TOL_F32
        assert rel_err(to_np_f32(a16), q4.quantized_matmul(xf, w, s, b)) < TOL_BF16
        assert torch.equal(ops.linear(xd, *dp, out_dtype=torch.float32), a32)
        assert torch.equal(ops.linear(xd, *dp), a16)
