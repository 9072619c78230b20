"""BASELINE config 5 at full size (8192 tokens): parity by sampled rows and by
properties that hold at any size (prefill row == decode over the same keys;
library GEMM == fused-kernel GEMM)."""
import numpy as np
import pytest
import torch

from oracle import q4
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits
from tests.gpu_util import rel_err, to_dev, to_np_f32
from tests.test_gpu_attention import _c_decode

pytestmark = pytest.mark.gpu
TOL_BF16 = 2e-2
TOL_F32 = 1e-3


def test_config5_attention_8k_rows_match_oracle_and_decode(dev):
    from lokahi_amd import ops
    L, Hq, Hkv, D = 8192, 32, 8, 128
    g = torch.Generator(device=dev).manual_seed(8192)
    q = torch.randn((1, Hq, L, D), generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn((1, Hkv, L, D), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((1, Hkv, L, D), generator=g, device=dev).to(torch.bfloat16)
    out = ops.attention(q, k, v, causal=True, q_block_size=512, k_block_size=512)
    for row in (0, 63, 64, 1000, 4095, 8191):  # tile edges, the diagonal, the last row
        qr = q[:, :, row:row + 1].contiguous()
        kr, vr = k[:, :, :row + 1].contiguous(), v[:, :, :row + 1].contiguous()
        dec = ops.attention(qr, kr, vr)  # decode kernel: query at position row
        got = to_np_f32(out[:, :, row:row + 1])
        assert rel_err(got, to_np_f32(dec)) < TOL_BF16, row
        if row in (64, 4095, 8191):
            kb = kr.cpu().view(torch.int16).numpy().view(np.uint16)
            vb = vr.cpu().view(torch.int16).numpy().view(np.uint16)
            ref = _c_decode(to_np_f32(qr), kb, vb)
            assert rel_err(got, ref) < TOL_BF16, row


@pytest.mark.parametrize("name,N,K", [("q/o", 4096, 4096), ("k/v", 1024, 4096),
                                      ("up", 14336, 4096), ("down", 4096, 14336)])
def test_config5_layer_gemms_8k_sampled_rows(dev, name, N, K):
    """Every config-5 linear shape at M = 8192 on the default prefill path;
    rows at tile edges against the float64 oracle, plus linearity in x."""
    from lokahi_amd import ops
    from tests.gpu_util import bits
    M = 8192
    g = torch.Generator(device=dev).manual_seed(N * 7 + K)
    tw, ts, tb = ops.quantize(torch.randn((N, K), generator=g, device=dev) * 0.02)
    tx = torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16)
    y = ops.linear(tx, tw, ts, tb, out_dtype=torch.float32)
    w, s, b = bits(tw), bits(ts), bits(tb)
    rows = np.array([0, 1, 127, 128, 255, 256, 4097, 8190, 8191])
    xr = bf16_bits_to_f32(bits(tx[torch.from_numpy(rows).to(dev)]))
    ref = q4.quantized_matmul(xr, w, s, b)
    assert rel_err(to_np_f32(y)[rows], ref) < TOL_BF16, name
    # the MFMA path stages each dequantized weight as bf16 (one RNE rounding of
    # s*q + b, as MLX's qmm stages tiles in the activation dtype): against that
    # matrix the fp32 tolerance holds
    from oracle.bf16 import round_bf16
    wq = round_bf16(q4.dequantize(w, s, b, 64).astype(np.float32)).astype(np.float64)
    ref16 = xr.astype(np.float64) @ wq.T
    assert rel_err(to_np_f32(y)[rows], ref16) < TOL_F32, name
    # bf16 output path and linearity: y(2x) == 2 y(x) exactly (power-of-two scale)
    y2 = ops.linear(tx * 2, tw, ts, tb, out_dtype=torch.float32)
    assert torch.equal(y2, 2 * y)
    yb = ops.linear(tx, tw, ts, tb)
    assert yb.dtype == torch.bfloat16
    assert rel_err(to_np_f32(yb)[rows], ref) < TOL_BF16


def test_multi_linear_gemm_one_launch_equals_separate_launches(dev):
    """q/k/v-shaped linears in one launch of the 256-column kernel (weights
    re-laid side by side, each tile writing its own output) against one
    launch per linear; M = 8192 + 100 ends in a partial row tile, and a
    linear whose N is not a multiple of 256 takes the 128-tile kernel."""
    from lokahi_amd import ops
    M, K = 8192 + 100, 4096
    g = torch.Generator(device=dev).manual_seed(6144)
    ws = [ops.quantize(torch.randn((n, K), generator=g, device=dev) * 0.02)
          for n in (4096, 1024, 1024, 1000)]
    x = torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16)
    fused = ops.linear_multi(x, ws)
    for w, y in zip(ws, fused):
        assert torch.equal(y, ops.linear(x, *w))
    # the float64 oracle on rows of each problem, including remainder rows
    from tests.gpu_util import bits
    rows = np.array([0, 255, 256, 8191, 8192, 8291])
    xr = bf16_bits_to_f32(bits(x[torch.from_numpy(rows).to(dev)]))
    for (w, s, b), y in zip(ws, fused):
        ref = q4.quantized_matmul(xr, bits(w), bits(s), bits(b))
        assert rel_err(to_np_f32(y)[rows], ref) < TOL_BF16
