"""Decoder glue kernels vs the oracle: RMSNorm (+residual), SiLU*up, embed, argmax."""
import numpy as np
import pytest
import torch

from oracle import llama as oll
from oracle.bf16 import f32_to_bf16_bits, round_bf16
from tests.gpu_util import bf16_dev, bits, to_np_f32

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,H", [(1, 4096), (3, 3072), (2, 8192), (5, 100), (1, 14336)])
def test_rmsnorm_with_and_without_residual(dev, rows, H):
    from lokahi_amd import ops
    rng = np.random.default_rng(H)
    x = round_bf16(rng.normal(size=(rows, H)).astype(np.float32))
    r = round_bf16(rng.normal(size=(rows, H)).astype(np.float32))
    w = f32_to_bf16_bits(rng.uniform(0.5, 1.5, H).astype(np.float32))
    tx = bf16_dev(x, dev)
    y = ops.rmsnorm(tx, torch.from_numpy(w.view(np.int16)).view(torch.bfloat16).to(dev), 1e-5)
    ref = oll.rms_norm(x, w, 1e-5)
    # RNE of the same fp32 value except where the fp32 reductions differ in the last bit
    assert np.mean(bits(y) == f32_to_bf16_bits(ref)) > 0.995
    assert np.abs(to_np_f32(y) - ref).max() <= 2 ** -7 * np.abs(ref).max()
    tx = bf16_dev(x, dev)
    y = ops.rmsnorm(tx, torch.from_numpy(w.view(np.int16)).view(torch.bfloat16).to(dev), 1e-5,
                    residual=bf16_dev(r, dev))
    h = round_bf16(x + r)
    assert np.array_equal(bits(tx), f32_to_bf16_bits(h))  # residual stream updated in place
    ref = oll.rms_norm(h, w, 1e-5)
    assert np.mean(bits(y) == f32_to_bf16_bits(ref)) > 0.995


def test_silu_mul_and_embed(dev):
    from lokahi_amd import ops
    rng = np.random.default_rng(1)
    g = round_bf16(rng.normal(0, 3, 20000).astype(np.float32))
    u = round_bf16(rng.normal(size=20000).astype(np.float32))
    a = ops.silu_mul(bf16_dev(g, dev), bf16_dev(u, dev))
    ref = oll.silu_mul(g, u)
    assert np.mean(bits(a) == f32_to_bf16_bits(ref)) > 0.995
    assert np.abs(to_np_f32(a) - ref).max() <= 2 ** -7 * np.abs(ref).max()
    table = f32_to_bf16_bits(rng.normal(size=(50, 64)).astype(np.float32))
    ids = np.array([[3, 0, 49, 3]])
    e = ops.embed(torch.from_numpy(table.view(np.int16)).view(torch.bfloat16).to(dev),
                  torch.from_numpy(ids).to(dev))
    assert np.array_equal(bits(e), table[ids])


def test_argmax_ties_pick_lowest_index(dev):
    from lokahi_amd import ops
    rng = np.random.default_rng(2)
    V = 128256
    lg = rng.normal(size=(3, V)).astype(np.float32)
    lg[1, [7, 90000, 128255]] = 50.0
    lg[2, :] = 1.0
    out = ops.argmax(torch.from_numpy(lg).to(dev)).cpu().numpy()
    assert out.tolist() == [int(np.argmax(lg[0])), 7, 0]
    small = np.array([[0.0, 2.0, 2.0, -1.0]], np.float32)
    assert ops.argmax(torch.from_numpy(small).to(dev)).cpu().numpy().tolist() == [1]


def test_silu_mul_vector_and_scalar_paths_agree_bit_for_bit(dev):
    """16-byte path (aligned, n % 8 == 0) and per-element path (an odd length
    at an odd offset) run the same arithmetic per value."""
    from lokahi_amd import ops
    rng = np.random.default_rng(3)
    g = round_bf16(rng.normal(0, 4, 40008).astype(np.float32))
    u = round_bf16(rng.normal(size=40008).astype(np.float32))
    tg, tu = bf16_dev(g, dev), bf16_dev(u, dev)
    vec = bits(ops.silu_mul(tg, tu))
    sca = bits(ops.silu_mul(tg[1:40002], tu[1:40002]))
    assert np.array_equal(vec[1:40002], sca)
    ref = oll.silu_mul(g, u)
    assert np.mean(vec == f32_to_bf16_bits(ref)) > 0.995
