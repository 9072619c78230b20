"""RoPE and KV-cache append/read on the GPU vs the oracle (bit-exact where integer/copy)."""
import numpy as np
import pytest
import torch

from oracle import rope
from oracle.bf16 import f32_to_bf16_bits, round_bf16
from oracle.kvcache import OracleKVCache
from tests.gpu_util import bf16_dev, bits, to_np_f32

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("D,theta", [(64, 10000.0), (128, 500000.0), (4, 10000.0)])
def test_rope_fp32_bit_exact(dev, D, theta):
    from lokahi_amd import ops
    rng = np.random.default_rng(D)
    B, Hq, Hkv, L = 2, 4, 2, 9
    q = rng.normal(size=(B, Hq, L, D)).astype(np.float32)
    k = rng.normal(size=(B, Hkv, L, D)).astype(np.float32)
    pos = np.stack([np.arange(L), np.arange(100, 100 + L) * 37])
    c, s = rope.cos_sin(pos, D, theta)
    tq, tk = torch.from_numpy(q).to(dev), torch.from_numpy(k).to(dev)
    ops.rope(tq, tk, torch.from_numpy(pos).to(dev), theta)
    assert np.array_equal(bits(tq), rope.apply(q, c, s).view(np.uint32))
    assert np.array_equal(bits(tk), rope.apply(k, c, s).view(np.uint32))


def test_rope_bf16_bit_exact(dev):
    from lokahi_amd import ops
    rng = np.random.default_rng(5)
    B, H, L, D = 1, 8, 33, 128
    q = round_bf16(rng.normal(size=(B, H, L, D)).astype(np.float32))
    pos = np.arange(500, 500 + L)[None]
    c, s = rope.cos_sin(pos, D, 500000.0)
    tq = bf16_dev(q, dev)
    ops.rope(tq, None, torch.from_numpy(pos).to(dev), 500000.0)
    assert np.array_equal(bits(tq), f32_to_bf16_bits(rope.apply(q, c, s)))


def _states(start, length):
    v = np.arange(start, start + length * 8, dtype=np.float32).reshape(1, 2, length, 4)
    return v, v + 100


def test_kv_cache_reference_known_answers(dev):
    # tests/test_mlx_kvcache.py:28-68 on the device cache
    from types import SimpleNamespace
    from lokahi_amd.kvcache import HipKVCache
    cfg = SimpleNamespace(num_hidden_layers=2, num_key_value_heads=2, num_attention_heads=2,
                          hidden_size=8)
    cache = HipKVCache(cfg, batch_size=1, max_length=16, dtype=torch.float32)
    k0, v0 = _states(0, 3)
    k1, v1 = _states(24, 1)
    cache.update(torch.from_numpy(k0).to(dev), torch.from_numpy(v0).to(dev), 0,
                 {"cache_position": torch.arange(0, 3)})
    keys, values = cache.update(torch.from_numpy(k1).to(dev), torch.from_numpy(v1).to(dev), 0,
                                {"cache_position": torch.tensor([3])})
    assert cache.get_seq_length(0) == 4 and cache.get_seq_length(1) == 0
    assert tuple(keys.shape) == (1, 2, 4, 4)
    assert np.array_equal(keys[:, :, :3].cpu().numpy(), k0)
    assert np.array_equal(values[:, :, 3:].cpu().numpy(), v1)
    assert 0 in cache and 1 not in cache and len(cache) == 1
    with pytest.raises(ValueError, match="append exactly"):
        cache.update(torch.from_numpy(k0).to(dev), torch.from_numpy(v0).to(dev), 0,
                     {"cache_position": torch.tensor([0, 1, 2])})
    with pytest.raises(ValueError, match="outside configured layer count"):
        cache.update(torch.from_numpy(k0).to(dev), torch.from_numpy(v0).to(dev), 5)
    cache.clear()
    assert cache.get_seq_length(0) == 0


def test_kv_append_matches_oracle_bit_exact_over_many_steps(dev):
    from types import SimpleNamespace
    from lokahi_amd.kvcache import HipKVCache
    cfg = SimpleNamespace(num_hidden_layers=3, num_key_value_heads=8, num_attention_heads=32,
                          hidden_size=4096)
    rng = np.random.default_rng(1)
    cache = HipKVCache(cfg, batch_size=2, max_length=64, dtype=torch.bfloat16)
    ref = OracleKVCache(3)
    for step, L in enumerate([7, 1, 1, 20, 1]):
        for layer in (0, 2):
            k = round_bf16(rng.normal(size=(2, 8, L, 128)).astype(np.float32))
            v = round_bf16(rng.normal(size=(2, 8, L, 128)).astype(np.float32))
            K, V = cache.update(bf16_dev(k, dev), bf16_dev(v, dev), layer)
            rk, rv = ref.update(k, v, layer)
            assert np.array_equal(bits(K), f32_to_bf16_bits(rk))
            assert np.array_equal(bits(V), f32_to_bf16_bits(rv))
            assert cache.get_seq_length(layer) == ref.get_seq_length(layer)
    assert cache.get_seq_length(1) == 0 and cache.get_seq_length(None) == 30
    with pytest.raises(ValueError, match="capacity"):
        z = torch.zeros((2, 8, 40, 128), dtype=torch.bfloat16, device=dev)
        cache.update(z, z, 0)


def test_fused_rope_kv_append_matches_oracle(dev):
    from types import SimpleNamespace
    from lokahi_amd.kvcache import HipKVCache
    B, Hq, Hkv, D, theta = 1, 8, 2, 64, 10000.0
    cfg = SimpleNamespace(num_hidden_layers=1, num_key_value_heads=Hkv, num_attention_heads=Hq,
                          hidden_size=Hq * D)
    rng = np.random.default_rng(2)
    cache = HipKVCache(cfg, batch_size=B, max_length=32, dtype=torch.bfloat16)
    ref = OracleKVCache(1)
    pos0 = 0
    for L in (5, 1, 1):
        q = round_bf16(rng.normal(size=(B, L, Hq * D)).astype(np.float32))
        k = round_bf16(rng.normal(size=(B, L, Hkv * D)).astype(np.float32))
        v = round_bf16(rng.normal(size=(B, L, Hkv * D)).astype(np.float32))
        qo = torch.empty((B, Hq, L, D), dtype=torch.bfloat16, device=dev)
        cache.rope_append(0, bf16_dev(q, dev), bf16_dev(k, dev), bf16_dev(v, dev), Hq, L, theta, qo)
        c, s = rope.cos_sin(np.arange(pos0, pos0 + L)[None], D, theta)
        qh = q.reshape(B, L, Hq, D).transpose(0, 2, 1, 3)
        kh = k.reshape(B, L, Hkv, D).transpose(0, 2, 1, 3)
        vh = v.reshape(B, L, Hkv, D).transpose(0, 2, 1, 3)
        assert np.array_equal(bits(qo), f32_to_bf16_bits(rope.apply(qh, c, s)))
        rk, rv = ref.update(round_bf16(rope.apply(kh, c, s)), vh, 0)
        K, V = cache.views(0)
        assert np.array_equal(bits(K), f32_to_bf16_bits(rk))
        assert np.array_equal(bits(V), f32_to_bf16_bits(rv))
        pos0 += L
    assert cache.get_seq_length(0) == 7


def test_fused_rope_kv_append_long_rows_matches_oracle(dev):
    """From 256 rows (B * L) the fused kernel deals each thread a slice of
    the heads and computes (cos, sin) once per slice; 8B geometry (32 q / 8
    KV heads, D 128, theta 5e5) at B = 2, L = 300 then a one-token append,
    bit-exact against the oracle."""
    from types import SimpleNamespace
    from lokahi_amd.kvcache import HipKVCache
    B, Hq, Hkv, D, theta = 2, 32, 8, 128, 500000.0
    cfg = SimpleNamespace(num_hidden_layers=1, num_key_value_heads=Hkv, num_attention_heads=Hq,
                          hidden_size=Hq * D)
    rng = np.random.default_rng(5)
    cache = HipKVCache(cfg, batch_size=B, max_length=320, dtype=torch.bfloat16)
    ref = OracleKVCache(1)
    pos0 = 0
    for L in (300, 1):
        q = round_bf16(rng.normal(size=(B, L, Hq * D)).astype(np.float32))
        k = round_bf16(rng.normal(size=(B, L, Hkv * D)).astype(np.float32))
        v = round_bf16(rng.normal(size=(B, L, Hkv * D)).astype(np.float32))
        qo = torch.empty((B, Hq, L, D), dtype=torch.bfloat16, device=dev)
        cache.rope_append(0, bf16_dev(q, dev), bf16_dev(k, dev), bf16_dev(v, dev), Hq, L, theta, qo)
        c, s = rope.cos_sin(np.arange(pos0, pos0 + L)[None], D, theta)
        qh = q.reshape(B, L, Hq, D).transpose(0, 2, 1, 3)
        kh = k.reshape(B, L, Hkv, D).transpose(0, 2, 1, 3)
        vh = v.reshape(B, L, Hkv, D).transpose(0, 2, 1, 3)
        assert np.array_equal(bits(qo), f32_to_bf16_bits(rope.apply(qh, c, s)))
        rk, rv = ref.update(round_bf16(rope.apply(kh, c, s)), vh, 0)
        K, V = cache.views(0)
        assert np.array_equal(bits(K), f32_to_bf16_bits(rk))
        assert np.array_equal(bits(V), f32_to_bf16_bits(rv))
        pos0 += L
    assert cache.get_seq_length(0) == 301


def test_engine_prefill_rope_append_matches_op_by_op_path(dev):
    """The engine's prefill appends RoPE'd K and V with the 16-byte kernel
    over the (cos, sin) table; the op-by-op path uses the per-pair kernel
    that evaluates cos/sin itself.  Layer 0 sees the same projections on
    both paths, so its cache rows must agree bit for bit."""
    import numpy as np
    from lokahi_amd.llama import DecoderEngine, HipLlamaForCausalLM, LlamaConfig, weights_to_device
    from oracle import llama as oll
    cfg = oll.Config(vocab_size=1024, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                     num_attention_heads=4, num_key_value_heads=2)
    lc = LlamaConfig(**{f: getattr(cfg, f) for f in cfg.__dataclass_fields__})
    model = HipLlamaForCausalLM(lc, weights_to_device(oll.random_weights(cfg, seed=8, std=0.05)))
    ids = torch.from_numpy(np.random.default_rng(8).integers(0, 1024, (1, 48)))
    c1 = model.new_cache(1, 64)
    eng = DecoderEngine(model, c1, max_batch=1, max_tokens=64)
    eng.forward(ids)
    c2 = model.new_cache(1, 64)
    model(ids, past_key_values=c2, use_cache=True, logits="last")
    k1, v1 = c1.views(0)
    k2, v2 = c2.views(0)
    assert torch.equal(k1[:, :, :48].cpu(), k2[:, :, :48].cpu())
    assert torch.equal(v1[:, :, :48].cpu(), v2[:, :, :48].cpu())
