"""KV cache disk tier (mlx_kvcache.py:183-284, 310-367) on the device cache."""
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

CFG = SimpleNamespace(num_hidden_layers=3, num_key_value_heads=2, num_attention_heads=2,
                      hidden_size=8)


def _states(start, length, dev):
    v = np.arange(start, start + length * 8, dtype=np.float32).reshape(1, 2, length, 4)
    return torch.from_numpy(v).to(dev), torch.from_numpy(v + 100).to(dev)


def test_disk_round_trip_preserves_values_and_length(dev, tmp_path):
    # tests/test_mlx_kvcache.py:70-86
    from lokahi_amd.kvcache import HipKVCache
    cache = HipKVCache(CFG, str(tmp_path), max_length=16, dtype=torch.float32)
    keys, values = _states(0, 2, dev)
    cache.update(keys, values, 1, {"cache_position": torch.tensor([0, 1])})
    cache.save_to_disk(1)
    path = Path(tmp_path) / "kvcache_layer_1.npz"
    assert cache.get_seq_length(1) == 2 and path.exists()
    assert 1 in cache and len(cache) == 1 and cache.in_memory_layers() == []
    with np.load(path) as f:  # the reference's file layout
        assert sorted(f.files) == ["key", "seen_tokens", "value"]
        assert np.array_equal(f["key"], keys.cpu().numpy()) and int(f["seen_tokens"]) == 2
    cache.k_storage[1].zero_()  # the reload restores the file, not the stale slot
    restored = cache[1]
    assert torch.equal(restored["key"], keys) and torch.equal(restored["value"], values)
    assert cache.get_seq_length(1) == 2
    cache.clear()
    assert not path.exists() and cache.get_seq_length(1) == 0


def test_memory_only_cache_requires_explicit_disk_destination(dev, tmp_path):
    # tests/test_mlx_kvcache.py:88-93
    from lokahi_amd.kvcache import HipKVCache
    cache = HipKVCache(CFG, None, max_length=8, dtype=torch.float32)
    keys, values = _states(0, 1, dev)
    cache.update(keys, values, 0)
    with pytest.raises(ValueError, match="filename is required"):
        cache.save_to_disk(0)
    cache.save_to_disk(0, str(tmp_path / "x" / "layer0.npz"))  # explicit file is fine
    assert (tmp_path / "x" / "layer0.npz").exists()


def test_bf16_round_trip_and_append_after_reload(dev, tmp_path):
    from lokahi_amd.kvcache import HipKVCache
    rng = np.random.default_rng(3)
    cache = HipKVCache(CFG, str(tmp_path), max_length=32, dtype=torch.bfloat16)
    k = torch.from_numpy(rng.normal(size=(1, 2, 5, 4)).astype(np.float32)).to(dev).bfloat16()
    v = torch.from_numpy(rng.normal(size=(1, 2, 5, 4)).astype(np.float32)).to(dev).bfloat16()
    cache.update(k, v, 0)
    cache.offload_layers_to_disk()
    cache.v_storage[0].zero_()
    k2, v2 = k[:, :, :2] + 1, v[:, :, :2] - 1
    keys, values = cache.update(k2, v2, 0, {"cache_position": torch.tensor([5, 6])})  # reloads first
    assert torch.equal(keys, torch.cat([k, k2], 2)) and torch.equal(values, torch.cat([v, v2], 2))


def test_reference_written_file_loads(dev, tmp_path):
    # a file in the reference's layout (fp32 K, V as numpy arrays + seen_tokens)
    from lokahi_amd.kvcache import HipKVCache
    cache = HipKVCache(CFG, str(tmp_path), max_length=8, dtype=torch.float32)
    key = np.arange(1 * 2 * 3 * 4, dtype=np.float32).reshape(1, 2, 3, 4)
    np.savez_compressed(tmp_path / "ref.npz", key=key, value=-key, seen_tokens=3)
    cache._disk_offloaded[2] = str(tmp_path / "ref.npz")
    got = cache[2]
    assert np.array_equal(got["key"].cpu().numpy(), key) and cache.get_seq_length(2) == 3
    np.savez_compressed(tmp_path / "bad.npz", key=np.zeros((1, 3, 2, 4), np.float32),
                        value=np.zeros((1, 3, 2, 4), np.float32), seen_tokens=2)
    cache._disk_offloaded[1] = str(tmp_path / "bad.npz")
    with pytest.raises(ValueError, match="geometry"):
        cache[1]


def test_disk_cache_keeps_at_most_n_layers_in_memory(dev, tmp_path):
    from lokahi_amd.kvcache import HipDiskKVCache
    with pytest.raises(ValueError, match="positive"):
        HipDiskKVCache(CFG, str(tmp_path), max_layers_in_memory=0)
    cache = HipDiskKVCache(CFG, str(tmp_path), max_layers_in_memory=1, max_length=8,
                           dtype=torch.float32)
    for layer in range(3):
        keys, values = _states(10 * layer, 2, dev)
        cache.update(keys, values, layer)
        assert cache.in_memory_layers() == [layer]
    assert len(cache) == 3 and sorted(cache._disk_offloaded) == [0, 1]
    assert torch.equal(cache[0]["key"], _states(0, 2, dev)[0])


def test_engine_reloads_offloaded_layers_before_appending(dev, tmp_path):
    """The native engine appends into device memory: layers offloaded to disk
    are restored first, so no later access reloads a stale file over them."""
    from oracle import llama as oll
    from lokahi_amd.kvcache import HipKVCache
    from lokahi_amd.llama import HipLlamaForCausalLM, LlamaConfig, weights_to_device
    cfg = oll.Config(vocab_size=128, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                     num_attention_heads=2, num_key_value_heads=1, rope_theta=10000.0)
    hw = oll.random_weights(cfg, seed=5, std=0.05)
    lc = LlamaConfig(**{f: getattr(cfg, f) for f in cfg.__dataclass_fields__})
    model = HipLlamaForCausalLM(lc, weights_to_device(hw))
    prompt = torch.tensor([[3, 9, 27, 81, 115]])

    ref_cache = model.new_cache(1, 32)
    ref_tokens = model.generate(prompt[:, :3], max_new_tokens=1, past_key_values=ref_cache)
    ref_tokens = model.generate(prompt[:, 3:], max_new_tokens=6, past_key_values=ref_cache)

    cache = HipKVCache(cfg, str(tmp_path), max_length=32, dtype=torch.bfloat16)
    model.generate(prompt[:, :3], max_new_tokens=1, past_key_values=cache)
    cache.offload_layers_to_disk()
    assert cache.in_memory_layers() == []
    got = model.generate(prompt[:, 3:], max_new_tokens=6, past_key_values=cache)
    assert torch.equal(got, ref_tokens)
    want = ref_cache.get_seq_length()
    assert want == 3 + 2 + 5
    for li in range(cfg.num_hidden_layers):
        assert cache.get_seq_length(li) == want  # no reload cuts the engine's appends off
        k, v = cache.views(li)
        rk, rv = ref_cache.views(li)
        assert torch.equal(k, rk) and torch.equal(v, rv)
