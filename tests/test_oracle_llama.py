"""Pins the oracle's decoder and greedy loop (CPU only)."""
from types import SimpleNamespace

import numpy as np

from oracle import llama as oll
from oracle.kvcache import OracleKVCache


def tiny():
    cfg = oll.Config(vocab_size=17, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                     num_attention_heads=2, num_key_value_heads=1, rms_norm_eps=1e-6,
                     rope_theta=10000.0)
    return cfg, oll.OracleLlama(cfg, oll.random_weights(cfg, seed=7, std=0.15))


def test_cached_decode_matches_full_forward():
    # tests/test_mlx_generation.py:140-156
    cfg, model = tiny()
    ids = np.array([[2, 5, 3, 11]])
    full = model.forward(ids, None, use_cache=False)
    cache = OracleKVCache(cfg.num_hidden_layers)
    model.forward(ids[:, :3], cache)
    dec = model.forward(ids[:, 3:], cache)
    assert cache.get_seq_length() == 4
    # bf16 activations: decode and full forward share every rounding point
    np.testing.assert_allclose(full[:, -1], dec[:, -1], atol=1e-5, rtol=1e-5)


def test_greedy_prefills_once_then_decodes_one_token():
    # tests/test_mlx_generation.py:282-323 (recording model)
    class Recording:
        def __init__(self):
            self.config = SimpleNamespace(num_hidden_layers=1)
            self.input_lengths, self.cache_lengths = [], []

        def __call__(self, input_ids, past_key_values=None, use_cache=False):
            self.input_lengths.append(input_ids.shape[1])
            self.cache_lengths.append(past_key_values.get_seq_length())
            b, L = input_ids.shape
            st = np.broadcast_to(input_ids[:, None, :, None].astype(np.float32), (b, 1, L, 2))
            start = past_key_values.get_seq_length()
            past_key_values.update(st, st, 0, {"cache_position": np.arange(start, start + L)})
            return np.broadcast_to(np.array([0.0, 0.0, 0.0, 1.0, 0.0]), (b, L, 5))

    m = Recording()
    out = oll.greedy_generate(m, np.array([[1, 2, 4, 2]]), max_new_tokens=3,
                              cache=OracleKVCache(1))
    assert m.input_lengths == [4, 1, 1]
    assert m.cache_lengths == [0, 4, 5]
    assert out.shape == (1, 7) and np.array_equal(out[:, -3:], [[3, 3, 3]])


def test_greedy_is_deterministic_and_validates():
    cfg, model = tiny()
    a = oll.greedy_generate(model, np.array([[1, 2, 3]]), max_new_tokens=3)
    b = oll.greedy_generate(model, np.array([[1, 2, 3]]), max_new_tokens=3)
    assert np.array_equal(a, b) and a.shape == (1, 6)
    import pytest
    with pytest.raises(ValueError):
        oll.greedy_generate(model, np.array([[1]]), max_new_tokens=1, temperature=0)
