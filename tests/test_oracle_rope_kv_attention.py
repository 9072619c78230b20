"""Pins the oracle's RoPE, KV-cache contract and attention (CPU only)."""
import numpy as np
import pytest
import torch

from oracle import attention as att
from oracle import rope
from oracle.kvcache import OracleKVCache


# ------------------------------------------------------------------- RoPE
def test_rope_equals_complex_rotation():
    rng = np.random.default_rng(11)
    B, H, L, D = 2, 3, 5, 16
    x = rng.normal(size=(B, H, L, D)).astype(np.float32)
    pos = np.array([[0, 2, 5, 9, 100]] * B)
    c, s = rope.cos_sin(pos, D, 10000.0)
    got = rope.apply(x, c, s)
    # textbook form: pair (x_i, x_{i+D/2}) as a complex number times e^{i*theta_i*pos}
    z = x[..., : D // 2].astype(np.float64) + 1j * x[..., D // 2:].astype(np.float64)
    inv = 1.0 / 10000.0 ** (np.arange(0, D, 2) / D)
    rot = z * np.exp(1j * pos[:, None, :, None] * inv)
    ref = np.concatenate([rot.real, rot.imag], axis=-1)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


def test_rope_identity_at_zero_norm_preserving_and_relative():
    rng = np.random.default_rng(12)
    D = 8
    q = rng.normal(size=(1, 1, 1, D)).astype(np.float32)
    k = rng.normal(size=(1, 1, 1, D)).astype(np.float32)
    c0, s0 = rope.cos_sin(np.array([[0]]), D, 500000.0)
    assert np.array_equal(rope.apply(q, c0, s0), q)
    c, s = rope.cos_sin(np.array([[37]]), D, 500000.0)
    r = rope.apply(q, c, s)
    pair = lambda v: v[..., :D // 2] ** 2 + v[..., D // 2:] ** 2  # noqa: E731
    np.testing.assert_allclose(pair(r), pair(q), rtol=1e-5)

    def dot(pq, pk):
        cq, sq = rope.cos_sin(np.array([[pq]]), D, 10000.0)
        ck, sk = rope.cos_sin(np.array([[pk]]), D, 10000.0)
        return float((rope.apply(q, cq, sq) * rope.apply(k, ck, sk)).sum())
    assert abs(dot(10, 3) - dot(17, 10)) < 1e-4  # depends only on pq - pk


def test_rope_matches_reference_test_form():
    # tests/test_mlx_generation.py:259-280: seed 11, dim 4, positions [0,2,5]
    rng = np.random.default_rng(11)
    q = rng.normal(size=(1, 2, 3, 4)).astype(np.float32)
    c, s = rope.cos_sin(np.array([[0, 2, 5]]), 4, 10000.0)
    half = lambda v: np.concatenate([-v[..., 2:], v[..., :2]], axis=-1)  # noqa: E731
    ref = q * c[:, None] + half(q) * s[:, None]
    np.testing.assert_allclose(rope.apply(q, c, s), ref, atol=1e-6)


# --------------------------------------------------------------- KV cache
def _states(start, length):
    values = np.arange(start, start + length * 8, dtype=np.float32).reshape(1, 2, length, 4)
    return values, values + 100


def test_kv_update_appends_and_tracks_lengths():
    # known answers of tests/test_mlx_kvcache.py:28-50
    cache = OracleKVCache(2)
    k0, v0 = _states(0, 3)
    k1, v1 = _states(24, 1)
    cache.update(k0, v0, 0, {"cache_position": np.arange(0, 3)})
    keys, values = cache.update(k1, v1, 0, {"cache_position": np.array([3])})
    assert cache.get_seq_length(0) == 4 and cache.get_seq_length(1) == 0
    assert keys.shape == (1, 2, 4, 4)
    assert np.array_equal(keys[:, :, :3], k0) and np.array_equal(values[:, :, 3:], v1)


def test_kv_rejects_replayed_positions_and_bad_layers():
    cache = OracleKVCache(2)
    k, v = _states(0, 2)
    cache.update(k, v, 0, {"cache_position": np.array([0, 1])})
    with pytest.raises(ValueError, match="append exactly"):
        cache.update(k, v, 0, {"cache_position": np.array([0, 1])})
    with pytest.raises(ValueError, match="outside configured layer count"):
        cache.update(k, v, 2)
    with pytest.raises(ValueError, match="rank 4"):
        cache.update(k[0], v[0], 0)


# -------------------------------------------------------------- attention
def _torch_sdpa64(q, k, v, qpos=None, causal=False):
    q, k, v = (torch.from_numpy(np.asarray(t, np.float64)) for t in (q, k, v))
    g = q.shape[1] // k.shape[1]
    k = k.repeat_interleave(g, dim=1)
    v = v.repeat_interleave(g, dim=1)
    mask = None
    if causal:
        kp = torch.arange(k.shape[2])
        mask = kp[None, None, None, :] <= torch.as_tensor(qpos)[:, None, :, None]
    return torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask).numpy()


@pytest.mark.parametrize("qb,kb", [(3, 4), (1, 1), (32768, 1024), (2, 5)])
def test_unmasked_matches_torch_sdpa(qb, kb):
    rng = np.random.default_rng(0)
    q = rng.standard_normal((1, 4, 7, 6), dtype=np.float32)
    k = rng.standard_normal((1, 2, 9, 6), dtype=np.float32)
    v = rng.standard_normal((1, 2, 9, 6), dtype=np.float32)
    got = att.chunked_gqa(q, k, v, causal=False, q_block_size=qb, k_block_size=kb)
    np.testing.assert_allclose(got, _torch_sdpa64(q, k, v), atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(att.naive_gqa(q, k, v), _torch_sdpa64(q, k, v), atol=1e-12)


def test_causal_prefill_and_decode_match_torch_sdpa():
    rng = np.random.default_rng(0)
    q = rng.standard_normal((2, 4, 7, 6), dtype=np.float32)
    k = rng.standard_normal((2, 2, 7, 6), dtype=np.float32)
    v = rng.standard_normal((2, 2, 7, 6), dtype=np.float32)
    pos = np.broadcast_to(np.arange(7), (2, 7))
    got = att.chunked_gqa(q, k, v, pos, causal=True, q_block_size=3, k_block_size=2)
    np.testing.assert_allclose(got, _torch_sdpa64(q, k, v, pos, True), atol=1e-5, rtol=1e-5)
    qd = rng.standard_normal((1, 4, 1, 6), dtype=np.float32)
    kd = rng.standard_normal((1, 2, 6, 6), dtype=np.float32)
    vd = rng.standard_normal((1, 2, 6, 6), dtype=np.float32)
    got = att.chunked_gqa(qd, kd, vd, np.array([[5]]), causal=True, q_block_size=1, k_block_size=2)
    np.testing.assert_allclose(got, _torch_sdpa64(qd, kd, vd, [[5]], True), atol=1e-5, rtol=1e-5)


def test_future_values_do_not_change_earlier_outputs():
    rng = np.random.default_rng(0)
    q = rng.standard_normal((1, 2, 5, 4), dtype=np.float32)
    k = rng.standard_normal((1, 1, 5, 4), dtype=np.float32)
    v = rng.standard_normal((1, 1, 5, 4), dtype=np.float32)
    v2 = v.copy()
    v2[:, :, 3:] += 1000.0
    a = att.chunked_gqa(q, k, v, k_block_size=2)
    b = att.chunked_gqa(q, k, v2, k_block_size=2)
    assert np.allclose(a[:, :, :3], b[:, :, :3])
    assert not np.allclose(a[:, :, 3:], b[:, :, 3:])


def test_attention_validation_messages():
    one = np.ones((1, 3, 2, 4), np.float32)
    kv = np.ones((1, 2, 2, 4), np.float32)
    with pytest.raises(ValueError, match="divisible"):
        att.chunked_gqa(one, kv, kv)
    with pytest.raises(ValueError, match="key length >= query length"):
        att.chunked_gqa(np.ones((1, 2, 3, 4), np.float32), kv, kv)
    with pytest.raises(ValueError, match="block sizes must be positive"):
        att.chunked_gqa(kv, kv, kv, q_block_size=0)
