"""Writes the golden vectors under tests/golden/ from the CPU oracle.

Run from the repository root:  python tests/golden/make_golden.py

The reference (Ikaikaalika/lokahi) commits no numeric golden files for this
path; its known answers are in-test (tests/test_mlx_attention.py:53-137,
tests/test_mlx_generation.py:140-156, 259-323, tests/test_mlx_kvcache.py:23-68).
These fixtures freeze the oracle's outputs on seeded inputs of the same kinds
and the BASELINE config shapes (scaled down where the oracle would be slow),
so the GPU path is checked against committed data and the oracle against its
own earlier outputs.  Inputs are stored (not regenerated) so the fixtures
stand on their own.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import attention as att  # noqa: E402
from oracle import llama as oll  # noqa: E402
from oracle import q4, rope  # noqa: E402
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16  # noqa: E402
from oracle.kvcache import OracleKVCache  # noqa: E402


def q4_linear():
    """Config-2 kind (q4 group 64, bf16 x, fp32 accumulate) at [1..4] x [256 -> 96]."""
    rng = np.random.default_rng(2)
    w = rng.normal(0, 0.02, (96, 256)).astype(np.float32)
    packed, s, b = q4.quantize(w)
    x = f32_to_bf16_bits(rng.normal(0, 1, (4, 256)).astype(np.float32))
    y = q4.quantized_matmul(bf16_bits_to_f32(x), packed, s, b)
    np.savez_compressed(HERE / "q4_linear.npz", w=packed, scales=s, biases=b, x=x, y=y,
                        codes=q4.unpack(packed))


def rope_case():
    """RoPE rotate-half at positions [0, 2, 5] (the positions of
    tests/test_mlx_generation.py:259-280), theta 1e4, fp32."""
    rng = np.random.default_rng(11)
    q = rng.normal(size=(1, 2, 3, 8)).astype(np.float32)
    k = rng.normal(size=(1, 1, 3, 8)).astype(np.float32)
    pos = np.array([[0, 2, 5]], dtype=np.int32)
    c, s = rope.cos_sin(pos, 8, 10000.0)
    np.savez_compressed(HERE / "rope.npz", q=q, k=k, pos=pos, q_out=rope.apply(q, c, s),
                        k_out=rope.apply(k, c, s))


def attention_case():
    """Config-1 geometry (Hq8/Hkv2, D64, theta 1e4, fp32) at L=40, chunks 16:
    RoPE, causal chunked prefill, then one cached decode at position 40."""
    rng = np.random.default_rng(1)
    L, D = 40, 64
    q = rng.normal(size=(1, 8, L + 1, D)).astype(np.float32)
    k = rng.normal(size=(1, 2, L + 1, D)).astype(np.float32)
    v = rng.normal(size=(1, 2, L + 1, D)).astype(np.float32)
    pos = np.arange(L + 1, dtype=np.int32)[None]
    c, s = rope.cos_sin(pos, D, 10000.0)
    qr, kr = rope.apply(q, c, s), rope.apply(k, c, s)
    pre = att.chunked_gqa(qr[:, :, :L], kr[:, :, :L], v[:, :, :L], pos[:, :L], True, 16, 16)
    dec = att.chunked_gqa(qr[:, :, L:], kr, v, pos[:, L:], True, 16, 16)
    np.savez_compressed(HERE / "attention.npz", q=q, k=k, v=v, pos=pos, prefill=pre, decode=dec)


def kv_case():
    """The arange known answers of tests/test_mlx_kvcache.py:28-50 (layer 0
    gets a [1,1,4,2] block then one more row; layer 1 stays empty)."""
    cache = OracleKVCache(2)
    k0 = np.arange(8, dtype=np.float32).reshape(1, 1, 4, 2)
    v0 = k0 + 100
    cache.update(k0, v0, 0, {"cache_position": np.arange(4)})
    k1 = np.array([[[[8, 9]]]], dtype=np.float32)
    K, V = cache.update(k1, k1 + 100, 0, {"cache_position": np.array([4])})
    np.savez_compressed(HERE / "kvcache.npz", k0=k0, v0=v0, k1=k1, K=K, V=V,
                        lengths=np.array([cache.get_seq_length(0), cache.get_seq_length(1)]))


TINY = oll.Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=3,
                  num_attention_heads=4, num_key_value_heads=1, rms_norm_eps=1e-5,
                  rope_theta=500000.0)


def greedy_case():
    """Greedy ids of a tiny q4 Llama (weights std 0.05, seed 31) on a 19-token
    prompt, 12 new tokens; bf16 activation flow, fp32 logits."""
    hw = oll.random_weights(TINY, seed=31, std=0.05)
    prompt = np.random.default_rng(31).integers(0, TINY.vocab_size, (1, 19))
    ids = oll.greedy_generate(oll.OracleLlama(TINY, hw), prompt, max_new_tokens=12,
                              cache=OracleKVCache(3))
    np.savez_compressed(HERE / "greedy_tiny.npz", prompt=prompt, ids=ids,
                        config=np.array([TINY.vocab_size, TINY.hidden_size,
                                         TINY.intermediate_size, TINY.num_hidden_layers,
                                         TINY.num_attention_heads, TINY.num_key_value_heads]),
                        seed=np.array(31))


if __name__ == "__main__":
    q4_linear()
    rope_case()
    attention_case()
    kv_case()
    greedy_case()
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))
