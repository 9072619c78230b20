"""Committed golden vectors (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU tests: the oracle reproduces every fixture (it has not drifted).
GPU tests: the HIP path reproduces the fixtures to the build's bar -- bit-exact
for int4 unpacking, RoPE, KV contents/lengths and greedy ids; rel-err <= 1e-3
for fp32 outputs and <= 2e-2 for bf16 outputs.
"""
from pathlib import Path

import numpy as np
import pytest

from oracle import attention as att
from oracle import llama as oll
from oracle import q4, rope
from oracle.bf16 import bf16_bits_to_f32, round_bf16
from oracle.kvcache import OracleKVCache

GOLD = Path(__file__).resolve().parent / "golden"
TOL_F32 = 1e-3
TOL_BF16 = 2e-2


def load(name):
    return np.load(GOLD / f"{name}.npz", allow_pickle=False)


def rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / np.abs(ref).max())


def tiny_config(f):
    v, h, i, n, hq, hkv = (int(a) for a in f["config"])
    return oll.Config(vocab_size=v, hidden_size=h, intermediate_size=i, num_hidden_layers=n,
                      num_attention_heads=hq, num_key_value_heads=hkv, rms_norm_eps=1e-5,
                      rope_theta=500000.0)


# ------------------------------------------------------------------ oracle (CPU)
def test_oracle_reproduces_q4_fixture():
    f = load("q4_linear")
    assert np.array_equal(q4.unpack(f["w"]), f["codes"])
    assert np.array_equal(q4.pack(f["codes"]), f["w"])
    y = q4.quantized_matmul(bf16_bits_to_f32(f["x"]), f["w"], f["scales"], f["biases"])
    assert np.array_equal(y, f["y"])


def test_oracle_reproduces_rope_fixture():
    f = load("rope")
    c, s = rope.cos_sin(f["pos"], 8, 10000.0)
    assert np.array_equal(rope.apply(f["q"], c, s), f["q_out"])
    assert np.array_equal(rope.apply(f["k"], c, s), f["k_out"])


def test_oracle_reproduces_attention_fixture():
    f = load("attention")
    L = f["prefill"].shape[2]
    c, s = rope.cos_sin(f["pos"], 64, 10000.0)
    qr, kr = rope.apply(f["q"], c, s), rope.apply(f["k"], c, s)
    pos = f["pos"]
    pre = att.chunked_gqa(qr[:, :, :L], kr[:, :, :L], f["v"][:, :, :L], pos[:, :L], True, 16, 16)
    dec = att.chunked_gqa(qr[:, :, L:], kr, f["v"], pos[:, L:], True, 16, 16)
    assert np.array_equal(pre, f["prefill"]) and np.array_equal(dec, f["decode"])


def test_oracle_reproduces_kv_fixture():
    f = load("kvcache")
    cache = OracleKVCache(2)
    cache.update(f["k0"], f["v0"], 0, {"cache_position": np.arange(4)})
    K, V = cache.update(f["k1"], f["k1"] + 100, 0, {"cache_position": np.array([4])})
    assert np.array_equal(K, f["K"]) and np.array_equal(V, f["V"])
    assert [cache.get_seq_length(0), cache.get_seq_length(1)] == f["lengths"].tolist() == [5, 0]


def test_oracle_reproduces_greedy_fixture():
    f = load("greedy_tiny")
    cfg = tiny_config(f)
    hw = oll.random_weights(cfg, seed=int(f["seed"]), std=0.05)
    ids = oll.greedy_generate(oll.OracleLlama(cfg, hw), f["prompt"], max_new_tokens=12,
                              cache=OracleKVCache(cfg.num_hidden_layers))
    assert np.array_equal(ids, f["ids"])


# ------------------------------------------------------------------- HIP (GPU)
@pytest.mark.gpu
def test_hip_q4_linear_matches_fixture(dev):
    import torch
    from lokahi_amd import ops
    from tests.gpu_util import to_dev, to_np_f32
    f = load("q4_linear")
    w, s, b = (to_dev(f[n], dev) for n in ("w", "scales", "biases"))
    x = to_dev(f["x"], dev)
    for m in (1, 2, 4):
        y32 = ops.linear(x[:m], w, s, b, out_dtype=torch.float32).cpu().numpy()
        assert rel(y32, f["y"][:m]) < TOL_F32
        ybf = to_np_f32(ops.linear(x[:m], w, s, b))
        assert rel(ybf, round_bf16(f["y"][:m])) < TOL_BF16


@pytest.mark.gpu
def test_hip_rope_matches_fixture_bit_exact(dev):
    import torch
    from lokahi_amd import ops
    f = load("rope")
    q = torch.from_numpy(f["q"].copy()).to(dev)
    k = torch.from_numpy(f["k"].copy()).to(dev)
    ops.rope(q, k, torch.from_numpy(f["pos"]).to(dev), 10000.0)
    assert np.array_equal(q.cpu().numpy(), f["q_out"])
    assert np.array_equal(k.cpu().numpy(), f["k_out"])


@pytest.mark.gpu
def test_hip_attention_matches_fixture(dev):
    import torch
    from lokahi_amd import ops
    f = load("attention")
    L = f["prefill"].shape[2]
    q = torch.from_numpy(f["q"].copy()).to(dev)
    k = torch.from_numpy(f["k"].copy()).to(dev)
    v = torch.from_numpy(f["v"].copy()).to(dev)
    pos = torch.from_numpy(f["pos"]).to(dev)
    ops.rope(q, k, pos, 10000.0)
    pre = ops.attention(q[:, :, :L].contiguous(), k[:, :, :L].contiguous(),
                        v[:, :, :L].contiguous(), query_positions=pos[:, :L].contiguous(),
                        q_block_size=16, k_block_size=16)
    assert rel(pre.cpu().numpy(), f["prefill"]) < TOL_F32
    dec = ops.attention(q[:, :, L:].contiguous(), k, v, query_positions=pos[:, L:].contiguous())
    assert rel(dec.cpu().numpy(), f["decode"]) < TOL_F32


@pytest.mark.gpu
def test_hip_kv_cache_matches_fixture(dev):
    import torch
    from types import SimpleNamespace
    from lokahi_amd.kvcache import HipKVCache
    f = load("kvcache")
    cfg = SimpleNamespace(num_hidden_layers=2, num_key_value_heads=1, num_attention_heads=1,
                          hidden_size=2)
    cache = HipKVCache(cfg, batch_size=1, max_length=8, dtype=torch.float32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    cache.update(t(f["k0"]), t(f["v0"]), 0, {"cache_position": torch.arange(4)})
    K, V = cache.update(t(f["k1"]), t(f["k1"] + 100), 0, {"cache_position": torch.tensor([4])})
    assert np.array_equal(K.cpu().numpy(), f["K"]) and np.array_equal(V.cpu().numpy(), f["V"])
    assert [cache.get_seq_length(0), cache.get_seq_length(1)] == f["lengths"].tolist()


@pytest.mark.gpu
@pytest.mark.parametrize("use_graph", [True, False])
def test_hip_greedy_ids_match_fixture(dev, use_graph):
    import torch
    from lokahi_amd.llama import HipLlamaForCausalLM, LlamaConfig, weights_to_device
    f = load("greedy_tiny")
    cfg = tiny_config(f)
    hw = oll.random_weights(cfg, seed=int(f["seed"]), std=0.05)
    lc = LlamaConfig(**{n: getattr(cfg, n) for n in cfg.__dataclass_fields__})
    model = HipLlamaForCausalLM(lc, weights_to_device(hw))
    got = model.generate(torch.from_numpy(f["prompt"]), max_new_tokens=12,
                         use_graph=use_graph).cpu().numpy()
    assert np.array_equal(got, f["ids"])
