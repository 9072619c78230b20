"""MLX checkpoint reading (safetensors, config, names) on the CPU."""
import json

import numpy as np
import pytest

from lokahi_amd import loader
from oracle import llama as oll
from oracle import q4
from oracle.bf16 import bf16_bits_to_f32, round_bf16
from tests import mlx_checkpoint

TINY = oll.Config(vocab_size=96, hidden_size=128, intermediate_size=192, num_hidden_layers=2,
                  num_attention_heads=2, num_key_value_heads=1, rms_norm_eps=1e-5,
                  rope_theta=10000.0)


def _tensors(rng):
    return {
        "a.u32": ("U32", rng.integers(0, 2**32, (5, 8), dtype=np.uint64).astype(np.uint32)),
        "b.bf16": ("BF16", rng.integers(0, 2**16, (3, 64), dtype=np.uint32).astype(np.uint16)),
        "c.f32": ("F32", rng.normal(size=(7,)).astype(np.float32)),
        "d.f16": ("F16", rng.normal(size=(2, 2)).astype(np.float16)),
        "e.i32": ("I32", rng.integers(-9, 9, (4,)).astype(np.int32)),
        "f.i8": ("I8", rng.integers(-9, 9, (6,)).astype(np.int8)),
    }


def test_reader_roundtrip_and_header(tmp_path):
    t = _tensors(np.random.default_rng(0))
    path = tmp_path / "x.safetensors"
    loader.write_safetensors(path, t, {"format": "mlx"})
    r = loader.SafeTensorReader(path)
    assert sorted(r.keys()) == sorted(t)  # __metadata__ is not a tensor
    for name, (dt, a) in t.items():
        got = r.get(name)
        assert r.dtype(name) == dt and got.dtype == a.dtype and np.array_equal(got, a)
    with pytest.raises(KeyError, match="not found"):
        r.get("missing")
    raw = path.read_bytes()  # 8-byte little-endian header length, then JSON
    n = int.from_bytes(raw[:8], "little")
    assert json.loads(raw[8:8 + n])["__metadata__"] == {"format": "mlx"}


def test_reader_agrees_with_the_safetensors_library(tmp_path):
    st_np = pytest.importorskip("safetensors.numpy")
    st_torch = pytest.importorskip("safetensors.torch")
    import torch
    rng = np.random.default_rng(1)
    t = _tensors(rng)
    ours = tmp_path / "ours.safetensors"
    loader.write_safetensors(ours, t)
    plain = tmp_path / "plain.safetensors"  # safetensors.numpy has no bfloat16
    loader.write_safetensors(plain, {k: v for k, v in t.items() if v[0] != "BF16"})
    lib = st_np.load_file(str(plain))  # the library reads our files ...
    for name, (dt, a) in t.items():
        if dt != "BF16":
            assert np.array_equal(lib[name], a)
    bf = st_torch.load_file(str(ours))["b.bf16"]
    assert bf.dtype == torch.bfloat16
    assert np.array_equal(bf.view(torch.int16).numpy().view(np.uint16), t["b.bf16"][1])
    theirs = tmp_path / "theirs.safetensors"  # ... and we read the library's file
    src = {"w": torch.from_numpy(rng.normal(size=(4, 64)).astype(np.float32)).to(torch.bfloat16),
           "u": torch.from_numpy(np.arange(12, dtype=np.int32))}
    st_torch.save_file(src, str(theirs))
    r = loader.SafeTensorReader(theirs)
    assert r.dtype("w") == "BF16"
    assert np.array_equal(r.get("w"), src["w"].view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(r.get("u"), src["u"].numpy())


def test_config_validation():
    base = {"vocab_size": 96, "hidden_size": 128, "intermediate_size": 192,
            "num_hidden_layers": 2, "num_attention_heads": 2, "num_key_value_heads": 1}
    cfg = loader.config_from_dict({**base, "quantization_config": {"group_size": 64, "bits": 4}})
    assert (cfg.head_dim, cfg.group_size) == (64, 64)
    assert cfg.rms_norm_eps == 1e-6 and cfg.rope_theta == 10000.0  # llama_mlx.py:462, 701
    for q, msg in (({"group_size": 64, "bits": 8}, "4-bit"),
                   ({"group_size": 32, "bits": 4}, "group_size 64"),
                   ({"group_size": 64, "bits": 4, "mode": "mxfp4"}, "affine")):
        with pytest.raises(ValueError, match=msg):
            loader.config_from_dict({**base, "quantization": q})
    with pytest.raises(ValueError, match="not quantized"):
        loader.config_from_dict(base)
    assert loader.quantization_parameters({"quantization": {"group_size": 64, "bits": 4}}) == \
        (64, 4, "affine")


@pytest.mark.parametrize("embed,head", [("q4", "tied"), ("bf16", "q4"), ("bf16", "bf16")])
def test_exported_names_match_the_layout(tmp_path, embed, head):
    hw = oll.random_weights(TINY, seed=3)
    mlx_checkpoint.export(tmp_path, TINY, hw, embed=embed, head=head)
    names = set()
    for f in tmp_path.glob("*.safetensors"):
        names |= set(loader.SafeTensorReader(f).keys())
    cfg = loader.config_from_dict(json.loads((tmp_path / "config.json").read_text()))
    assert names == set(loader.checkpoint_names(cfg, quantized_embed=embed == "q4", head=head))


def test_oracle_quantized_embedding_and_tied_head():
    hw = oll.random_weights(TINY, seed=4)
    trip = q4.quantize(bf16_bits_to_f32(hw["embed_tokens"]), 64)
    wq = {k: v for k, v in hw.items() if k not in ("embed_tokens", "lm_head")}
    for suf, a in zip(("weight", "scales", "biases"), trip):
        wq["embed_tokens." + suf] = a
    m = oll.OracleLlama(TINY, wq)
    ids = np.array([[3, 17, 95, 0]])
    # embedding rows: nibble k%8 of word k/8 (LSB first) times scale plus bias, per element
    rows = m._embed(ids)[0]
    w, s, b = (x[ids[0]] for x in trip)
    s, b = bf16_bits_to_f32(s).astype(np.float64), bf16_bits_to_f32(b).astype(np.float64)
    ref = np.empty((4, TINY.hidden_size))
    for r in range(4):
        for k in range(TINY.hidden_size):
            qv = (int(w[r, k // 8]) >> (4 * (k % 8))) & 15
            ref[r, k] = s[r, k // 64] * qv + b[r, k // 64]
    assert np.array_equal(rows, round_bf16(ref.astype(np.float32)))
    # tied head = the head given explicitly as the same triple
    explicit = dict(wq)
    for suf, a in zip(("weight", "scales", "biases"), trip):
        explicit["lm_head." + suf] = a
    a = m.forward(ids, None, use_cache=False)
    e = oll.OracleLlama(TINY, explicit).forward(ids, None, use_cache=False)
    assert np.array_equal(a, e)
