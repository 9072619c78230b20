"""Weight packs onto the HIP path: a packed MLX checkpoint runs the engine
with the same weights as the safetensors load (identical tokens, oracle
tokens), and the device decoder places exact payloads."""
import json

import numpy as np
import pytest
import torch

from oracle import llama as oll
from oracle.kvcache import OracleKVCache
from tests import mlx_checkpoint
from tests.gpu_util import rel_err, to_np_f32

pytestmark = pytest.mark.gpu

SMALL = oll.Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=3,
                   num_attention_heads=4, num_key_value_heads=1, rms_norm_eps=1e-5,
                   rope_theta=500000.0)


@pytest.mark.parametrize("embed,head,seed", [("q4", "tied", 46), ("bf16", "bf16", 51)])
def test_packed_checkpoint_generates_oracle_tokens(dev, tmp_path, embed, head, seed):
    from lokahi_amd import weight_pack as wp
    from lokahi_amd.loader import load_mlx_llama
    hw = oll.random_weights(SMALL, seed=seed, std=0.05)
    ow = mlx_checkpoint.export(tmp_path / "ckpt", SMALL, hw, embed=embed, head=head)
    wp.pack_mlx_checkpoint(tmp_path / "ckpt", tmp_path / "m.strata-pack")
    config = json.loads((tmp_path / "ckpt" / "config.json").read_text())
    packed = wp.load_pack_llama(tmp_path / "m.strata-pack", config, device=0)
    direct = load_mlx_llama(tmp_path / "ckpt", device=0)
    prompt = np.random.default_rng(seed).integers(0, SMALL.vocab_size, (1, 21))
    x = torch.from_numpy(prompt)
    lp = to_np_f32(packed(x, logits="last"))[:, -1]
    ld = to_np_f32(direct(x, logits="last"))[:, -1]
    assert np.array_equal(lp, ld)  # same bytes on the device, same kernels
    ref = oll.OracleLlama(SMALL, ow)
    assert rel_err(lp, ref.forward(prompt, None, use_cache=False)[:, -1]) < 2e-2
    got = packed.generate(x, max_new_tokens=12).cpu().numpy()
    exp = oll.greedy_generate(ref, prompt, max_new_tokens=12, cache=OracleKVCache(3))
    assert np.array_equal(got, exp), f"\n{got}\n{exp}"


def test_device_decoder_places_exact_payloads(dev, tmp_path):
    from lokahi_amd import weight_pack as wp
    rng = np.random.default_rng(8)
    w = rng.integers(0, 2**32, (64, 16), dtype=np.uint64).astype(np.uint32)
    s = rng.integers(0, 2**16, (64, 2), dtype=np.uint32).astype(np.uint16)
    f = rng.normal(size=(5, 3)).astype(np.float32)
    path = tmp_path / "d.strata-pack"
    wp.write_weight_pack(path, [("w", w.tobytes()), ("s", s.tobytes()), ("f", f.tobytes())])
    group = wp.WeightGroup("layer.0", 0, (wp.TensorRef("weight", w.shape, "uint32", "w"),
                                          wp.TensorRef("scales", s.shape, "bfloat16", "s"),
                                          wp.TensorRef("norm", f.shape, "float32", "f")))
    with wp.WeightPackGroupTensorStore(path, decoder=wp.device_decoder(0)) as store:
        got = store.load_group(group)
    assert got["weight"].dtype == torch.uint32 and got["weight"].is_cuda
    assert np.array_equal(got["weight"].view(torch.int32).cpu().numpy().view(np.uint32), w)
    assert got["scales"].dtype == torch.bfloat16
    assert np.array_equal(got["scales"].view(torch.int16).cpu().numpy().view(np.uint16), s)
    assert np.array_equal(got["norm"].cpu().numpy(), f)
