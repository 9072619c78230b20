"""MLX 4-bit checkpoints loaded onto the HIP path: engine vs oracle."""
import numpy as np
import pytest
import torch

from oracle import llama as oll
from oracle import q4
from oracle.bf16 import f32_to_bf16_bits, round_bf16
from oracle.kvcache import OracleKVCache
from tests import mlx_checkpoint
from tests.gpu_util import rel_err, to_np_f32

pytestmark = pytest.mark.gpu

SMALL = oll.Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=3,
                   num_attention_heads=4, num_key_value_heads=1, rms_norm_eps=1e-5,
                   rope_theta=500000.0)


def test_dequantize_matches_oracle(dev):
    from lokahi_amd import ops
    rng = np.random.default_rng(5)
    w, s, b = q4.quantize(rng.normal(0, 0.05, (300, 192)).astype(np.float32), 64)
    got = ops.dequantize(*(torch.from_numpy(a.view(np.int32 if a.dtype == np.uint32 else np.int16))
                           .to(dev).view(torch.uint32 if a.dtype == np.uint32 else torch.bfloat16)
                           for a in (w, s, b)))
    exp = f32_to_bf16_bits(round_bf16(q4.dequantize(w, s, b, 64).astype(np.float32)))
    assert np.array_equal(got.view(torch.int16).cpu().numpy().view(np.uint16), exp)


# Seeds whose oracle top-2 logit margin stays >= 0.07 over the 12 generated
# tokens: closer calls are decided by bf16 rounding noise, not by the kernels.
@pytest.mark.parametrize("embed,head,seed", [("q4", "tied", 46), ("bf16", "q4", 46),
                                             ("bf16", "bf16", 51)])
def test_loaded_checkpoint_generates_oracle_tokens(dev, tmp_path, embed, head, seed):
    from lokahi_amd.loader import load_mlx_llama
    hw = oll.random_weights(SMALL, seed=seed, std=0.05)
    ow = mlx_checkpoint.export(tmp_path, SMALL, hw, embed=embed, head=head)
    model = load_mlx_llama(tmp_path, device=0)
    ref = oll.OracleLlama(SMALL, ow)
    prompt = np.random.default_rng(seed).integers(0, SMALL.vocab_size, (1, 21))
    logits = to_np_f32(model(torch.from_numpy(prompt), logits="last"))[:, -1]
    exp_logits = ref.forward(prompt, None, use_cache=False)[:, -1]
    assert rel_err(logits, exp_logits) < 2e-2
    got = model.generate(torch.from_numpy(prompt), max_new_tokens=12).cpu().numpy()
    exp = oll.greedy_generate(ref, prompt, max_new_tokens=12, cache=OracleKVCache(3))
    assert np.array_equal(got, exp), f"\n{got}\n{exp}"


MID = oll.Config(vocab_size=1024, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                 num_attention_heads=4, num_key_value_heads=2, rms_norm_eps=1e-5,
                 rope_theta=500000.0)


def test_q4_head_with_prefill_pack_generates_oracle_tokens(dev, tmp_path):
    """A q4 lm_head set after the engine re-laid its prefill linears (every
    linear's N a multiple of 256, a 48-token prompt: the prefill runs the
    MFMA GEMM on the load-time layout), then greedy decode on the q4 head's
    GEMV layout; the oracle's smallest top-2 gap over the 8 tokens is 0.148
    at seed 60."""
    from lokahi_amd.loader import load_mlx_llama
    hw = oll.random_weights(MID, seed=60, std=0.05)
    ow = mlx_checkpoint.export(tmp_path, MID, hw, embed="bf16", head="q4")
    model = load_mlx_llama(tmp_path, device=0)
    ref = oll.OracleLlama(MID, ow)
    prompt = np.random.default_rng(60).integers(0, MID.vocab_size, (1, 48))
    got = model.generate(torch.from_numpy(prompt), max_new_tokens=8).cpu().numpy()
    exp = oll.greedy_generate(ref, prompt, max_new_tokens=8, cache=OracleKVCache(2))
    assert np.array_equal(got, exp), f"\n{got}\n{exp}"
