"""Llama-3.2-3B geometry (hidden 3072, FFN 8192, 24/8 heads,
head_dim 128, vocab 128256, RMSNorm eps 1e-5, RoPE theta 5e5) through the
native engine (greedy loop of ``generation.py:7-50`` over
``llama_mlx.py:863-912``).

* a 2-layer model of that geometry: greedy token ids bit-exact against the
  NumPy oracle;
* the full 28-layer model with 64-token prompts and 16 greedy tokens: ids
  bit-exact against the C decoder oracle (``oracle/c/strata_oracle_llama.c``,
  pinned against the NumPy oracle in ``tests/test_oracle_llama_c.py``) in a
  well-conditioned weight draw, and prefill logits within the oracle's own
  accumulation-order noise in the default (chaotic) draw;
* the full 28-layer model with the 2048-token prompt and 256 greedy tokens:
  graph-replayed steps give the same ids as host-launched steps, and the
  engine's logits match the op-by-op driver's.
"""
import numpy as np
import pytest
import torch

from oracle import llama as oll
from oracle.kvcache import OracleKVCache
from tests.gpu_util import bits, rel_err, to_np_f32

pytestmark = pytest.mark.gpu


def _cfg(layers):
    from lokahi_amd.llama import LlamaConfig
    return LlamaConfig(128256, 3072, 8192, layers, 24, 8, 1e-5, 500000.0)


def test_config4_two_layer_3b_geometry_tokens_bit_exact_vs_oracle(dev):
    from lokahi_amd.llama import HipLlamaForCausalLM, random_weights
    cfg = _cfg(2)
    w = random_weights(cfg, seed=404)
    model = HipLlamaForCausalLM(cfg, w)
    host = {n: bits(t) for n, t in w.items()}
    ocfg = oll.Config(**{f: getattr(cfg, f) for f in oll.Config.__dataclass_fields__})
    ref = oll.OracleLlama(ocfg, host)
    prompt = np.random.default_rng(404).integers(0, cfg.vocab_size, (1, 48))
    got = model.generate(torch.from_numpy(prompt), max_new_tokens=8).cpu().numpy()
    exp = oll.greedy_generate(ref, prompt, max_new_tokens=8, cache=OracleKVCache(2))
    assert np.array_equal(got, exp), f"\n{got[:, 48:]}\n{exp[:, 48:]}"


def test_config4_full_28_layers_prompt_2048_plus_256_tokens(dev):
    from lokahi_amd.llama import DecoderEngine, HipLlamaForCausalLM, random_weights
    cfg = _cfg(28)
    model = HipLlamaForCausalLM(cfg, random_weights(cfg, seed=77))
    gen = torch.Generator().manual_seed(77)
    prompt = torch.randint(0, cfg.vocab_size, (1, 2048), generator=gen)
    cache = model.new_cache(1, 2048 + 256 + 8)
    eng = DecoderEngine(model, cache, max_batch=1, max_tokens=2048 + 32)

    graph = eng.generate(prompt, 256, use_graph=True)
    assert cache.get_seq_length() == 2048 + 255
    cache.clear()
    host = eng.generate(prompt, 256, use_graph=False)
    assert torch.equal(graph, host)
    assert graph.shape == (1, 2304) and torch.equal(graph[:, :2048].cpu(), prompt)

    # engine logits == op-by-op driver logits, after the prompt and after 32 tokens
    seq = graph[:, :2048 + 32]
    for n in (2048, 2048 + 32):
        cache.clear()
        eng_logits = eng.forward(seq[:, :n])
        cache2 = model.new_cache(1, n + 8)
        op_logits = model(seq[:, :n], past_key_values=cache2, use_cache=True, logits="last")
        a, b = to_np_f32(eng_logits), to_np_f32(op_logits[:, -1])
        assert rel_err(a, b) < 2e-2, n



# Full depth against the C oracle.  A 28-layer random-init model is a chaotic
# map: with the default draw (q4 scale 0.0067, embedding std 0.02) merely
# switching the oracle's own linears from double to fp32 accumulation moves
# the prefill logits by ~0.3 (of ~5) and changes the greedy ids within a few
# tokens, so no fp32 implementation can match its ids bit for bit.  With a
# smaller q4 scale and a unit-std embedding the residual stream is better
# conditioned (the fp32 probe moves the logits by ~0.02 and leaves all 16 ids
# unchanged; the layers still change 14 and 16 of the 16 ids of the two prompts
# below against a 0-layer model): there the ids must be bit-exact.  In the chaotic draw the engine's
# logits must stay within a small multiple of the probe's own change.
W_SEED = 2026
WELL = dict(scale=0.001, embed_std=1.0)


def _c_oracle(ocfg, hw):
    from oracle import llama_c
    return llama_c.CLlama(ocfg, hw)


def _full_model(hw):
    from lokahi_amd.llama import DecoderEngine, HipLlamaForCausalLM, weights_to_device
    model = HipLlamaForCausalLM(_cfg(28), weights_to_device(hw))
    cache = model.new_cache(1, 96)
    return model, cache, DecoderEngine(model, cache, max_batch=1, max_tokens=96)


def _prefill_logits(eng, cache, ids):
    cache.clear()
    return to_np_f32(eng.forward(torch.from_numpy(ids))).reshape(-1)


def test_config4_full_28_layers_tokens_bit_exact_vs_c_oracle(dev):
    ocfg = oll.Config(128256, 3072, 8192, 28, 24, 8)
    hw = oll.random_q4_weights(ocfg, W_SEED, **WELL)
    cm = _c_oracle(ocfg, hw)
    model, cache, eng = _full_model(hw)
    for ps in (3, 7):
        prompt = np.random.default_rng(ps).integers(0, ocfg.vocab_size, (1, 64))
        ids, margins, _ = cm.generate(prompt, 16)
        assert margins.min() >= 0.02, (ps, margins)  # no near-tie among the 16 argmaxes
        cache.clear()
        got = eng.generate(torch.from_numpy(prompt), 16).cpu().numpy()[0]
        assert np.array_equal(got, ids), f"prompt seed {ps}\n{got[64:]}\n{ids[64:]}"
        _, _, lg = cm.generate(prompt, 1)
        cm.set_f32_accum(True)
        try:
            _, _, lg32 = cm.generate(prompt, 1)
        finally:
            cm.set_f32_accum(False)
        probe = np.abs(lg32 - lg).max()
        gpu = np.abs(_prefill_logits(eng, cache, prompt) - lg).max()
        assert gpu <= 2.0 * probe + 1e-3, (ps, gpu, probe)


def test_config4_full_28_layers_chaotic_draw_within_accumulation_noise(dev):
    ocfg = oll.Config(128256, 3072, 8192, 28, 24, 8)
    hw = oll.random_q4_weights(ocfg, W_SEED)
    cm = _c_oracle(ocfg, hw)
    prompt = np.random.default_rng(2).integers(0, ocfg.vocab_size, (1, 64))
    ids, margins, lg = cm.generate(prompt, 1)
    cm.set_f32_accum(True)
    try:
        _, _, lg32 = cm.generate(prompt, 1)
    finally:
        cm.set_f32_accum(False)
    probe = np.abs(lg32 - lg).max()
    model, cache, eng = _full_model(hw)
    del hw
    g = _prefill_logits(eng, cache, prompt)
    gpu = np.abs(g - lg).max()
    assert gpu <= 3.0 * probe, (gpu, probe)
