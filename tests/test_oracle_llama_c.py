"""Pins the C Llama decoder (oracle/c/strata_oracle_llama.c) against the NumPy
``OracleLlama`` + ``greedy_generate`` (CPU only).

The two share the dtype flow but not the code: NumPy matmuls against a loop
of scalar C, ``np.exp`` against ``expf``, batched against per-row RoPE.  A
dropped rounding, a wrong head mapping, an off-by-one cache position or a
transposed head weight changes the greedy ids or moves the logits by far
more than float32 rounding, so ids must agree exactly and the final logits
to float32 level.  The prompt runs through one prefill forward and every
later token through a cached one-token step, as ``generation.py:7-50``.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import llama as oll
from oracle.kvcache import OracleKVCache

llama_c = pytest.importorskip("oracle.llama_c")

CFGS = {
    "mha": oll.Config(vocab_size=384, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=2, num_key_value_heads=2),
    "gqa": oll.Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=3,
                      num_attention_heads=4, num_key_value_heads=1),
    "gqa_hd128": oll.Config(vocab_size=640, hidden_size=512, intermediate_size=768,
                            num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2),
}


def _model(cfg, seed, std=0.05):
    w = oll.random_weights(cfg, seed=seed, std=std)
    if not llama_c._SO.exists():
        pytest.skip("oracle/libstrata_oracle.so not built (make -C oracle/c)")
    return w, llama_c.CLlama(cfg, w)


@pytest.mark.parametrize("name,seed,n_prompt,n_new", [
    ("mha", 1, 7, 10), ("gqa", 2, 19, 12), ("gqa_hd128", 3, 33, 8), ("gqa", 4, 1, 6)])
def test_c_decoder_greedy_ids_match_numpy_oracle(name, seed, n_prompt, n_new):
    cfg = CFGS[name]
    w, cm = _model(cfg, seed)
    prompt = np.random.default_rng(seed).integers(0, cfg.vocab_size, (1, n_prompt))
    ids, margins, last = cm.generate(prompt, n_new)
    ref = oll.OracleLlama(cfg, w)
    exp = oll.greedy_generate(ref, prompt, max_new_tokens=n_new,
                              cache=OracleKVCache(cfg.num_hidden_layers))
    assert np.array_equal(ids, exp[0]), f"\n{ids}\n{exp[0]}"
    assert margins.shape == (n_new,) and (margins >= 0).all()
    # the logits that picked the last token: one cached forward over the prefix
    cache = OracleKVCache(cfg.num_hidden_layers)
    ref.forward(exp[:, :-2], cache, use_cache=True)
    lg = ref.forward(exp[:, -2:-1], cache, use_cache=True)[0, -1]
    assert np.max(np.abs(last - lg)) <= 1e-5 * np.max(np.abs(lg)) + 1e-7
    assert int(np.argmax(lg)) == ids[-1]


def test_c_decoder_tied_head_and_bad_arguments():
    cfg = CFGS["mha"]
    w, _ = _model(cfg, 5)
    w = dict(w)
    del w["lm_head"]
    cm = llama_c.CLlama(cfg, w)
    prompt = np.array([[3, 1, 4, 1, 5]])
    ids, _, _ = cm.generate(prompt, 5)
    exp = oll.greedy_generate(oll.OracleLlama(cfg, w), prompt, max_new_tokens=5,
                              cache=OracleKVCache(cfg.num_hidden_layers))
    assert np.array_equal(ids, exp[0])
    with pytest.raises(ValueError):
        cm.generate(np.array([[cfg.vocab_size]]), 2)
    with pytest.raises(ValueError):
        cm.generate(np.zeros((1, 0), dtype=np.int64), 2)
    assert np.array_equal(cm.generate(prompt, 0)[0], prompt[0])


def test_c_decoder_step_by_step_prompt_equals_prefill():
    """Feeding the prompt one token at a time gives the same ids as one
    prefill (the cached decode == full forward contract,
    tests/test_mlx_generation.py:140-156), with the float64 linears making
    the two paths agree to the last bit of the chosen ids."""
    cfg = CFGS["gqa"]
    w, cm = _model(cfg, 6)
    prompt = np.random.default_rng(6).integers(0, cfg.vocab_size, (1, 9))
    ids, _, _ = cm.generate(prompt, 6)
    ref = oll.OracleLlama(cfg, w)
    cache = OracleKVCache(cfg.num_hidden_layers)
    for t in range(prompt.shape[1] - 1):
        ref.forward(prompt[:, t:t + 1], cache, use_cache=True)
    seq = list(prompt[0])
    nxt = prompt[:, -1:]
    for _ in range(6):
        lg = ref.forward(nxt, cache, use_cache=True)[0, -1]
        seq.append(int(np.argmax(lg)))
        nxt = np.array([[seq[-1]]])
    assert np.array_equal(ids, np.array(seq))
