"""Write oracle weights as an MLX 4-bit Llama checkpoint directory (test fixture).

Tensor names follow ``src/ollm/llama_mlx.py:470-495`` and ``740-912``; the
config carries ``quantization = {group_size: 64, bits: 4}`` as MLX 4-bit
checkpoints do.  ``embed`` is "bf16" or "q4"; ``head`` is "bf16", "q4" or
"tied" (no ``lm_head`` tensor).  Returns the oracle weight dict that
describes the same model (triples under ``embed_tokens.*`` / ``lm_head.*``).
"""
import json
from pathlib import Path

import numpy as np

from lokahi_amd.loader import write_safetensors
from oracle import q4
from oracle.bf16 import bf16_bits_to_f32

PROJ = {"q_proj": "self_attn", "k_proj": "self_attn", "v_proj": "self_attn", "o_proj": "self_attn",
        "gate_proj": "mlp", "up_proj": "mlp", "down_proj": "mlp"}


def export(model_dir, cfg, hw, *, embed="bf16", head="bf16", extra_config=None):
    model_dir = Path(model_dir)
    model_dir.mkdir(parents=True, exist_ok=True)
    ow = dict(hw)
    t = {}
    if embed == "q4":
        trip = q4.quantize(bf16_bits_to_f32(hw["embed_tokens"]), cfg.group_size)
        del ow["embed_tokens"]
        for suf, a in zip(("weight", "scales", "biases"), trip):
            ow["embed_tokens." + suf] = a
            t["model.embed_tokens." + suf] = ("U32" if suf == "weight" else "BF16", a)
    else:
        t["model.embed_tokens.weight"] = ("BF16", hw["embed_tokens"])
    if head == "q4":
        trip = q4.quantize(bf16_bits_to_f32(hw["lm_head"]), cfg.group_size)
        del ow["lm_head"]
        for suf, a in zip(("weight", "scales", "biases"), trip):
            ow["lm_head." + suf] = a
            t["lm_head." + suf] = ("U32" if suf == "weight" else "BF16", a)
    elif head == "bf16":
        t["lm_head.weight"] = ("BF16", hw["lm_head"])
    else:
        del ow["lm_head"]
    t["model.norm.weight"] = ("BF16", hw["norm"])
    for i in range(cfg.num_hidden_layers):
        p, base = f"layers.{i}.", f"model.layers.{i}."
        t[base + "input_layernorm.weight"] = ("BF16", hw[p + "input_layernorm"])
        t[base + "post_attention_layernorm.weight"] = ("BF16", hw[p + "post_attention_layernorm"])
        for lin, sub in PROJ.items():
            for suf in ("weight", "scales", "biases"):
                t[f"{base}{sub}.{lin}.{suf}"] = ("U32" if suf == "weight" else "BF16",
                                                  hw[f"{p}{lin}.{suf}"])
    # two shards with an index, as multi-file MLX checkpoints are laid out
    names = sorted(t)
    half = len(names) // 2
    shards = {"model-00001-of-00002.safetensors": names[:half],
              "model-00002-of-00002.safetensors": names[half:]}
    for fname, part in shards.items():
        write_safetensors(model_dir / fname, {n: t[n] for n in part}, {"format": "mlx"})
    (model_dir / "model.safetensors.index.json").write_text(json.dumps(
        {"metadata": {}, "weight_map": {n: f for f, part in shards.items() for n in part}}))
    conf = {"model_type": "llama", "vocab_size": cfg.vocab_size, "hidden_size": cfg.hidden_size,
            "intermediate_size": cfg.intermediate_size,
            "num_hidden_layers": cfg.num_hidden_layers,
            "num_attention_heads": cfg.num_attention_heads,
            "num_key_value_heads": cfg.num_key_value_heads, "rms_norm_eps": cfg.rms_norm_eps,
            "rope_theta": cfg.rope_theta, "tie_word_embeddings": head == "tied",
            "quantization": {"group_size": cfg.group_size, "bits": 4}}
    conf.update(extra_config or {})
    (model_dir / "config.json").write_text(json.dumps(conf))
    return ow
