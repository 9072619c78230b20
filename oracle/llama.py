"""Llama decoder + greedy-generation oracle (test infrastructure).

Restates the reference's model adapter around the hot-path ops:

* ``MLXRMSNorm`` (``src/ollm/llama_mlx.py:77-92``),
* ``MLXLlamaAttention.__call__`` (220-342): q/k/v ``_linear`` (257-268),
  reshape to ``[B, H, L, D]`` (271-281), RoPE (284-286), cache update
  (289-297), chunked attention with ``q_block=32768`` and
  ``k_block = 1024 if L > 128 else 1e6`` (300-308), o_proj (313-316),
* ``MLXLlamaMLP`` (345-432): ``down(silu(gate(x)) * up(x))``,
* ``MLXLlamaDecoderLayer.__call__`` (608-658): pre-norm residual blocks,
* ``MLXLlamaModel.__call__`` (740-833): embedding gather, ``cache_position =
  arange(past, past + L)``, final norm,
* ``MLXLlamaForCausalLM.__call__`` (863-912): lm_head,
* ``greedy_generate_mx`` (``src/ollm/generation.py:7-50``).

Dtype flow (the "bf16" flow this build's decode driver implements): every
activation tensor that crosses an op boundary is rounded to bf16 (hidden
states, q/k/v, the KV cache, attention output, MLP intermediates), while each
op computes internally in fp32 (RMSNorm, RoPE, attention, SiLU) or in float64
here / fp32 on the GPU (the linears).  Logits are fp32 (bf16 lm_head weights,
fp32 accumulation) so that the greedy argmax is not decided by bf16 ties.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional

import numpy as np

from . import attention as attn
from . import q4, rope
from .bf16 import bf16_bits_to_f32, round_bf16
from .kvcache import OracleKVCache


@dataclass
class Config:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    rms_norm_eps: float = 1e-5
    rope_theta: float = 500000.0
    group_size: int = 64

    @property
    def head_dim(self) -> int:
        # llama_mlx.py:448 head_dim = hidden // heads
        return self.hidden_size // self.num_attention_heads


def rms_norm(x: np.ndarray, weight_bits: np.ndarray, eps: float) -> np.ndarray:
    """fp32 RMSNorm of bf16-valued ``x`` (``llama_mlx.py:77-92``), rounded to bf16.

    Operand order follows the uncompiled branch (``llama_mlx.py:89-91``:
    ``x * rsqrt(var + eps)`` then ``weight * x``); the compiled branch
    (``metal_optimizations.py:96``) forms ``weight * x`` first.  The two
    differ by at most one fp32 rounding before the bf16 rounding.  Pinned
    against torch's fp32 ``rms_norm`` and a float64 closed form in
    ``tests/test_oracle_pins.py``."""
    x = np.asarray(x, dtype=np.float32)
    var = np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True)
    r = (1.0 / np.sqrt(var + eps)).astype(np.float32)
    w = bf16_bits_to_f32(weight_bits)
    return round_bf16((x * r).astype(np.float32) * w)


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """``silu(g) * u`` in fp32, rounded to bf16 (``llama_mlx.py:399-407``)."""
    g = g.astype(np.float64)
    with np.errstate(over="ignore"):  # exp(-g) = inf for g << 0 gives silu = -0
        return round_bf16((g / (1.0 + np.exp(-g)) * u).astype(np.float32))


class OracleLlama:
    """NumPy Llama with q4 linears; embedding and lm_head bf16 or q4.

    Weight names: ``embed_tokens`` (bf16 bits) or the triple
    ``embed_tokens.weight/.scales/.biases`` (gathered rows dequantized and
    rounded to bf16, as ``mx.dequantize`` returns them, ``llama_mlx.py:722-738``;
    the exact rounding of MLX's dequantize is parity unpinned: it is taken as
    one RNE rounding of the exact ``s*q + b``); ``lm_head`` (bf16 bits) or the
    triple ``lm_head.weight/...``; with neither, the head is tied to the
    embedding (``llama_mlx.py:886-910``)."""

    def __init__(self, cfg: Config, weights: Dict[str, np.ndarray]):
        self.cfg = cfg
        self.w = weights
        # dequantize once (float64) for speed on repeated calls
        self._deq: Dict[str, np.ndarray] = {}

    def _lin(self, x: np.ndarray, name: str) -> np.ndarray:
        if name not in self._deq:
            self._deq[name] = q4.dequantize(self.w[name + ".weight"], self.w[name + ".scales"],
                                            self.w[name + ".biases"], self.cfg.group_size)
        return round_bf16((x.astype(np.float64) @ self._deq[name].T).astype(np.float32))

    def forward(self, ids: np.ndarray, cache: Optional[OracleKVCache] = None,
                use_cache: bool = True) -> np.ndarray:
        cfg = self.cfg
        ids = np.asarray(ids)
        b, L = ids.shape
        hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        h = self._embed(ids)                                               # [B, L, H]
        active = cache if use_cache else None
        past = active.get_seq_length() if active is not None else 0
        cache_position = np.arange(past, past + L, dtype=np.int32)
        position_ids = np.broadcast_to(cache_position[None, :], (b, L))
        cos, sin = rope.cos_sin(position_ids, d, cfg.rope_theta)
        for li in range(cfg.num_hidden_layers):
            p = f"layers.{li}."
            xn = rms_norm(h, self.w[p + "input_layernorm"], cfg.rms_norm_eps)
            q = self._lin(xn, p + "q_proj").reshape(b, L, hq, d).transpose(0, 2, 1, 3)
            k = self._lin(xn, p + "k_proj").reshape(b, L, hkv, d).transpose(0, 2, 1, 3)
            v = self._lin(xn, p + "v_proj").reshape(b, L, hkv, d).transpose(0, 2, 1, 3)
            q = round_bf16(rope.apply(q, cos, sin))
            k = round_bf16(rope.apply(k, cos, sin))
            if active is not None:
                k, v = active.update(k, v, li, {"cache_position": cache_position})
            o = attn.chunked_gqa(q, k, v, query_positions=position_ids, causal=True,
                                 q_block_size=32768,
                                 k_block_size=(1024 if L > 128 else 1000000))
            o = round_bf16(o).transpose(0, 2, 1, 3).reshape(b, L, hq * d)
            h = round_bf16(h + self._lin(o, p + "o_proj"))
            xn = rms_norm(h, self.w[p + "post_attention_layernorm"], cfg.rms_norm_eps)
            a = silu_mul(self._lin(xn, p + "gate_proj"), self._lin(xn, p + "up_proj"))
            h = round_bf16(h + self._lin(a, p + "down_proj"))
        hn = rms_norm(h, self.w["norm"], cfg.rms_norm_eps)
        return self._head(hn)

    def _embed(self, ids: np.ndarray) -> np.ndarray:
        if "embed_tokens" in self.w:
            return bf16_bits_to_f32(self.w["embed_tokens"][ids])
        rows = q4.dequantize(self.w["embed_tokens.weight"][ids.reshape(-1)],
                             self.w["embed_tokens.scales"][ids.reshape(-1)],
                             self.w["embed_tokens.biases"][ids.reshape(-1)], self.cfg.group_size)
        return round_bf16(rows.astype(np.float32)).reshape(*ids.shape, -1)

    def _head(self, hn: np.ndarray) -> np.ndarray:
        """fp32 logits: bf16 head, q4 head, or the tied embedding (bf16 or q4)."""
        if "head_f64" not in self._deq:
            w = self.w
            if "lm_head" in w:
                m = bf16_bits_to_f32(w["lm_head"]).astype(np.float64)
            elif "lm_head.weight" in w:
                m = q4.dequantize(w["lm_head.weight"], w["lm_head.scales"], w["lm_head.biases"],
                                  self.cfg.group_size)
            elif "embed_tokens" in w:
                m = bf16_bits_to_f32(w["embed_tokens"]).astype(np.float64)
            else:
                m = q4.dequantize(w["embed_tokens.weight"], w["embed_tokens.scales"],
                                  w["embed_tokens.biases"], self.cfg.group_size)
            self._deq["head_f64"] = m
        return (hn.astype(np.float64) @ self._deq["head_f64"].T).astype(np.float32)


def greedy_generate(model, input_ids: np.ndarray, *, max_new_tokens: int,
                    temperature: float = 1.0, cache=None) -> np.ndarray:
    """Prefill once, then one-token cached decodes (``generation.py:7-50``)."""
    input_ids = np.asarray(input_ids)
    if max_new_tokens < 0:
        raise ValueError("max_new_tokens must be non-negative")
    if temperature <= 0:
        raise ValueError("temperature must be positive")
    if input_ids.ndim != 2 or input_ids.shape[1] == 0:
        raise ValueError("input_ids must have shape [batch, sequence] with sequence > 0")
    if max_new_tokens == 0:
        return input_ids
    if cache is None:
        cache = OracleKVCache(getattr(getattr(model, "cfg", None), "num_hidden_layers", None))
    generated = input_ids
    model_input = input_ids
    for _ in range(max_new_tokens):
        logits = model.forward(model_input, cache, use_cache=True) if hasattr(model, "forward") \
            else model(model_input, past_key_values=cache, use_cache=True)
        nxt = np.argmax(np.asarray(logits)[:, -1, :] / temperature, axis=-1)[:, None]
        generated = np.concatenate([generated, nxt.astype(generated.dtype)], axis=1)
        model_input = nxt.astype(generated.dtype)
    return generated


def random_weights(cfg: Config, seed: int, std: float = 0.02) -> Dict[str, np.ndarray]:
    """Seeded random-init weights (q4 linears, bf16 norms/embedding/lm_head).

    Test-scale helper: draws N(0, std) float32 weights with NumPy and
    quantizes them with ``q4.quantize``; norm weights are ones.
    """
    from .bf16 import f32_to_bf16_bits
    rng = np.random.default_rng(seed)
    hs, fs = cfg.hidden_size, cfg.intermediate_size
    hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    w: Dict[str, np.ndarray] = {}
    w["embed_tokens"] = f32_to_bf16_bits(rng.normal(0, std, (cfg.vocab_size, hs)).astype(np.float32))
    shapes = {"q_proj": (hq * d, hs), "k_proj": (hkv * d, hs), "v_proj": (hkv * d, hs),
              "o_proj": (hs, hq * d), "gate_proj": (fs, hs), "up_proj": (fs, hs),
              "down_proj": (hs, fs)}
    ones = f32_to_bf16_bits(np.ones(hs, dtype=np.float32))
    for li in range(cfg.num_hidden_layers):
        p = f"layers.{li}."
        for name, shp in shapes.items():
            pw, s, bb = q4.quantize(rng.normal(0, std, shp).astype(np.float32), cfg.group_size)
            w[p + name + ".weight"], w[p + name + ".scales"], w[p + name + ".biases"] = pw, s, bb
        w[p + "input_layernorm"] = ones.copy()
        w[p + "post_attention_layernorm"] = ones.copy()
    w["norm"] = ones.copy()
    w["lm_head"] = f32_to_bf16_bits(rng.normal(0, std, (cfg.vocab_size, hs)).astype(np.float32))
    return w


def flatten_names(cfg: Config) -> List[str]:
    names = ["embed_tokens", "norm", "lm_head"]
    for li in range(cfg.num_hidden_layers):
        p = f"layers.{li}."
        names += [p + "input_layernorm", p + "post_attention_layernorm"]
        for n in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"):
            names += [p + n + ".weight", p + n + ".scales", p + n + ".biases"]
    return names


def random_q4_weights(cfg: Config, seed: int, scale: float = 0.0067,
                      embed_std: float = 0.02) -> Dict[str, np.ndarray]:
    """Seeded full-size weights drawn directly in the q4 format (test helper).

    Codes are uniform 0..15; per group ``s = scale * (1 + 0.1 n1)`` and
    ``b = -7.5 s (1 + 0.05 n2)`` (bf16), which gives weights of std ~0.03
    centred near 0, as a group-64 quantization of N(0, 0.02) would; embedding
    and lm_head are N(0, 0.02) bf16 (truncated draws), norms ones.  Skips ``quantize`` so that a
    28-layer 3B model is drawn in seconds."""
    rng = np.random.default_rng(seed)
    hs, fs = cfg.hidden_size, cfg.intermediate_size
    hq, hkv, d, g = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.group_size
    shapes = {"q_proj": (hq * d, hs), "k_proj": (hkv * d, hs), "v_proj": (hkv * d, hs),
              "o_proj": (hs, hq * d), "gate_proj": (fs, hs), "up_proj": (fs, hs),
              "down_proj": (hs, fs)}

    def bf16(x):  # truncation: any bit pattern is a valid draw, and it is fast
        return (np.ascontiguousarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)

    def normal(shape, std):
        return bf16(rng.standard_normal(shape, dtype=np.float32) * np.float32(std))

    w: Dict[str, np.ndarray] = {"embed_tokens": normal((cfg.vocab_size, hs), embed_std)}
    ones = bf16(np.ones(hs, dtype=np.float32))
    for li in range(cfg.num_hidden_layers):
        p = f"layers.{li}."
        for name, (n, k) in shapes.items():
            s = np.float32(scale) * (1 + np.float32(0.1) * rng.standard_normal((n, k // g), dtype=np.float32))
            b = np.float32(-7.5) * s * (1 + np.float32(0.05) * rng.standard_normal((n, k // g), dtype=np.float32))
            w[p + name + ".weight"] = rng.integers(0, 2 ** 32, (n, k // 8), dtype=np.uint32)
            w[p + name + ".scales"] = bf16(s)
            w[p + name + ".biases"] = bf16(b)
        w[p + "input_layernorm"] = ones
        w[p + "post_attention_layernorm"] = ones
    w["norm"] = ones
    w["lm_head"] = normal((cfg.vocab_size, hs), 0.02)
    return w
