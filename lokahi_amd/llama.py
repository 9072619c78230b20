"""Llama decoder driver over the HIP hot path.

Reproduces the reference's model adapter around the replaced ops:
``MLXLlamaDecoderLayer.__call__`` (``src/ollm/llama_mlx.py:608-658``),
``MLXLlamaAttention.__call__`` (220-342), ``MLXLlamaMLP`` (345-432),
``MLXLlamaModel.__call__`` (740-833), ``MLXLlamaForCausalLM.__call__``
(863-912) and ``greedy_generate_mx`` (``src/ollm/generation.py:7-50``).

Every op is a libstrata_hip.so kernel: embedding gather, fused
residual-add + RMSNorm, one q4 launch for q/k/v and one for gate/up, fused
RoPE + KV append, split-K (decode) or MFMA (prefill) attention, SiLU*up,
bf16 (or q4) lm_head GEMV and device argmax.  Activations are bf16 between ops
(the "bf16" dtype flow); logits are fp32.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional

import torch

from . import ops
from .kvcache import HipKVCache

LINEARS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


@dataclass
class LlamaConfig:
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
        return self.hidden_size // self.num_attention_heads  # llama_mlx.py:448


LLAMA3_8B = LlamaConfig(128256, 4096, 14336, 32, 32, 8, 1e-5, 500000.0)
LLAMA32_3B = LlamaConfig(128256, 3072, 8192, 28, 24, 8, 1e-5, 500000.0)


def weights_to_device(weights: Dict[str, "object"], device: int = 0) -> Dict[str, torch.Tensor]:
    """Upload a host weight dict (uint32 packed, uint16 bf16 bits) to the device."""
    import numpy as np
    out: Dict[str, torch.Tensor] = {}
    dev = torch.device("cuda", device)
    for name, arr in weights.items():
        a = np.ascontiguousarray(arr)
        if a.dtype == np.uint16:
            t = torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)
        elif a.dtype == np.uint32:
            t = torch.from_numpy(a.view(np.int32)).view(torch.uint32)
        else:
            t = torch.from_numpy(a)
        out[name] = t.to(dev)
    return out


def random_weights(cfg: LlamaConfig, seed: int, std: float = 0.02,
                   device: int = 0) -> Dict[str, torch.Tensor]:
    """Seeded random-init weights generated and quantized on the device.

    Linears ~ N(0, std) quantized to q4 group-64 by the library's quantizer;
    embedding and lm_head ~ N(0, std) in bf16; norm weights are ones.
    """
    dev = torch.device("cuda", device)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    hs, fs = cfg.hidden_size, cfg.intermediate_size
    hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    shapes = {"q_proj": (hq * d, hs), "k_proj": (hkv * d, hs), "v_proj": (hkv * d, hs),
              "o_proj": (hs, hq * d), "gate_proj": (fs, hs), "up_proj": (fs, hs),
              "down_proj": (hs, fs)}
    w: Dict[str, torch.Tensor] = {}

    def normal(shape, dtype=torch.float32):
        return (torch.randn(shape, generator=gen, device=dev, dtype=torch.float32) * std).to(dtype)

    w["embed_tokens"] = normal((cfg.vocab_size, hs), torch.bfloat16)
    ones = torch.ones(hs, dtype=torch.bfloat16, device=dev)
    for li in range(cfg.num_hidden_layers):
        p = f"layers.{li}."
        for name, shp in shapes.items():
            src = normal(shp)
            pw, sc, bi = ops.quantize(src, cfg.group_size)
            del src
            w[p + name + ".weight"], w[p + name + ".scales"], w[p + name + ".biases"] = pw, sc, bi
        w[p + "input_layernorm"] = ones.clone()
        w[p + "post_attention_layernorm"] = ones.clone()
    w["norm"] = ones.clone()
    w["lm_head"] = normal((cfg.vocab_size, hs), torch.bfloat16)
    return w


class HipLlamaForCausalLM:
    def __init__(self, config: LlamaConfig, weights: Dict[str, torch.Tensor], device: int = 0):
        self.config = config
        self.w = weights
        self.device = torch.device("cuda", device)

    def _q4(self, name: str):
        return self.w[name + ".weight"], self.w[name + ".scales"], self.w[name + ".biases"]

    def new_cache(self, batch_size: int = 1, max_length: int = 4096) -> HipKVCache:
        return HipKVCache(self.config, batch_size=batch_size, max_length=max_length,
                          dtype=torch.bfloat16, device=self.device.index or 0)

    @torch.no_grad()
    def __call__(self, input_ids: torch.Tensor, past_key_values: Optional[HipKVCache] = None,
                 use_cache: bool = False, logits: str = "all") -> torch.Tensor:
        cfg = self.config
        ids = input_ids.to(self.device)
        B, L = ids.shape
        hq, d, H = cfg.num_attention_heads, cfg.head_dim, cfg.hidden_size
        g = cfg.group_size
        cache = past_key_values if use_cache else None
        if cache is None:  # a private cache holding just this call's keys
            cache = self.new_cache(B, L)
        past = cache.get_seq_length()
        positions = torch.arange(past, past + L, dtype=torch.int32, device=self.device)

        h = ops.embed(self.w["embed_tokens"], ids)  # [B, L, H] bf16
        delta = None
        for li in range(cfg.num_hidden_layers):
            p = f"layers.{li}."
            xn = ops.rmsnorm(h, self.w[p + "input_layernorm"], cfg.rms_norm_eps, residual=delta)
            q, k, v = ops.linear_multi(xn, [self._q4(p + "q_proj"), self._q4(p + "k_proj"),
                                            self._q4(p + "v_proj")], group_size=g)
            qr = torch.empty((B, hq, L, d), dtype=torch.bfloat16, device=self.device)
            cache.rope_append(li, q, k, v, hq, L, cfg.rope_theta, qr)
            kview, vview = cache.views(li)
            attn = ops.attention(qr, kview, vview, query_positions=positions[None, :].expand(B, L),
                                 causal=True, q_block_size=32768,
                                 k_block_size=(1024 if L > 128 else 1000000),
                                 kv_strides=cache.kv_strides)
            attn_tm = attn.transpose(1, 2).reshape(B, L, hq * d)
            o = ops.linear(attn_tm, *self._q4(p + "o_proj"), group_size=g)
            xn = ops.rmsnorm(h, self.w[p + "post_attention_layernorm"], cfg.rms_norm_eps,
                             residual=o)
            gate, up = ops.linear_multi(xn, [self._q4(p + "gate_proj"), self._q4(p + "up_proj")],
                                        group_size=g)
            a = ops.silu_mul(gate, up)
            delta = ops.linear(a, *self._q4(p + "down_proj"), group_size=g)
        hn = ops.rmsnorm(h, self.w["norm"], cfg.rms_norm_eps, residual=delta)
        if logits == "last":
            hn = hn[:, -1:, :].contiguous()
        if "lm_head.weight" in self.w:  # q4 head (MLX 4-bit checkpoint, maybe tied)
            return ops.linear(hn, *self._q4("lm_head"), group_size=g, out_dtype=torch.float32)
        return ops.linear(hn, self.w["lm_head"], None, None, out_dtype=torch.float32)

    def generate(self, input_ids: torch.Tensor, max_new_tokens: int = 100,
                 temperature: float = 1.0, past_key_values: Optional[HipKVCache] = None,
                 engine: bool = True, use_graph: bool = False):
        """Greedy generation (``generation.py:7-50``).

        ``engine=True`` runs the native decoder (prefill + decode steps
        launched from C++, tokens chosen on the device); ``engine=False``
        drives the same kernels op by op from Python.  ``use_graph=True``
        replays each decode step as a captured HIP graph instead: the same
        kernels and tokens, with no host launches per step, but 7-11% fewer
        tok/s than direct launches on ROCm 7 (MI355X, 8B and 3B shapes).
        """
        if not engine:
            return greedy_generate(self, input_ids, max_new_tokens=max_new_tokens,
                                   temperature=temperature, past_key_values=past_key_values)
        if max_new_tokens < 0:
            raise ValueError("max_new_tokens must be non-negative")
        if temperature <= 0:
            raise ValueError("temperature must be positive")
        if input_ids.ndim != 2 or input_ids.shape[1] == 0:
            raise ValueError("input_ids must have shape [batch, sequence] with sequence > 0")
        if max_new_tokens == 0:
            return input_ids
        B, L = input_ids.shape
        cache = past_key_values
        if cache is None:
            cache = self.new_cache(B, L + max_new_tokens)
        dec = DecoderEngine(self, cache, max_batch=B, max_tokens=B * L)
        return dec.generate(input_ids, max_new_tokens, temperature, use_graph)


@torch.no_grad()
def greedy_generate(model, input_ids: torch.Tensor, *, max_new_tokens: int,
                    temperature: float = 1.0, past_key_values=None) -> torch.Tensor:
    """One prompt prefill, then one-token cached decodes (generation.py:7-50)."""
    if max_new_tokens < 0:
        raise ValueError("max_new_tokens must be non-negative")
    if temperature <= 0:
        raise ValueError("temperature must be positive")
    if input_ids.ndim != 2 or input_ids.shape[1] == 0:
        raise ValueError("input_ids must have shape [batch, sequence] with sequence > 0")
    if max_new_tokens == 0:
        return input_ids
    cache = past_key_values
    if cache is None:
        cache = model.new_cache(input_ids.shape[0], input_ids.shape[1] + max_new_tokens)
    generated = input_ids
    model_input = input_ids
    for _ in range(max_new_tokens):
        logits = model(model_input, past_key_values=cache, use_cache=True, logits="last")
        last = logits[:, -1, :]
        if temperature != 1.0:
            last = (last / temperature).contiguous()
        nxt = ops.argmax(last).to(torch.int64)[:, None]
        generated = torch.cat([generated.to(nxt.device), nxt], dim=1)
        model_input = nxt
    return generated


class DecoderEngine:
    """ctypes handle of the native ``strata_decoder`` for one model + KV cache."""

    def __init__(self, model: "HipLlamaForCausalLM", cache: HipKVCache, max_batch: int = 1,
                 max_tokens: int = 4096):
        import ctypes as C
        from . import _abi
        from .ops import _ctx
        cfg = model.config
        w = model.w
        self.model, self.cache = model, cache
        self._lib = _abi.load()
        dev = model.device.index or 0

        def q4(name):
            t = w[name + ".weight"]
            return _abi.Q4Weight(t.data_ptr(), w[name + ".scales"].data_ptr(),
                                 w[name + ".biases"].data_ptr(), t.shape[0], None)

        layers = (_abi.LlamaLayerC * cfg.num_hidden_layers)()
        for li in range(cfg.num_hidden_layers):
            p = f"layers.{li}."
            layers[li] = _abi.LlamaLayerC(
                w[p + "input_layernorm"].data_ptr(), w[p + "post_attention_layernorm"].data_ptr(),
                *[q4(p + n) for n in LINEARS])
        ccfg = _abi.LlamaConfigC(cfg.vocab_size, cfg.hidden_size, cfg.intermediate_size,
                                 cfg.num_hidden_layers, cfg.num_attention_heads,
                                 cfg.num_key_value_heads, cfg.head_dim, cfg.group_size,
                                 cfg.rms_norm_eps, cfg.rope_theta)
        h = C.c_void_p()
        q4_head = "lm_head.weight" in w
        _abi.check(self._lib.strata_decoder_create(
            _ctx(dev), C.byref(ccfg), w["embed_tokens"].data_ptr(), w["norm"].data_ptr(),
            None if q4_head else w["lm_head"].data_ptr(), layers, cache.handle, max_batch,
            max_tokens, C.byref(h)))
        self.handle = h
        if q4_head:
            head = q4("lm_head")
            _abi.check(self._lib.strata_decoder_set_lm_head_q4(h, C.byref(head)))
        self._layers = layers  # keep the struct array alive with the handle
        self.vocab = cfg.vocab_size
        self._outs = {}

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        """Last-position fp32 logits [B, vocab] for ids [B, L] appended to the cache."""
        import ctypes as C
        from . import _abi
        from .ops import _stream
        self.cache.load_offloaded_layers()
        ids32 = ids.to(device=self.model.device, dtype=torch.int32).contiguous()
        B, L = ids32.shape
        out = torch.empty((B, self.vocab), dtype=torch.float32, device=self.model.device)
        _abi.check(self._lib.strata_decoder_forward(self.handle, ids32.data_ptr(), B, L,
                                                    out.data_ptr(),
                                                    _stream(self.model.device.index or 0)))
        return out

    def generate(self, prompt: torch.Tensor, max_new: int, temperature: float = 1.0,
                 use_graph: bool = False) -> torch.Tensor:
        from . import _abi
        from .ops import _stream
        self.cache.load_offloaded_layers()
        ids32 = prompt.to(device=self.model.device, dtype=torch.int32).contiguous()
        B, L = ids32.shape
        # one output buffer per (B, max_new), reused across calls
        key = (B, max_new)
        if key not in self._outs:
            self._outs[key] = torch.empty((B, max_new), dtype=torch.int32,
                                          device=self.model.device)
        out = self._outs[key]
        _abi.check(self._lib.strata_decoder_generate(
            self.handle, ids32.data_ptr(), B, L, max_new, float(temperature),
            1 if use_graph else 0, out.data_ptr(), _stream(self.model.device.index or 0)))
        return torch.cat([prompt.to(out.device, torch.int64), out.to(torch.int64)], dim=1)

    def __del__(self):
        try:
            if getattr(self, "handle", None):
                self._lib.strata_decoder_destroy(self.handle)
                self.handle = None
        except Exception:
            pass
