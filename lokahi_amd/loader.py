"""MLX 4-bit Llama checkpoints -> device weights for the HIP path.

Reads what the reference loads for this path:

* safetensors files as ``SafeTensorMLXReader`` reads them
  (``src/ollm/mlx_loader.py:260-335``): an 8-byte little-endian header
  length, a JSON header of ``{name: {dtype, shape, data_offsets}}``
  (``__metadata__`` skipped), data after the header; dtypes F32, F16, BF16
  (kept as uint16 bit patterns), U32, I32, I8; an unknown name is a
  ``KeyError``;
* the quantization parameters of ``_quantization_parameters``
  (``llama_mlx.py:40-50``): ``config.quantization`` or
  ``config.quantization_config`` with ``group_size``, ``bits`` and ``mode``
  (default ``"affine"``);
* the parameter names of the decoder layers (``llama_mlx.py:470-495``):
  ``model.layers.{i}.self_attn.{q,k,v,o}_proj`` and
  ``model.layers.{i}.mlp.{gate,up,down}_proj`` as ``.weight`` (U32 packed)
  + ``.scales`` + ``.biases`` (BF16), the two layer norms,
  ``model.embed_tokens`` (BF16, or quantized and expanded with
  ``mx.dequantize`` at gather time, 722-738), ``model.norm`` and
  ``lm_head`` (BF16 or quantized), which falls back to the embedding when the
  checkpoint ties them (886-910).

The HIP path runs 4-bit group-64 affine linears only: other quantization
settings and dense linears are rejected with ``ValueError``.  A quantized
embedding table is expanded once on the device (``strata_dequantize_q4``;
element-wise, so gathering rows of the expanded table equals dequantizing
gathered rows); a quantized or tied-quantized head stays q4 and runs on the
q4 GEMV.
"""
from __future__ import annotations

import json
import struct
import warnings
from pathlib import Path
from typing import Dict, Iterable, List, Optional, Tuple

import numpy as np

from .llama import LINEARS, HipLlamaForCausalLM, LlamaConfig

# safetensors dtype -> numpy storage dtype (BF16 as its uint16 bit pattern)
NP_DTYPES = {
    "F32": np.float32,
    "F16": np.float16,
    "BF16": np.uint16,
    "U32": np.uint32,
    "I32": np.int32,
    "I8": np.int8,
}
_DTYPE_OF = {np.dtype(np.float32): "F32", np.dtype(np.float16): "F16",
             np.dtype(np.uint32): "U32", np.dtype(np.int32): "I32", np.dtype(np.int8): "I8"}

_PROJ_PREFIX = {"q_proj": "self_attn", "k_proj": "self_attn", "v_proj": "self_attn",
                "o_proj": "self_attn", "gate_proj": "mlp", "up_proj": "mlp", "down_proj": "mlp"}


class SafeTensorReader:
    """Header-indexed reader of one ``.safetensors`` file (memory-mapped)."""

    def __init__(self, path):
        self.path = Path(path)
        with open(self.path, "rb") as f:
            (header_len,) = struct.unpack("<Q", f.read(8))
            self.header = json.loads(f.read(header_len))
        self.data_offset = 8 + header_len
        self._map = np.memmap(self.path, dtype=np.uint8, mode="r")

    def keys(self) -> List[str]:
        return [k for k in self.header if k != "__metadata__"]

    def dtype(self, name: str) -> str:
        return self._info(name)["dtype"]

    def _info(self, name: str) -> dict:
        if name not in self.header or name == "__metadata__":
            raise KeyError(f"Tensor '{name}' not found in {self.path}")
        return self.header[name]

    def get(self, name: str) -> np.ndarray:
        """The tensor as a host array (BF16 -> uint16 bits), copied out of the map."""
        info = self._info(name)
        dt = info["dtype"]
        if dt not in NP_DTYPES:
            raise ValueError(f"unsupported safetensors dtype {dt} for '{name}'")
        off0, off1 = info["data_offsets"]
        shape = tuple(info["shape"])
        raw = self._map[self.data_offset + off0:self.data_offset + off1]
        arr = raw.view(NP_DTYPES[dt])
        if arr.size != int(np.prod(shape, dtype=np.int64)):
            raise ValueError(f"'{name}': {off1 - off0} bytes do not hold {dt}{list(shape)}")
        return np.array(arr.reshape(shape))


def write_safetensors(path, tensors: Dict[str, Tuple[str, np.ndarray]],
                      metadata: Optional[Dict[str, str]] = None) -> None:
    """Write ``{name: (dtype, array)}`` in the safetensors layout (BF16 arrays
    are uint16 bit patterns).  Tensors are stored in name order, 8-byte aligned."""
    header: Dict[str, object] = {}
    if metadata:
        header["__metadata__"] = dict(metadata)
    blobs = []
    off = 0
    for name in sorted(tensors):
        dt, arr = tensors[name]
        a = np.ascontiguousarray(arr)
        if dt == "BF16":
            if a.dtype != np.uint16:
                raise ValueError(f"'{name}': BF16 data must be uint16 bit patterns")
        elif NP_DTYPES.get(dt) != a.dtype.type:
            raise ValueError(f"'{name}': array dtype {a.dtype} does not match {dt}")
        b = a.tobytes()
        header[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    hb = json.dumps(header, separators=(",", ":")).encode()
    hb += b" " * (-len(hb) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for b in blobs:
            f.write(b)


def quantization_parameters(config: dict) -> Tuple[Optional[int], Optional[int], str]:
    """``(group_size, bits, mode)`` as ``llama_mlx.py:40-50`` reads them."""
    q = config.get("quantization") or config.get("quantization_config")
    if not isinstance(q, dict):
        return None, None, "affine"
    return int(q["group_size"]), int(q["bits"]), str(q.get("mode", "affine"))


def config_from_dict(config: dict) -> LlamaConfig:
    """``LlamaConfig`` of an MLX/HF Llama ``config.json``; only 4-bit group-64
    affine checkpoints run on this path."""
    group, bits, mode = quantization_parameters(config)
    if group is None:
        raise ValueError("checkpoint is not quantized: the HIP path runs 4-bit affine linears")
    if bits != 4:
        raise ValueError(f"only 4-bit quantization is supported (got bits={bits})")
    if group != 64:
        raise ValueError(f"only group_size 64 is supported (got {group})")
    if mode != "affine":
        raise ValueError(f"only affine quantization is supported (got mode={mode!r})")
    hs, heads = int(config["hidden_size"]), int(config["num_attention_heads"])
    return LlamaConfig(
        vocab_size=int(config["vocab_size"]),
        hidden_size=hs,
        intermediate_size=int(config["intermediate_size"]),
        num_hidden_layers=int(config["num_hidden_layers"]),
        num_attention_heads=heads,
        num_key_value_heads=int(config.get("num_key_value_heads", heads)),
        rms_norm_eps=float(config.get("rms_norm_eps", 1e-6)),     # llama_mlx.py:462
        rope_theta=float(config.get("rope_theta", 10000.0)),      # llama_mlx.py:699-702
        group_size=group,
    )


def _files(model_dir: Path) -> List[Path]:
    index = model_dir / "model.safetensors.index.json"
    if index.exists():
        names = sorted(set(json.loads(index.read_text())["weight_map"].values()))
        return [model_dir / n for n in names]
    files = sorted(model_dir.glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"no .safetensors files in {model_dir}")
    return files


class _Tensors:
    def __init__(self, readers: Iterable[SafeTensorReader]):
        self.where: Dict[str, SafeTensorReader] = {}
        for r in readers:
            for k in r.keys():
                self.where[k] = r

    def __contains__(self, name: str) -> bool:
        return name in self.where

    def get(self, name: str, dtype: Optional[str] = None, shape=None) -> np.ndarray:
        if name not in self.where:
            raise KeyError(f"Tensor '{name}' not found in the checkpoint")
        r = self.where[name]
        if dtype is not None and r.dtype(name) != dtype:
            raise ValueError(f"'{name}' is {r.dtype(name)}, expected {dtype}")
        a = r.get(name)
        if shape is not None and tuple(a.shape) != tuple(shape):
            raise ValueError(f"'{name}' has shape {list(a.shape)}, expected {list(shape)}")
        return a


def checkpoint_names(cfg: LlamaConfig, *, quantized_embed: bool, head: str) -> List[str]:
    """Tensor names an MLX 4-bit Llama checkpoint holds; ``head`` is "q4",
    "bf16" or "tied"."""
    names = ["model.embed_tokens.weight", "model.norm.weight"]
    if quantized_embed:
        names += ["model.embed_tokens.scales", "model.embed_tokens.biases"]
    if head != "tied":
        names.append("lm_head.weight")
        if head == "q4":
            names += ["lm_head.scales", "lm_head.biases"]
    for i in range(cfg.num_hidden_layers):
        base = f"model.layers.{i}."
        names += [base + "input_layernorm.weight", base + "post_attention_layernorm.weight"]
        for lin in LINEARS:
            p = f"{base}{_PROJ_PREFIX[lin]}.{lin}."
            names += [p + "weight", p + "scales", p + "biases"]
    return names


def load_mlx_llama(model_dir, device: int = 0) -> HipLlamaForCausalLM:
    """Load an MLX 4-bit Llama checkpoint directory (``config.json`` +
    safetensors) into a ``HipLlamaForCausalLM`` on ``cuda:device``."""
    model_dir = Path(model_dir)
    raw = json.loads((model_dir / "config.json").read_text())
    cfg = config_from_dict(raw)
    return build_llama(cfg, _Tensors(SafeTensorReader(p) for p in _files(model_dir)), device)


def build_llama(cfg: LlamaConfig, t, device: int = 0) -> HipLlamaForCausalLM:
    """Device weights from a tensor source ``t`` (``name in t``;
    ``t.get(name, dtype, shape)`` -> ndarray) holding MLX checkpoint names."""
    import torch

    from . import ops

    dev = torch.device("cuda", device)
    hs, fs, g = cfg.hidden_size, cfg.intermediate_size, cfg.group_size
    hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    rows = {"q_proj": (hq * d, hs), "k_proj": (hkv * d, hs), "v_proj": (hkv * d, hs),
            "o_proj": (hs, hq * d), "gate_proj": (fs, hs), "up_proj": (fs, hs),
            "down_proj": (hs, fs)}

    def up(a: np.ndarray) -> "torch.Tensor":
        # read-only (mapped) host arrays are copied to the device at once
        with warnings.catch_warnings():
            warnings.simplefilter("ignore", UserWarning)
            if a.dtype == np.uint16:
                return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(dev)
            if a.dtype == np.uint32:
                return torch.from_numpy(a.view(np.int32)).view(torch.uint32).to(dev)
            return torch.from_numpy(a).to(dev)

    def q4(prefix: str, n: int, k: int) -> Tuple["torch.Tensor", "torch.Tensor", "torch.Tensor"]:
        if prefix + ".scales" not in t:
            raise ValueError(f"'{prefix}' is not quantized: the HIP path runs 4-bit linears")
        return (up(t.get(prefix + ".weight", "U32", (n, k // 8))),
                up(t.get(prefix + ".scales", "BF16", (n, k // g))),
                up(t.get(prefix + ".biases", "BF16", (n, k // g))))

    def bf16(name: str, shape) -> "torch.Tensor":
        return up(t.get(name, "BF16", shape))

    w: Dict[str, "torch.Tensor"] = {}
    embed_q4 = None
    if "model.embed_tokens.scales" in t:
        embed_q4 = q4("model.embed_tokens", cfg.vocab_size, hs)
        w["embed_tokens"] = ops.dequantize(*embed_q4, group_size=g)
    else:
        w["embed_tokens"] = bf16("model.embed_tokens.weight", (cfg.vocab_size, hs))
    for i in range(cfg.num_hidden_layers):
        base = f"model.layers.{i}."
        p = f"layers.{i}."
        for lin in LINEARS:
            n, k = rows[lin]
            trip = q4(f"{base}{_PROJ_PREFIX[lin]}.{lin}", n, k)
            w[p + lin + ".weight"], w[p + lin + ".scales"], w[p + lin + ".biases"] = trip
        w[p + "input_layernorm"] = bf16(base + "input_layernorm.weight", (hs,))
        w[p + "post_attention_layernorm"] = bf16(base + "post_attention_layernorm.weight", (hs,))
    w["norm"] = bf16("model.norm.weight", (hs,))
    if "lm_head.weight" in t:
        if "lm_head.scales" in t:
            trip = q4("lm_head", cfg.vocab_size, hs)
            w["lm_head.weight"], w["lm_head.scales"], w["lm_head.biases"] = trip
        else:
            w["lm_head"] = bf16("lm_head.weight", (cfg.vocab_size, hs))
    elif embed_q4 is not None:  # tied to the quantized embedding: project through the triple
        w["lm_head.weight"], w["lm_head.scales"], w["lm_head.biases"] = embed_q4
    else:
        w["lm_head"] = w["embed_tokens"]
    return HipLlamaForCausalLM(cfg, w, device=device)
