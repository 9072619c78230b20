"""Device KV cache with the reference's ``MLXKVCache`` contract.

Mirrors ``src/ollm/mlx_kvcache.py:21-307`` (``update``, ``get_seq_length``,
``get_max_cache_shape``, ``__getitem__``, ``__contains__``, ``__len__``,
``clear``) on top of the library's ``strata_kv`` object: one preallocated
``[layers, B, Hkv, Lmax, D]`` buffer per K and V (allocated by PyTorch so that
the views returned by ``update`` are ordinary tensors), O(Lnew) appends
instead of the reference's whole-cache ``concatenate``, and host-side
per-layer lengths validated by the library ("append exactly").
"""
from __future__ import annotations

import ctypes as C
from typing import Any, Dict, Optional, Tuple

import torch

from . import _abi
from .ops import _code, _ctx, _dev, _stream


class HipKVCache:
    def __init__(self, config: Any, *, batch_size: int = 1, max_length: int = 4096,
                 dtype: torch.dtype = torch.bfloat16, device: int = 0):
        layers = int(getattr(config, "num_hidden_layers"))
        hkv = int(getattr(config, "num_key_value_heads", None)
                  or getattr(config, "num_attention_heads"))
        head_dim = int(getattr(config, "head_dim", None)
                       or config.hidden_size // config.num_attention_heads)
        self.config = config
        self.num_layers, self.batch, self.hkv, self.lmax, self.head_dim = (
            layers, batch_size, hkv, max_length, head_dim)
        self.dtype = dtype
        self.device = torch.device("cuda", device)
        shape = (layers, batch_size, hkv, max_length, head_dim)
        self.k_storage = torch.empty(shape, dtype=dtype, device=self.device)
        self.v_storage = torch.empty(shape, dtype=dtype, device=self.device)
        self._lib = _abi.load()
        h = C.c_void_p()
        _abi.check(self._lib.strata_kv_create(_ctx(device), layers, batch_size, hkv, max_length,
                                              head_dim, _code(self.k_storage),
                                              self.k_storage.data_ptr(),
                                              self.v_storage.data_ptr(), C.byref(h)))
        self.handle = h

    # ---------------------------------------------------------------- helpers
    def _len(self, layer: int) -> int:
        n = C.c_int()
        _abi.check(self._lib.strata_kv_len(self.handle, layer, C.byref(n)))
        return n.value

    def _validate_layer(self, layer_idx) -> None:
        if not isinstance(layer_idx, int) or layer_idx < 0:
            raise ValueError("layer_idx must be a non-negative integer")
        if layer_idx >= self.num_layers:
            raise ValueError(
                f"layer_idx {layer_idx} is outside configured layer count {self.num_layers}")

    def views(self, layer_idx: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """``[B, Hkv, len, D]`` views of the layer's cached keys and values."""
        n = self._len(layer_idx)
        return self.k_storage[layer_idx, :, :, :n], self.v_storage[layer_idx, :, :, :n]

    @property
    def kv_strides(self) -> Tuple[int, int]:
        return self.hkv * self.lmax * self.head_dim, self.lmax * self.head_dim

    # ------------------------------------------------------ reference contract
    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               cache_kwargs: Optional[Dict[str, Any]] = None):
        """Append ``[B, Hkv, Lnew, D]`` states; return the full cached K, V views."""
        self._validate_layer(layer_idx)
        if key_states.ndim != 4 or value_states.ndim != 4:
            raise ValueError("key and value states must have rank 4")
        if key_states.shape != value_states.shape:
            raise ValueError("key and value states must have identical shapes")
        b, h, lnew, d = key_states.shape
        if (b, h, d) != (self.batch, self.hkv, self.head_dim):
            raise ValueError("new key states must match cached batch, head, and feature dimensions")
        prev = self._len(layer_idx)
        if cache_kwargs and cache_kwargs.get("cache_position") is not None:
            pos = torch.as_tensor(cache_kwargs["cache_position"]).reshape(-1).cpu()
            expected = torch.arange(prev, prev + lnew)
            if pos.shape != expected.shape or not torch.equal(pos.to(expected.dtype), expected):
                raise ValueError(
                    "cache_position must append exactly after the cached sequence; "
                    f"expected {expected.tolist()}, got {pos.tolist()}")
        dev = _dev(key_states)
        ks = key_states.contiguous()
        vs = value_states.to(ks.dtype).contiguous()
        _abi.check(self._lib.strata_kv_append(self.handle, layer_idx, ks.data_ptr(), vs.data_ptr(),
                                              _code(ks), lnew, prev, _stream(dev)))
        return self.views(layer_idx)

    def rope_append(self, layer_idx: int, q_src: torch.Tensor, k_src: torch.Tensor,
                    v_src: torch.Tensor, num_heads: int, seq_len: int, theta: float,
                    q_out: torch.Tensor) -> None:
        """Fused RoPE + append from token-major projection outputs (decoder fast path)."""
        prev = self._len(layer_idx)
        _abi.check(self._lib.strata_rope_kv_append(
            self.handle, layer_idx, q_src.data_ptr(), k_src.data_ptr(), v_src.data_ptr(),
            _code(q_src), num_heads, seq_len, prev, float(theta), q_out.data_ptr(),
            _stream(_dev(q_src))))

    def get_seq_length(self, layer_idx: Optional[int] = 0) -> int:
        if layer_idx is None:
            return self._len(-1)
        if not isinstance(layer_idx, int) or layer_idx < 0 or layer_idx >= self.num_layers:
            return 0
        return self._len(layer_idx)

    def get_max_cache_shape(self) -> Optional[int]:
        return self.lmax

    def __getitem__(self, layer_idx: int):
        self._validate_layer(layer_idx)
        if self._len(layer_idx) == 0:
            raise KeyError(layer_idx)
        k, v = self.views(layer_idx)
        return {"key": k, "value": v}

    def __contains__(self, layer_idx) -> bool:
        return isinstance(layer_idx, int) and 0 <= layer_idx < self.num_layers \
            and self._len(layer_idx) > 0

    def __len__(self) -> int:
        return sum(1 for i in range(self.num_layers) if self._len(i) > 0)

    def clear(self) -> None:
        _abi.check(self._lib.strata_kv_clear(self.handle))

    def __del__(self):
        try:
            if getattr(self, "handle", None):
                self._lib.strata_kv_destroy(self.handle)
                self.handle = None
        except Exception:
            pass
