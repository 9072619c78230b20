"""KV-cache append/read oracle (test infrastructure).

Restates ``MLXKVCache.update`` (``src/ollm/mlx_kvcache.py:65-125``),
``_validate_layer_index`` (127-135), ``_validate_state_shapes`` (137-141),
``_validate_cache_position`` (143-158) and ``get_seq_length`` (160-172): per
layer, K/V ``[B, Hkv, L, D]`` grow by concatenation along axis 2, the layer
length is ``K.shape[2]``, and ``cache_position`` must equal
``arange(prev, prev + new)`` or ``ValueError("... append exactly ...")``.
"""
from __future__ import annotations

from typing import Any, Dict, Optional

import numpy as np


class OracleKVCache:
    def __init__(self, num_layers: Optional[int] = None):
        self.num_layers = num_layers
        self._cache: Dict[int, Dict[str, np.ndarray]] = {}
        self._lengths: Dict[int, int] = {}
        self._seen_tokens = 0

    def update(self, key_states, value_states, layer_idx: int,
               cache_kwargs: Optional[Dict[str, Any]] = None):
        if not isinstance(layer_idx, int) or layer_idx < 0:
            raise ValueError("layer_idx must be a non-negative integer")
        if self.num_layers is not None and layer_idx >= self.num_layers:
            raise ValueError(
                f"layer_idx {layer_idx} is outside configured layer count {self.num_layers}")
        k = np.asarray(key_states)
        v = np.asarray(value_states)
        if k.ndim != 4 or v.ndim != 4:
            raise ValueError("key and value states must have rank 4")
        if k.shape != v.shape:
            raise ValueError("key and value states must have identical shapes")
        prev = self._lengths.get(layer_idx, 0)
        if cache_kwargs and cache_kwargs.get("cache_position") is not None:
            pos = np.asarray(cache_kwargs["cache_position"]).reshape(-1)
            expected = np.arange(prev, prev + k.shape[2])
            if pos.shape != expected.shape or not np.array_equal(pos, expected):
                raise ValueError(
                    "cache_position must append exactly after the cached sequence; "
                    f"expected {expected.tolist()}, got {pos.tolist()}")
        if layer_idx in self._cache:
            ck = self._cache[layer_idx]["key"]
            if ck.shape[:2] + ck.shape[3:] != k.shape[:2] + k.shape[3:]:
                raise ValueError(
                    "new key states must match cached batch, head, and feature dimensions")
            self._cache[layer_idx]["key"] = np.concatenate([ck, k], axis=2)
            self._cache[layer_idx]["value"] = np.concatenate(
                [self._cache[layer_idx]["value"], v], axis=2)
        else:
            self._cache[layer_idx] = {"key": k.copy(), "value": v.copy()}
        self._lengths[layer_idx] = self._cache[layer_idx]["key"].shape[2]
        self._seen_tokens = max(self._lengths.values(), default=0)
        return self._cache[layer_idx]["key"], self._cache[layer_idx]["value"]

    def get_seq_length(self, layer_idx: Optional[int] = 0) -> int:
        if layer_idx is None:
            return max(self._lengths.values(), default=0)
        return self._lengths.get(layer_idx, 0)
