"""Device KV cache with the reference's ``MLXKVCache`` contract.

Mirrors ``src/ollm/mlx_kvcache.py:21-307`` (``update``, ``get_seq_length``,
``get_max_cache_shape``, ``__getitem__``, ``__contains__``, ``__len__``,
``clear``) on top of the library's ``strata_kv`` object: one preallocated
``[layers, B, Hkv, Lmax, D]`` buffer per K and V (allocated by PyTorch so that
the views returned by ``update`` are ordinary tensors), O(Lnew) appends
instead of the reference's whole-cache ``concatenate``, and host-side
per-layer lengths validated by the library ("append exactly").

Disk tier (``mlx_kvcache.py:183-284``): ``save_to_disk`` writes a layer as
``.npz`` with ``key``, ``value`` (``[B, Hkv, len, D]``; a bf16 cache is
widened to float32 exactly, numpy having no bfloat16) and ``seen_tokens``;
the layer is then "offloaded" and is reloaded from its file
(``strata_kv_restore``) before the next read or append.  The device buffer
is preallocated and stays reserved: HBM is the hot tier and the file a
persistent snapshot.  ``clear`` deletes the files the cache wrote.
``HipDiskKVCache`` adds the automatic offload of ``MLXLlamaDiskCache``
(310-367).
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path
from typing import Any, Dict, List, Optional, Tuple

import numpy as np
import torch

from . import _abi
from .ops import _code, _ctx, _dev, _stream


class HipKVCache:
    def __init__(self, config: Any, cache_dir: Optional[str] = None, stats: Optional[Any] = None,
                 *, batch_size: int = 1, max_length: int = 4096,
                 dtype: torch.dtype = torch.bfloat16, device: int = 0):
        layers = int(getattr(config, "num_hidden_layers"))
        hkv = int(getattr(config, "num_key_value_heads", None)
                  or getattr(config, "num_attention_heads"))
        head_dim = int(getattr(config, "head_dim", None)
                       or config.hidden_size // config.num_attention_heads)
        self.config = config
        self.cache_dir = cache_dir
        self.stats = stats
        self._disk_offloaded: Dict[int, str] = {}   # layer -> file
        self._managed_disk_files: set = set()
        if cache_dir is not None:
            os.makedirs(cache_dir, exist_ok=True)
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
        if layer_idx in self._disk_offloaded:
            self._load_layer_from_disk(layer_idx)
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
        if layer_idx in self._disk_offloaded:  # mlx_kvcache.py:88-89
            self._load_layer_from_disk(layer_idx)
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
        if layer_idx in self._disk_offloaded:
            self._load_layer_from_disk(layer_idx)
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
        if layer_idx in self._disk_offloaded:
            self._load_layer_from_disk(layer_idx)
        if self._len(layer_idx) == 0:
            raise KeyError(layer_idx)
        k, v = self.views(layer_idx)
        return {"key": k, "value": v}

    def __contains__(self, layer_idx) -> bool:
        return isinstance(layer_idx, int) and 0 <= layer_idx < self.num_layers \
            and (self._len(layer_idx) > 0 or layer_idx in self._disk_offloaded)

    def __len__(self) -> int:
        return sum(1 for i in range(self.num_layers) if i in self)

    def clear(self) -> None:
        """Empty every layer and delete the files this cache wrote
        (``mlx_kvcache.py:271-284``)."""
        _abi.check(self._lib.strata_kv_clear(self.handle))
        for f in self._managed_disk_files:
            if os.path.exists(f):
                os.remove(f)
        self._disk_offloaded.clear()
        self._managed_disk_files.clear()

    # ------------------------------------------------------------ disk tier
    def in_memory_layers(self) -> List[int]:
        """Layers holding keys that are not offloaded."""
        return [i for i in range(self.num_layers)
                if i not in self._disk_offloaded and self._len(i) > 0]

    def save_to_disk(self, layer_idx: int, filename: Optional[str] = None) -> None:
        """Write a layer to ``.npz`` and mark it offloaded (``mlx_kvcache.py:183-220``)."""
        self._validate_layer(layer_idx)
        if layer_idx in self._disk_offloaded or self._len(layer_idx) == 0:
            return
        if filename is None:
            if self.cache_dir is None:
                raise ValueError("filename is required for a memory-only KV cache")
            filename = os.path.join(self.cache_dir, f"kvcache_layer_{layer_idx}.npz")
        dest = Path(filename)
        dest.parent.mkdir(parents=True, exist_ok=True)
        k, v = self.views(layer_idx)
        np.savez_compressed(dest, key=k.float().cpu().numpy(), value=v.float().cpu().numpy(),
                            seen_tokens=self.get_seq_length(None))
        self._disk_offloaded[layer_idx] = os.fspath(dest)
        self._managed_disk_files.add(os.fspath(dest))

    def _load_layer_from_disk(self, layer_idx: int) -> None:
        """Restore an offloaded layer from its file (``mlx_kvcache.py:222-250``)."""
        filename = self._disk_offloaded[layer_idx]
        with np.load(filename) as data:
            key, value = data["key"], data["value"]
        want = (self.batch, self.hkv, key.shape[2] if key.ndim == 4 else -1, self.head_dim)
        if key.ndim != 4 or key.shape != value.shape or key.shape != want:
            raise ValueError(f"{filename}: key/value {list(key.shape)} do not match the cache "
                             f"geometry [B={self.batch}, Hkv={self.hkv}, L, D={self.head_dim}]")
        L = key.shape[2]
        if L > self.lmax:
            raise ValueError(f"{filename}: {L} positions exceed the cache capacity {self.lmax}")
        kt = torch.from_numpy(np.ascontiguousarray(key, dtype=np.float32)).to(self.device)
        vt = torch.from_numpy(np.ascontiguousarray(value, dtype=np.float32)).to(self.device)
        _abi.check(self._lib.strata_kv_restore(self.handle, layer_idx, kt.data_ptr(),
                                               vt.data_ptr(), _code(kt), L,
                                               _stream(self.device.index or 0)))
        torch.cuda.current_stream(self.device).synchronize()  # kt/vt die with this frame
        del self._disk_offloaded[layer_idx]

    def load_offloaded_layers(self) -> None:
        """Restore every offloaded layer onto the device.

        The native decoder appends into device memory directly; a layer left
        on disk would later be reloaded over those appends (stale K/V, length
        reset to the file's).  Callers that hand the cache to native code
        call this first."""
        for idx in sorted(self._disk_offloaded):
            self._load_layer_from_disk(idx)

    def offload_layers_to_disk(self, layer_indices: Optional[List[int]] = None) -> None:
        """``mlx_kvcache.py:252-264``: all cached layers when ``layer_indices`` is None."""
        for idx in (self.in_memory_layers() if layer_indices is None else layer_indices):
            self.save_to_disk(idx)

    def __del__(self):
        try:
            if getattr(self, "handle", None):
                self._lib.strata_kv_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


class HipDiskKVCache(HipKVCache):
    """``MLXLlamaDiskCache`` (``mlx_kvcache.py:310-367``): after each update,
    layers beyond ``max_layers_in_memory`` (lowest indices first, never the
    layer just updated) are offloaded to ``cache_dir``."""

    def __init__(self, config: Any, cache_dir: str = "./kvcache", stats: Optional[Any] = None,
                 max_layers_in_memory: int = 4, **kwargs):
        if max_layers_in_memory <= 0:
            raise ValueError("max_layers_in_memory must be positive")
        super().__init__(config, cache_dir, stats, **kwargs)
        self.max_layers_in_memory = max_layers_in_memory

    def update(self, key_states, value_states, layer_idx, cache_kwargs=None):
        result = super().update(key_states, value_states, layer_idx, cache_kwargs)
        live = self.in_memory_layers()
        if len(live) > self.max_layers_in_memory:
            for idx in live[:-self.max_layers_in_memory]:
                if idx != layer_idx:
                    self.save_to_disk(idx)
        return result
