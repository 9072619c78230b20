"""Torch-tensor front end of the hot-path kernels (device memory and streams
come from PyTorch-ROCm; all compute runs in libstrata_hip.so).

Each function mirrors the reference operation it replaces:

* ``linear``            -> ``_linear`` (``src/ollm/llama_mlx.py:53-74``)
* ``linear_multi``      -> several ``_linear`` calls sharing x (257-268, 395-407)
* ``rope``              -> ``MLXRotaryEmbedding`` + ``apply_rotary_pos_emb_mlx``
                           (``llama_mlx.py:95-182``)
* ``attention``         -> ``online_chunked_grouped_attention_mx``
                           (``src/ollm/backends/mlx_ops.py:32-152``)
* ``attention_no_mask`` -> ``online_chunked_grouped_attention_rope_no_mask_mx``
                           (``mlx_ops.py:155-178``)
"""
from __future__ import annotations

import ctypes as C
from typing import Optional, Sequence, Tuple

import torch

from . import _abi
from ._abi import BF16, F32, check

_DT = {torch.float32: F32, torch.bfloat16: BF16}


def _code(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected float32 or bfloat16") from None


def _dev(t: torch.Tensor) -> int:
    if t.device.type != "cuda":
        raise ValueError("tensors must live on the HIP device (torch 'cuda' device)")
    return t.device.index or 0


def _stream(device: int) -> C.c_void_p:
    return C.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _ctx(device: int):
    return _abi.context(device).handle


def _lib():
    return _abi.load()


# ----------------------------------------------------------------- linear
def linear(x: torch.Tensor, weight: torch.Tensor, scales: Optional[torch.Tensor],
           biases: Optional[torch.Tensor], *, group_size: Optional[int] = 64,
           bits: Optional[int] = 4, mode: str = "affine",
           out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """``y = x @ W.T`` with W q4-affine (scales given) or bf16 (scales None)."""
    dev = _dev(x)
    if mode != "affine":
        raise ValueError(f"unsupported quantization mode {mode!r}")
    lead = x.shape[:-1]
    K = x.shape[-1]
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    out_dtype = out_dtype or x.dtype
    if scales is None:
        N = weight.shape[0]
        if weight.dtype != torch.bfloat16 or weight.shape[1] != K:
            raise ValueError("dense weight must be bf16 [N, K]")
        y = torch.empty((M, N), dtype=out_dtype, device=x.device)
        check(_lib().strata_linear_bf16(_ctx(dev), x2.data_ptr(), _code(x2), M, K,
                                        weight.contiguous().data_ptr(), N, y.data_ptr(),
                                        _code(y), _stream(dev)))
        return y.reshape(*lead, N)
    N = weight.shape[0]
    _check_q4(weight, scales, biases, N, K, group_size, bits)
    y = torch.empty((M, N), dtype=out_dtype, device=x.device)
    check(_lib().strata_linear_q4(_ctx(dev), x2.data_ptr(), _code(x2), M, K, weight.data_ptr(),
                                  scales.data_ptr(), biases.data_ptr(), N, int(group_size),
                                  int(bits), y.data_ptr(), _code(y), _stream(dev)))
    return y.reshape(*lead, N)


def _check_q4(w, s, b, N, K, group_size, bits):
    if bits != 4:
        raise ValueError(f"only 4-bit quantization is supported (got bits={bits})")
    if group_size is None or K % group_size:
        raise ValueError(f"K={K} must be divisible by group_size={group_size}")
    if w.dtype not in (torch.uint32, torch.int32) or tuple(w.shape) != (N, K // 8):
        raise ValueError(f"packed weight must be uint32 [N, K/8] = [{N}, {K // 8}], "
                         f"got {w.dtype} {tuple(w.shape)}")
    for name, t in (("scales", s), ("biases", b)):
        if t is None or t.dtype != torch.bfloat16 or tuple(t.shape) != (N, K // group_size):
            raise ValueError(f"{name} must be bf16 [N, K/group_size]")
    if not (w.is_contiguous() and s.is_contiguous() and b.is_contiguous()):
        raise ValueError("quantized weight tensors must be contiguous")


def linear_multi(x: torch.Tensor, weights: Sequence[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]],
                 *, group_size: int = 64, bits: int = 4,
                 outs: Optional[Sequence[torch.Tensor]] = None,
                 out_dtype: Optional[torch.dtype] = None):
    """Several q4 linears sharing ``x`` in one launch; returns the outputs."""
    dev = _dev(x)
    K = x.shape[-1]
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    out_dtype = out_dtype or x.dtype
    arr = (_abi.Q4Weight * len(weights))()
    ys = []
    for i, (w, s, b) in enumerate(weights):
        N = w.shape[0]
        _check_q4(w, s, b, N, K, group_size, bits)
        y = outs[i] if outs is not None else torch.empty((M, N), dtype=out_dtype, device=x.device)
        ys.append(y)
        arr[i] = _abi.Q4Weight(w.data_ptr(), s.data_ptr(), b.data_ptr(), N, y.data_ptr())
    check(_lib().strata_linear_q4_multi(_ctx(dev), x2.data_ptr(), _code(x2), M, K, arr,
                                        len(weights), group_size, bits, _code(ys[0]),
                                        _stream(dev)))
    return [y.reshape(*lead, y.shape[-1]) for y in ys]


class Q4Layout:
    """Linears sharing ``x`` copied once into the decode GEMV's load-time
    layout (``strata_q4_layout_create``; the reference's load step is
    ``_load_layer_weights``, ``src/ollm/llama_mlx.py:550-580``).  Calling it
    runs ``_linear`` on each of them (``llama_mlx.py:53-74``) for 1..8 bf16
    rows of ``x`` on the matrix-core GEMV."""

    def __init__(self, weights: Sequence[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]],
                 *, group_size: int = 64, bits: int = 4):
        if not weights:
            raise ValueError("at least one weight is required")
        K = weights[0][0].shape[1] * 8
        self.device = _dev(weights[0][0])
        self.K = K
        self.N = []
        arr = (_abi.Q4Weight * len(weights))()
        for i, (w, s, b) in enumerate(weights):
            N = w.shape[0]
            _check_q4(w, s, b, N, K, group_size, bits)
            self.N.append(N)
            arr[i] = _abi.Q4Weight(w.data_ptr(), s.data_ptr(), b.data_ptr(), N, None)
        torch.cuda.synchronize(self.device)
        h = C.c_void_p()
        check(_lib().strata_q4_layout_create(_ctx(self.device), arr, len(weights), K, C.byref(h)))
        self._h = h

    def __call__(self, x: torch.Tensor, *, outs: Optional[Sequence[torch.Tensor]] = None,
                 out_dtype: Optional[torch.dtype] = None):
        if self._h is None:
            raise ValueError("layout is closed")
        if x.dtype != torch.bfloat16 or x.shape[-1] != self.K:
            raise ValueError(f"x must be bf16 [..., {self.K}]")
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.K).contiguous()
        M = x2.shape[0]
        out_dtype = out_dtype or torch.bfloat16
        ys = list(outs) if outs is not None else [
            torch.empty((M, n), dtype=out_dtype, device=x.device) for n in self.N]
        ptrs = (C.c_void_p * len(ys))(*[y.data_ptr() for y in ys])
        check(_lib().strata_linear_q4_layout(_ctx(self.device), x2.data_ptr(), BF16, M, self._h,
                                             ptrs, _code(ys[0]), _stream(self.device)))
        return [y.reshape(*lead, y.shape[-1]) for y in ys]

    def close(self):
        if getattr(self, "_h", None) is not None:
            torch.cuda.synchronize(self.device)
            _lib().strata_q4_layout_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def quantize(weight: torch.Tensor, group_size: int = 64):
    """Quantize a float32/bf16 ``[N, K]`` device tensor to (u32 packed, bf16 scales, bf16 biases)."""
    dev = _dev(weight)
    w = weight.contiguous()
    N, K = w.shape
    if K % group_size:
        raise ValueError("K must be divisible by group_size")
    packed = torch.empty((N, K // 8), dtype=torch.uint32, device=w.device)
    sc = torch.empty((N, K // group_size), dtype=torch.bfloat16, device=w.device)
    bi = torch.empty_like(sc)
    check(_lib().strata_quantize_q4(_ctx(dev), w.data_ptr(), _code(w), N, K, group_size,
                                    packed.data_ptr(), sc.data_ptr(), bi.data_ptr(), _stream(dev)))
    return packed, sc, bi


def dequantize(weight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               group_size: int = 64, bits: int = 4) -> torch.Tensor:
    """bf16 ``[N, K]`` = s*q + b of a q4 triple (``mx.dequantize``,
    ``src/ollm/llama_mlx.py:722-738``), fp32 math with one RNE rounding."""
    dev = _dev(weight)
    N, K = weight.shape[0], weight.shape[1] * 8
    _check_q4(weight, scales, biases, N, K, group_size, bits)
    out = torch.empty((N, K), dtype=torch.bfloat16, device=weight.device)
    check(_lib().strata_dequantize_q4(_ctx(dev), weight.data_ptr(), scales.data_ptr(),
                                      biases.data_ptr(), N, K, group_size, bits, out.data_ptr(),
                                      _stream(dev)))
    return out


# -------------------------------------------------------------------- RoPE
def rope(q: Optional[torch.Tensor], k: Optional[torch.Tensor], position_ids: torch.Tensor,
         theta: float) -> None:
    """In-place rotate-half RoPE on ``q [B,Hq,L,D]`` and ``k [B,Hkv,L,D]``."""
    ref = q if q is not None else k
    dev = _dev(ref)
    B, _, L, D = ref.shape
    pos = position_ids.to(device=ref.device, dtype=torch.int32)
    if pos.ndim == 1:
        pos = pos[None, :]
    pos = pos.expand(B, L).contiguous()
    for t in (q, k):
        if t is not None and (not t.is_contiguous() or t.dtype != ref.dtype):
            raise ValueError("q and k must be contiguous and share a dtype")
    check(_lib().strata_rope(_ctx(dev), _ptr(q), _ptr(k), pos.data_ptr(), B,
                             q.shape[1] if q is not None else 0,
                             k.shape[1] if k is not None else 0, L, D, float(theta),
                             _code(ref), _stream(dev)))


# --------------------------------------------------------------- attention
def _normalize_query_positions(query_positions, batch: int, lq: int, device) -> torch.Tensor:
    """``_normalize_query_positions`` (mlx_ops.py:17-29)."""
    pos = torch.as_tensor(query_positions, dtype=torch.int32, device=device)
    if pos.ndim == 1:
        pos = pos[None, :]
    if tuple(pos.shape) == (1, lq) and batch > 1:
        pos = pos.expand(batch, lq)
    if tuple(pos.shape) != (batch, lq):
        raise ValueError("query_positions must have shape [query_length] or "
                         f"[batch, query_length], got {tuple(pos.shape)}")
    return pos.contiguous()


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
              query_positions=None, causal: bool = True, q_block_size: int = 32768,
              k_block_size: int = 1024, eps: float = 1e-12, *,
              kv_strides: Optional[Tuple[int, int]] = None,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Chunked causal GQA attention; ``[B,Hq,Lq,D]`` in ``q.dtype``.

    ``kv_strides`` = (batch_stride, head_stride) in elements lets k/v be views
    into a larger KV-cache buffer whose time axis is longer than ``Lk``.
    """
    if q_block_size <= 0 or k_block_size <= 0:
        raise ValueError("attention block sizes must be positive")
    B, Hq, Lq, D = q.shape
    _, Hkv, Lk, Dk = k.shape
    if D != Dk:
        raise ValueError("q and k must share last-dim size")
    if k.shape[0] != B or v.shape[0] != B:
        raise ValueError("q, k, and v must share batch size")
    if v.shape[1] != Hkv or v.shape[2] != Lk:
        raise ValueError("k and v must share head and sequence dimensions")
    if v.shape[3] != D:
        raise ValueError("q, k, and v must share last-dim size")
    if Hkv <= 0 or Hq % Hkv != 0:
        raise ValueError("query heads must be divisible by key/value heads")
    if causal and Lk < Lq:
        raise ValueError("causal attention requires key length >= query length")
    dev = _dev(q)
    qpos = None
    if causal and query_positions is not None:
        qpos = _normalize_query_positions(query_positions, B, Lq, q.device)
    q = q.contiguous()
    if kv_strides is None:
        k = k.contiguous()
        v = v.contiguous()
        bs, hs = Hkv * Lk * D, Lk * D
    else:
        bs, hs = kv_strides
        if k.stride() != v.stride() or k.stride()[2:] != (D, 1) or (k.stride(0), k.stride(1)) != (bs, hs):
            raise ValueError("k/v views do not match the given kv_strides")
    if out is None:
        out = torch.empty((B, Hq, Lq, D), dtype=q.dtype, device=q.device)
    check(_lib().strata_attn_gqa(_ctx(dev), q.data_ptr(), _code(q), k.data_ptr(), _code(k),
                                 v.data_ptr(), _code(v), bs, hs, _ptr(qpos), B, Hq, Hkv, Lq, Lk,
                                 D, 1 if causal else 0, int(min(q_block_size, 2**31 - 1)),
                                 int(min(k_block_size, 2**31 - 1)), float(eps), out.data_ptr(),
                                 _stream(dev)))
    return out


def attention_no_mask(q, k, v, position_ids=None, q_block_size: int = 32768,
                      k_block_size: int = 1024, eps: float = 1e-12) -> torch.Tensor:
    """Unmasked compatibility entry point; ``position_ids`` is ignored."""
    del position_ids
    return attention(q, k, v, causal=False, q_block_size=q_block_size,
                     k_block_size=k_block_size, eps=eps)


# -------------------------------------------------------------------- glue
def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float,
            residual: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None):
    """bf16 RMSNorm; with ``residual`` the sum ``x + residual`` is first written into x."""
    dev = _dev(x)
    H = x.shape[-1]
    rows = x.numel() // H
    if out is None:
        out = torch.empty_like(x)
    check(_lib().strata_rmsnorm(_ctx(dev), x.data_ptr(), _ptr(residual), weight.data_ptr(), rows,
                                H, float(eps), out.data_ptr(), _stream(dev)))
    return out


def silu_mul(g: torch.Tensor, u: torch.Tensor, out: Optional[torch.Tensor] = None):
    dev = _dev(g)
    if out is None:
        out = torch.empty_like(g)
    check(_lib().strata_silu_mul(_ctx(dev), g.data_ptr(), u.data_ptr(), g.numel(), out.data_ptr(),
                                 _stream(dev)))
    return out


def add(x: torch.Tensor, r: torch.Tensor, out: Optional[torch.Tensor] = None):
    dev = _dev(x)
    if out is None:
        out = torch.empty_like(x)
    check(_lib().strata_add(_ctx(dev), x.data_ptr(), r.data_ptr(), x.numel(), out.data_ptr(),
                            _stream(dev)))
    return out


def embed(table: torch.Tensor, ids: torch.Tensor, out: Optional[torch.Tensor] = None):
    dev = _dev(table)
    V, H = table.shape
    ids32 = ids.to(device=table.device, dtype=torch.int32).contiguous()
    if out is None:
        out = torch.empty((*ids.shape, H), dtype=table.dtype, device=table.device)
    check(_lib().strata_embed(_ctx(dev), table.data_ptr(), V, H, ids32.data_ptr(), ids32.numel(),
                              out.data_ptr(), _stream(dev)))
    return out


def argmax(logits: torch.Tensor, out: Optional[torch.Tensor] = None):
    dev = _dev(logits)
    V = logits.shape[-1]
    lg = logits.reshape(-1, V)
    if lg.dtype != torch.float32 or not lg.is_contiguous():
        raise ValueError("argmax expects contiguous float32 logits")
    if out is None:
        out = torch.empty(lg.shape[0], dtype=torch.int32, device=logits.device)
    check(_lib().strata_argmax(_ctx(dev), lg.data_ptr(), lg.shape[0], V, out.data_ptr(),
                               _stream(dev)))
    return out
