"""Chunked causal grouped-query attention oracle (test infrastructure).

``chunked_gqa`` restates ``online_chunked_grouped_attention_mx``
(``src/ollm/backends/mlx_ops.py:32-152``) step by step in float32 NumPy:
shape/GQA validation (51-67), bottom-right default positions (69-72), the
KV-head / q-block / k-block loops (81-101), masked block max with fully
masked rows treated as 0 (106-118), masked exp/sum/PV (119-123), the guarded
online merge (125-145) and ``wv / max(s, eps)`` cast to ``q.dtype``
(146-152).  ``_normalize_query_positions`` follows 17-29.

``naive_gqa`` is the dense softmax reference of
``tests/test_mlx_attention.py:17-40``, computed in float64.
"""
from __future__ import annotations

from typing import Optional

import numpy as np


def normalize_query_positions(query_positions, batch: int, lq: int) -> np.ndarray:
    pos = np.asarray(query_positions, dtype=np.int32)
    if pos.ndim == 1:
        pos = pos[None, :]
    if pos.shape == (1, lq) and batch > 1:
        pos = np.broadcast_to(pos, (batch, lq))
    if pos.shape != (batch, lq):
        raise ValueError(
            "query_positions must have shape [query_length] or "
            f"[batch, query_length], got {pos.shape}")
    return pos


def validate(q_shape, k_shape, v_shape, causal: bool, q_block: int = 1, k_block: int = 1):
    if q_block <= 0 or k_block <= 0:
        raise ValueError("attention block sizes must be positive")
    b, hq, lq, d = q_shape
    _, hkv, lk, dk = k_shape
    if d != dk:
        raise ValueError("q and k must share last-dim size")
    if k_shape[0] != b or v_shape[0] != b:
        raise ValueError("q, k, and v must share batch size")
    if v_shape[1] != hkv or v_shape[2] != lk:
        raise ValueError("k and v must share head and sequence dimensions")
    if v_shape[3] != d:
        raise ValueError("q, k, and v must share last-dim size")
    if hkv <= 0 or hq % hkv != 0:
        raise ValueError("query heads must be divisible by key/value heads")
    if causal and lk < lq:
        raise ValueError("causal attention requires key length >= query length")


def chunked_gqa(q, k, v, query_positions: Optional[np.ndarray] = None,
                causal: bool = True, q_block_size: int = 32768,
                k_block_size: int = 1024, eps: float = 1e-12) -> np.ndarray:
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    v = np.asarray(v, dtype=np.float32)
    validate(q.shape, k.shape, v.shape, causal, q_block_size, k_block_size)
    b, hq, lq, d = q.shape
    hkv, lk = k.shape[1], k.shape[2]
    if causal:
        if query_positions is None:
            query_positions = np.arange(lk - lq, lk, dtype=np.int32)
        query_positions = normalize_query_positions(query_positions, b, lq)
    group = hq // hkv
    scale = np.float32(1.0 / np.sqrt(d))
    out = np.zeros((b, hq, lq, d), dtype=np.float32)
    for h in range(hkv):
        kh, vh = k[:, h], v[:, h]
        qs = q[:, h * group:(h + 1) * group]
        for q0 in range(0, lq, q_block_size):
            q1 = min(lq, q0 + q_block_size)
            qb = qs[:, :, q0:q1]
            nq = q1 - q0
            m = np.full((b, group, nq), -np.inf, dtype=np.float32)
            s = np.zeros((b, group, nq), dtype=np.float32)
            wv = np.zeros((b, group, nq, d), dtype=np.float32)
            for k0 in range(0, lk, k_block_size):
                k1 = min(lk, k0 + k_block_size)
                scores = np.einsum("bhqd,bkd->bhqk", qb, kh[:, k0:k1]).astype(np.float32) * scale
                if causal:
                    kp = np.arange(k0, k1, dtype=np.int32)
                    allowed = kp[None, None, None, :] <= query_positions[:, None, q0:q1, None]
                    scores = np.where(allowed, scores, -np.inf).astype(np.float32)
                    local_valid = allowed.any(axis=-1)
                else:
                    allowed = None
                    local_valid = np.ones((b, 1, nq), dtype=bool)
                with np.errstate(invalid="ignore"):
                    raw_max = scores.max(axis=-1)
                local_max = np.where(local_valid, raw_max, 0.0).astype(np.float32)
                with np.errstate(invalid="ignore", over="ignore"):
                    e = np.exp(scores - local_max[..., None]).astype(np.float32)
                if allowed is not None:
                    e = np.where(allowed, e, 0.0).astype(np.float32)
                sum_e = e.sum(axis=-1, dtype=np.float32)
                wv_chunk = np.einsum("bhqk,bkd->bhqd", e, vh[:, k0:k1]).astype(np.float32)
                prev_valid = s > 0
                lv = np.broadcast_to(local_valid, s.shape)
                both = prev_valid & lv
                new_m = np.where(both, np.maximum(m, local_max),
                                 np.where(prev_valid, m, local_max)).astype(np.float32)
                with np.errstate(invalid="ignore", over="ignore"):
                    alpha = np.where(prev_valid, np.exp(m - new_m), 0.0).astype(np.float32)
                    beta = np.where(lv, np.exp(local_max - new_m), 0.0).astype(np.float32)
                s = (alpha * s + beta * sum_e).astype(np.float32)
                wv = (alpha[..., None] * wv + beta[..., None] * wv_chunk).astype(np.float32)
                m = new_m
            out[:, h * group:(h + 1) * group, q0:q1] = wv / np.maximum(s[..., None], eps)
    return out


def naive_gqa(q, k, v, query_positions: Optional[np.ndarray] = None) -> np.ndarray:
    """Dense softmax GQA in float64 (``tests/test_mlx_attention.py:17-40``)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    _, hq, _, d = q.shape
    group = hq // k.shape[1]
    out = np.zeros_like(q)
    scale = 1.0 / np.sqrt(d)
    for h in range(hq):
        kv = h // group
        sc = np.einsum("bqd,bkd->bqk", q[:, h], k[:, kv]) * scale
        if query_positions is not None:
            kp = np.arange(k.shape[2])
            allowed = kp[None, None, :] <= np.asarray(query_positions)[:, :, None]
            sc = np.where(allowed, sc, -np.inf)
        sc -= sc.max(axis=-1, keepdims=True)
        w = np.exp(sc)
        w /= w.sum(axis=-1, keepdims=True)
        out[:, h] = np.einsum("bqk,bkd->bqd", w, v[:, kv])
    return out
