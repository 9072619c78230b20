"""Chunked causal GQA attention (decode split-K, prefill MFMA, generic) vs the oracle."""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention as att
from oracle import rope
from oracle.bf16 import round_bf16
from tests.gpu_util import bf16_dev, rel_err, to_np_f32

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parent.parent
TOL_F32 = 1e-3
TOL_BF16 = 2e-2


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


# ---- the reference's own cases (tests/test_mlx_attention.py:53-137), generic kernel (D=6/4)
def test_reference_cases(dev):
    from lokahi_amd import ops
    rng = np.random.default_rng(0)
    q = rng.standard_normal((1, 4, 7, 6), dtype=np.float32)
    k = rng.standard_normal((1, 2, 9, 6), dtype=np.float32)
    v = rng.standard_normal((1, 2, 9, 6), dtype=np.float32)
    out = ops.attention_no_mask(_t(q, dev), _t(k, dev), _t(v, dev), q_block_size=3, k_block_size=4)
    assert np.allclose(att.naive_gqa(q, k, v), out.cpu().numpy(), atol=1e-5, rtol=1e-5)
    q = rng.standard_normal((2, 4, 7, 6), dtype=np.float32)
    k = rng.standard_normal((2, 2, 7, 6), dtype=np.float32)
    v = rng.standard_normal((2, 2, 7, 6), dtype=np.float32)
    pos = np.broadcast_to(np.arange(7), (2, 7))
    out = ops.attention(_t(q, dev), _t(k, dev), _t(v, dev), query_positions=_t(pos, dev),
                        q_block_size=3, k_block_size=2)
    assert np.allclose(att.naive_gqa(q, k, v, pos), out.cpu().numpy(), atol=1e-5, rtol=1e-5)
    q = rng.standard_normal((1, 4, 1, 6), dtype=np.float32)
    k = rng.standard_normal((1, 2, 6, 6), dtype=np.float32)
    v = rng.standard_normal((1, 2, 6, 6), dtype=np.float32)
    out = ops.attention(_t(q, dev), _t(k, dev), _t(v, dev), query_positions=[[5]])
    assert np.allclose(att.naive_gqa(q, k, v, np.array([[5]])), out.cpu().numpy(), atol=1e-5)
    q = rng.standard_normal((1, 2, 5, 4), dtype=np.float32)
    k = rng.standard_normal((1, 1, 5, 4), dtype=np.float32)
    v = rng.standard_normal((1, 1, 5, 4), dtype=np.float32)
    v2 = v.copy()
    v2[:, :, 3:] += 1000.0
    a = ops.attention(_t(q, dev), _t(k, dev), _t(v, dev), k_block_size=2).cpu().numpy()
    b = ops.attention(_t(q, dev), _t(k, dev), _t(v2, dev), k_block_size=2).cpu().numpy()
    assert np.allclose(a[:, :, :3], b[:, :, :3]) and not np.allclose(a[:, :, 3:], b[:, :, 3:])
    with pytest.raises(ValueError, match="divisible"):
        ops.attention(torch.ones((1, 3, 2, 4), device=dev), torch.ones((1, 2, 2, 4), device=dev),
                      torch.ones((1, 2, 2, 4), device=dev))
    with pytest.raises(ValueError, match="key length >= query length"):
        ops.attention(torch.ones((1, 2, 3, 4), device=dev), torch.ones((1, 2, 2, 4), device=dev),
                      torch.ones((1, 2, 2, 4), device=dev))


def test_config1_chunked_gqa_rope_fp32_prefill_then_decode(dev):
    """B1, Hq8/Hkv2, D64, L512, chunks 128, theta 1e4, fp32."""
    from lokahi_amd import ops
    rng = np.random.default_rng(2024)
    B, Hq, Hkv, D, L = 1, 8, 2, 64, 512
    q = rng.normal(size=(B, Hq, L + 1, D)).astype(np.float32)
    k = rng.normal(size=(B, Hkv, L + 1, D)).astype(np.float32)
    v = rng.normal(size=(B, Hkv, L + 1, D)).astype(np.float32)
    pos = np.arange(L + 1)[None]
    c, s = rope.cos_sin(pos, D, 10000.0)
    qr, kr = rope.apply(q, c, s), rope.apply(k, c, s)
    tq, tk = _t(q, dev), _t(k, dev)
    ops.rope(tq, tk, _t(pos, dev), 10000.0)
    assert np.array_equal(tq.cpu().numpy(), qr) and np.array_equal(tk.cpu().numpy(), kr)
    tv = _t(v, dev)
    pre = ops.attention(tq[:, :, :L].contiguous(), tk[:, :, :L].contiguous(), tv[:, :, :L].contiguous(),
                        query_positions=_t(pos[:, :L], dev), q_block_size=128, k_block_size=128)
    ref = att.chunked_gqa(qr[:, :, :L], kr[:, :, :L], v[:, :, :L], pos[:, :L], True, 128, 128)
    assert rel_err(pre.cpu().numpy(), ref) < TOL_F32
    np.testing.assert_allclose(ref, att.naive_gqa(qr[:, :, :L], kr[:, :, :L], v[:, :, :L], pos[:, :L]),
                               atol=1e-4)
    dec = ops.attention(tq[:, :, L:].contiguous(), tk, tv, query_positions=[[L]])
    ref_d = att.chunked_gqa(qr[:, :, L:], kr, v, np.array([[L]]), True, 128, 128)
    assert rel_err(dec.cpu().numpy(), ref_d) < TOL_F32


def _c_decode(q, k, v):
    lib = C.CDLL(str(ROOT / "oracle" / "libstrata_oracle.so"))
    B, Hq, _, D = q.shape
    _, Hkv, L, _ = k.shape
    out = np.zeros((B, Hq, D), np.float32)
    P = C.c_void_p
    qf = np.ascontiguousarray(q.reshape(B, Hq, D), np.float32)
    lib.oracle_decode_attn(qf.ctypes.data_as(P), k.ctypes.data_as(P), v.ctypes.data_as(P), B, Hq,
                           Hkv, L, D, out.ctypes.data_as(P))
    return out.reshape(B, Hq, 1, D)


@pytest.mark.parametrize("B,L", [(1, 1024), (1, 8192), (16, 1024), (1, 32768), (16, 8192),
                                 (16, 32768)])
def test_config3_cached_decode_bf16(dev, B, L):
    """Hq32/Hkv8, D128, bf16 KV cache; append one token, then attend."""
    from types import SimpleNamespace
    from lokahi_amd import ops
    from lokahi_amd.kvcache import HipKVCache
    Hq, Hkv, D = 32, 8, 128
    g = torch.Generator(device=dev).manual_seed(B * 100000 + L)
    cfg = SimpleNamespace(num_hidden_layers=1, num_key_value_heads=Hkv, num_attention_heads=Hq,
                          hidden_size=Hq * D)
    cache = HipKVCache(cfg, batch_size=B, max_length=L + 1, dtype=torch.bfloat16)
    ctx_k = torch.randn((B, Hkv, L, D), generator=g, device=dev).to(torch.bfloat16)
    ctx_v = torch.randn((B, Hkv, L, D), generator=g, device=dev).to(torch.bfloat16)
    cache.update(ctx_k, ctx_v, 0)
    qn = torch.randn((B, 1, Hq * D), generator=g, device=dev).to(torch.bfloat16)
    kn = torch.randn((B, 1, Hkv * D), generator=g, device=dev).to(torch.bfloat16)
    vn = torch.randn((B, 1, Hkv * D), generator=g, device=dev).to(torch.bfloat16)
    qo = torch.empty((B, Hq, 1, D), dtype=torch.bfloat16, device=dev)
    cache.rope_append(0, qn, kn, vn, Hq, 1, 500000.0, qo)
    K, V = cache.views(0)
    out = ops.attention(qo, K, V, kv_strides=cache.kv_strides)
    assert cache.get_seq_length(0) == L + 1
    kb = K.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)
    vb = V.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)
    ref = _c_decode(to_np_f32(qo), kb, vb)
    assert rel_err(to_np_f32(out), ref) < TOL_BF16
    assert np.abs(to_np_f32(out) - ref).max() < 2e-2


@pytest.mark.parametrize("L,chunk", [(256, 64), (1000, 512), (2048, 512)])
def test_config5_prefill_bf16_mfma(dev, L, chunk):
    """BASELINE config 5 geometry (Hq32/Hkv8, D128, bf16, causal, chunk 512) at test sizes."""
    from lokahi_amd import ops
    rng = np.random.default_rng(L)
    B, Hq, Hkv, D = 1, 32, 8, 128
    q = round_bf16(rng.normal(size=(B, Hq, L, D)).astype(np.float32))
    k = round_bf16(rng.normal(size=(B, Hkv, L, D)).astype(np.float32))
    v = round_bf16(rng.normal(size=(B, Hkv, L, D)).astype(np.float32))
    out = ops.attention(bf16_dev(q, dev), bf16_dev(k, dev), bf16_dev(v, dev),
                        q_block_size=chunk, k_block_size=chunk)
    ref = att.chunked_gqa(q, k, v, None, True, chunk, chunk)
    assert rel_err(to_np_f32(out), ref) < TOL_BF16


@pytest.mark.parametrize("D,Hq,Hkv", [(64, 8, 2), (128, 12, 4), (64, 24, 8)])
def test_prefill_bf16_mfma32_ragged_positions_and_non_causal(dev, D, Hq, Hkv):
    """The bf16 32x32x16 prefill kernel off the bench geometry: head dims 64
    and 128, groups 4 and 3, batch 2, queries at explicit positions over a
    longer key range (32-key tiles with a tail, rows past Lq in the last
    128-row tile), and the non-causal form, against the float64 oracle."""
    from lokahi_amd import ops
    rng = np.random.default_rng(D * 100 + Hq)
    B, Lq, Lk = 2, 70, 150
    q = round_bf16(rng.normal(size=(B, Hq, Lq, D)).astype(np.float32))
    k = round_bf16(rng.normal(size=(B, Hkv, Lk, D)).astype(np.float32))
    v = round_bf16(rng.normal(size=(B, Hkv, Lk, D)).astype(np.float32))
    pos = np.stack([np.arange(Lk - Lq, Lk), np.sort(rng.integers(0, Lk, Lq))])
    tq, tk, tv = bf16_dev(q, dev), bf16_dev(k, dev), bf16_dev(v, dev)
    out = ops.attention(tq, tk, tv, query_positions=_t(pos, dev))
    assert rel_err(to_np_f32(out), att.naive_gqa(q, k, v, pos)) < TOL_BF16
    nm = ops.attention(tq, tk, tv, causal=False)
    assert rel_err(to_np_f32(nm), att.naive_gqa(q, k, v)) < TOL_BF16
    # bottom-right causal over Lq = Lk = 300 (several tiles, a partial last one)
    L = 300
    q2 = round_bf16(rng.normal(size=(1, Hq, L, D)).astype(np.float32))
    k2 = round_bf16(rng.normal(size=(1, Hkv, L, D)).astype(np.float32))
    v2 = round_bf16(rng.normal(size=(1, Hkv, L, D)).astype(np.float32))
    o2 = ops.attention(bf16_dev(q2, dev), bf16_dev(k2, dev), bf16_dev(v2, dev))
    ref2 = att.naive_gqa(q2, k2, v2, np.arange(L)[None])  # positions: causal
    assert rel_err(to_np_f32(o2), ref2) < TOL_BF16


def test_prefill_fp32_mfma_ragged_and_positions(dev):
    from lokahi_amd import ops
    rng = np.random.default_rng(77)
    B, Hq, Hkv, D = 2, 4, 1, 128
    Lq, Lk = 70, 150
    q = rng.normal(size=(B, Hq, Lq, D)).astype(np.float32)
    k = rng.normal(size=(B, Hkv, Lk, D)).astype(np.float32)
    v = rng.normal(size=(B, Hkv, Lk, D)).astype(np.float32)
    pos = np.stack([np.arange(Lk - Lq, Lk), np.sort(rng.integers(0, Lk, Lq))])
    out = ops.attention(_t(q, dev), _t(k, dev), _t(v, dev), query_positions=_t(pos, dev))
    ref = att.naive_gqa(q, k, v, pos)
    assert rel_err(out.cpu().numpy(), ref) < TOL_F32
    nm = ops.attention(_t(q, dev), _t(k, dev), _t(v, dev), causal=False)
    assert rel_err(nm.cpu().numpy(), att.naive_gqa(q, k, v)) < TOL_F32


def test_decode_equals_last_row_of_prefill_and_chunk_independence(dev):
    from lokahi_amd import ops
    rng = np.random.default_rng(5)
    B, Hq, Hkv, D, L = 1, 16, 4, 64, 300
    q = rng.normal(size=(B, Hq, L, D)).astype(np.float32)
    k = rng.normal(size=(B, Hkv, L, D)).astype(np.float32)
    v = rng.normal(size=(B, Hkv, L, D)).astype(np.float32)
    full = ops.attention(_t(q, dev), _t(k, dev), _t(v, dev)).cpu().numpy()
    last = ops.attention(_t(q[:, :, -1:], dev), _t(k, dev), _t(v, dev)).cpu().numpy()
    np.testing.assert_allclose(full[:, :, -1:], last, atol=1e-4, rtol=1e-4)
    other = ops.attention(_t(q, dev), _t(k, dev), _t(v, dev), q_block_size=7, k_block_size=3)
    np.testing.assert_allclose(full, other.cpu().numpy(), atol=1e-6)


@pytest.mark.parametrize("Hq,dtype", [(24, "bf16"), (48, "bf16"), (24, "f32")])
def test_decode_group_sizes_3_and_6(dev, Hq, dtype):
    """GQA groups of 3 (Llama-3.2-3B: 24 query / 8 KV heads) and 6 on the split-K decode kernel."""
    from lokahi_amd import ops
    rng = np.random.default_rng(Hq)
    B, Hkv, D, L = 2, 8, 128, 700
    q = round_bf16(rng.normal(size=(B, Hq, 1, D)).astype(np.float32))
    k = round_bf16(rng.normal(size=(B, Hkv, L, D)).astype(np.float32))
    v = round_bf16(rng.normal(size=(B, Hkv, L, D)).astype(np.float32))
    if dtype == "bf16":
        out = to_np_f32(ops.attention(bf16_dev(q, dev), bf16_dev(k, dev), bf16_dev(v, dev)))
        tol = TOL_BF16
    else:
        out = ops.attention(_t(q, dev), _t(k, dev), _t(v, dev)).cpu().numpy()
        tol = TOL_F32
    ref = att.chunked_gqa(q, k, v, None, True, 32768, 1024)
    assert rel_err(out, ref) < tol


@pytest.mark.parametrize("B,Hq,Hkv,D,L", [(16, 24, 8, 128, 300), (32, 8, 2, 64, 257),
                                          (8, 64, 8, 128, 97)])
def test_decode_batched_heads_mfma(dev, B, Hq, Hkv, D, L):
    """B * Hkv >= 64 runs the MFMA decode kernel (the G query heads of a KV head
    are the MFMA columns; G = 3, 4 and 8 here).  Per-row query positions cut
    each row's visible keys at a different point, including inside a 32-key
    tile and at the first key; the reference is float64 attention."""
    from lokahi_amd import ops
    rng = np.random.default_rng(B * 1000 + L)
    q = round_bf16(rng.normal(size=(B, Hq, 1, D)).astype(np.float32))
    k = round_bf16(rng.normal(size=(B, Hkv, L, D)).astype(np.float32))
    v = round_bf16(rng.normal(size=(B, Hkv, L, D)).astype(np.float32))
    pos = rng.integers(0, L, size=(B, 1))
    pos[0, 0], pos[-1, 0] = 0, L - 1
    out = to_np_f32(ops.attention(bf16_dev(q, dev), bf16_dev(k, dev), bf16_dev(v, dev),
                                  query_positions=torch.from_numpy(pos.astype(np.int32))))
    ref = att.naive_gqa(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), pos)
    assert rel_err(out, ref) < TOL_BF16
    assert np.abs(out - ref).max() < 2e-2


def test_decode_split_k_back_to_back_and_graph_replays(dev):
    """Split-K decode calls of different geometry in a row (the partials of
    one call in the scratch arena the next call reuses), then graph replays of
    one call with eager calls of another geometry in between: every output
    must match the float64 attention."""
    from lokahi_amd import ops
    rng = np.random.default_rng(2048)
    cases = [(1, 32, 8, 128, 2049), (1, 24, 8, 128, 777), (2, 8, 8, 64, 300),
             (1, 32, 8, 128, 4100), (1, 8, 1, 128, 1500), (1, 32, 8, 128, 65)]
    data = []
    for B, Hq, Hkv, D, L in cases:
        q = round_bf16(rng.normal(size=(B, Hq, 1, D)).astype(np.float32))
        k = round_bf16(rng.normal(size=(B, Hkv, L, D)).astype(np.float32))
        v = round_bf16(rng.normal(size=(B, Hkv, L, D)).astype(np.float32))
        ref = att.naive_gqa(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64))
        data.append(([bf16_dev(a, dev) for a in (q, k, v)], ref))
    for rep in range(2):
        for (tq, tk, tv), ref in data:
            out = to_np_f32(ops.attention(tq, tk, tv))
            assert rel_err(out, ref) < TOL_BF16 and np.abs(out - ref).max() < 2e-2, rep
    (tq, tk, tv), ref = data[0]
    out = torch.empty_like(tq)
    ops.attention(tq, tk, tv, out=out)  # eager first: sizes the scratch arena
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.attention(tq, tk, tv, out=out)
    (eq, ek, ev), eref = data[1]
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        got = to_np_f32(out)
        assert rel_err(got, ref) < TOL_BF16 and np.abs(got - ref).max() < 2e-2
        e = to_np_f32(ops.attention(eq, ek, ev))
        assert rel_err(e, eref) < TOL_BF16
