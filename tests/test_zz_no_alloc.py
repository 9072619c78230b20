"""strata_attn_gqa_noalloc (static scratch, no allocation) against
strata_attn_gqa through the C ABI: bit-identical outputs on two calls in a
row, the second smaller, plus the size limit's error."""
import ctypes as C

import pytest
import torch

pytestmark = pytest.mark.gpu


def _call(fn, q, k, v, out, causal=1):
    from lokahi_amd import _abi
    from lokahi_amd.ops import _code, _ctx, _stream
    B, Hq, Lq, D = q.shape
    _, Hkv, Lk, _ = k.shape
    return fn(_ctx(0), q.data_ptr(), _code(q), k.data_ptr(), _code(k), v.data_ptr(), _code(v),
              Hkv * Lk * D, Lk * D, None, B, Hq, Hkv, Lq, Lk, D, causal, 32768, 1024,
              C.c_float(1e-12), out.data_ptr(), _stream(0))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_attention_matches_allocating_entry_point(dev, dtype):
    from lokahi_amd import _abi
    lib = _abi.load()
    g = torch.Generator(device=dev).manual_seed(7)
    # decode (split-K partials in the static scratch), then a smaller decode,
    # then a prefill (no scratch)
    for B, Hq, Hkv, Lq, Lk in [(2, 32, 8, 1, 8192), (1, 24, 8, 1, 1500), (1, 8, 2, 130, 300)]:
        q = torch.randn((B, Hq, Lq, 128), generator=g, device=dev).to(dtype)
        k = torch.randn((B, Hkv, Lk, 128), generator=g, device=dev).to(dtype)
        v = torch.randn((B, Hkv, Lk, 128), generator=g, device=dev).to(dtype)
        ref = torch.empty_like(q)
        got = torch.full_like(q, float("nan"))
        _abi.check(_call(lib.strata_attn_gqa, q, k, v, ref))
        _abi.check(_call(lib.strata_attn_gqa_noalloc, q, k, v, got))
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (B, Hq, Lq, Lk)


def test_noalloc_attention_rejects_oversized_scratch_and_bad_shapes(dev, monkeypatch):
    from lokahi_amd import _abi
    lib = _abi.load()
    # one KV head with 128 query heads over 32k keys: 256 key splits, 17 MB
    # of partials, more than the static scratch holds: rejected before any
    # launch
    q = torch.zeros((1, 128, 1, 128), device=dev, dtype=torch.bfloat16)
    k = torch.zeros((1, 1, 32768, 128), device=dev, dtype=torch.bfloat16)
    out = torch.empty_like(q)
    rc = _call(lib.strata_attn_gqa_noalloc, q, k, k, out)
    assert rc == _abi.STRATA_EINVAL and "static scratch" in _abi.last_error()
    q3 = torch.zeros((1, 6, 1, 128), device=dev)
    k3 = torch.zeros((1, 4, 8, 128), device=dev)
    rc = _call(lib.strata_attn_gqa_noalloc, q3, k3, k3, torch.empty_like(q3))
    assert rc == _abi.STRATA_EINVAL and "divisible" in _abi.last_error()
