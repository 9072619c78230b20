"""Benchmark: Llama-3-8B-shaped q4 decode at batch 1 on one MI355X.

Headline (``value``): one "step" = one greedy decode token through the full
32-layer 8B-shaped model (q4 group-64 linears, bf16 embedding / lm_head, bf16
KV cache, RoPE theta 5e5) after a 2048-token prefill, with every input already
resident in HBM; ``value`` is decode tokens/s, the decode steps launched from
C++ by the native engine (its default; replaying each step as a captured HIP
graph measured 7-11% slower on this runtime).

``roofline``: the dominant kernel, the q4 GEMV, on the six-linear set of
config 2 ([4096->4096], [4096->1024] x2, [4096->14336] x2, [14336->4096]) as
the decode engine launches it (q/k/v in one launch, gate/up in one launch,
down alone).  Each launch kind is captured ``--gemv-iters`` times back to
back into one graph; HIP events on the capture stream bracket its replay, so
the average launch duration excludes host launch cost (it is the figure the
kernel-trace profile reports).  Weights rotate through six copies (680 MB) so
no launch finds them in the 256 MB Infinity Cache.

Further measurements on the same line (the other configs of the workload):
``attention_decode`` (config 3: cached decode GQA over bf16 KV, GB/s),
``prefill`` (config 5: q4 GEMM at M=8192 on MFMA and causal GQA prefill
attention, TFLOP/s), ``e2e_3b`` (config 4: Llama-3.2-3B-shaped greedy
generation, 2048-token prompt + 256 tokens), ``config1`` (fp32 chunked GQA +
RoPE latency) and ``cpu_baseline`` (the C restatement of the oracle on the
host cores, on a bounded sample of the per-token work).

``--profile gemv`` runs only the GEMV launches plus a 256 MiB device copy (a
plain copy kernel of known size), for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
passes; the measured HBM bytes per launch are kept in
profiles/q4_gemv_traffic.json and reported as ``roofline.traffic``.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
PROMPT = 2048


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=64)
    p.add_argument("--warmup", type=int, default=8)
    p.add_argument("--prompt", type=int, default=PROMPT)
    p.add_argument("--gemv-iters", type=int, default=50)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-extra", action="store_true", help="skip configs 1, 3, 4 and 5")
    p.add_argument("--profile", choices=["gemv", "prefill", "midrows", "floor"], default=None)
    return p.parse_args()


def q4_bytes(n, k, m=1):
    return n * k // 2 + 2 * 2 * n * (k // 64) + 2 * k * m + 2 * n * m


# The sources that determine the GEMV set's kernels and launches: the PMC
# traffic figure is tied to them.
GEMV_SOURCES = ("q4_gemv_mfma.hip", "strata_internal.h", "strata_common.h")


def csrc_hash() -> str:
    """sha256 over the GEMV set's kernel sources (name + bytes)."""
    import hashlib
    h = hashlib.sha256()
    csrc = ROOT / "lokahi_amd" / "csrc"
    for name in GEMV_SOURCES:
        h.update(name.encode())
        h.update((csrc / name).read_bytes())
    return h.hexdigest()


def graph_time_us(fn, iters, warm=2, reps=5):
    """Duration of `fn` captured `iters` times into one HIP graph, timed with
    events around each of `reps` replays; the median replay over `iters`."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(warm):
            fn(0)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(iters):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    times = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(st)
        g.replay()
        b.record(st)
        torch.cuda.synchronize()
        times.append(1e3 * a.elapsed_time(b) / iters)
    del g
    times.sort()
    return times[len(times) // 2]


def rep_stats(times):
    """min/median/p95/mean of a list of seconds, in milliseconds (the
    warmup-then-timed-repetitions protocol of linear_projection_bench.mm:83-110)."""
    t = sorted(times)
    p95 = t[min(len(t) - 1, int(round(0.95 * (len(t) - 1))))]
    return {"reps": len(t), "min_ms": round(1e3 * t[0], 3),
            "median_ms": round(1e3 * t[len(t) // 2], 3), "p95_ms": round(1e3 * p95, 3),
            "mean_ms": round(1e3 * sum(t) / len(t), 3)}


def gemv_sets():
    import torch
    from lokahi_amd import ops
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(7)

    def q4(n, k):
        return ops.quantize(torch.randn((n, k), generator=g, device=dev) * 0.02)

    copies = 6
    sets = [{"q": q4(4096, 4096), "k": q4(1024, 4096), "v": q4(1024, 4096),
             "gate": q4(14336, 4096), "up": q4(14336, 4096), "down": q4(4096, 14336)}
            for _ in range(copies)]
    x = torch.randn((1, 4096), generator=g, device=dev).to(torch.bfloat16)
    xd = torch.randn((1, 14336), generator=g, device=dev).to(torch.bfloat16)
    outs = {n: torch.empty((1, sets[0][n][0].shape[0]), dtype=torch.bfloat16, device=dev)
            for n in sets[0]}
    # the decode engine's load-time GEMV layout, one per launch group
    lays = [{"qkv": ops.Q4Layout([W["q"], W["k"], W["v"]]),
             "gate_up": ops.Q4Layout([W["gate"], W["up"]]),
             "down": ops.Q4Layout([W["down"]])} for W in sets]
    for W, L in zip(sets, lays):
        W["_lay"] = L
    launches = [
        ("qkv", lambda W: W["_lay"]["qkv"](x, outs=[outs["q"], outs["k"], outs["v"]]),
         q4_bytes(4096, 4096) + 2 * q4_bytes(1024, 4096) - 2 * 2 * 4096),  # x read once
        ("gate_up", lambda W: W["_lay"]["gate_up"](x, outs=[outs["gate"], outs["up"]]),
         2 * q4_bytes(14336, 4096) - 2 * 4096),
        ("down", lambda W: W["_lay"]["down"](xd, outs=[outs["down"]]),
         q4_bytes(4096, 14336)),
    ]
    return sets, launches


def gemv_roofline(iters):
    sets, launches = gemv_sets()
    copies = len(sets)
    per = {}
    for name, fn, nbytes in launches:
        us = graph_time_us(lambda i, fn=fn: fn(sets[i % copies]), iters)
        per[name] = {"bytes": nbytes, "avg_us": round(us, 3), "GBps": round(nbytes / (us * 1e3), 1)}
    tot_bytes = sum(v["bytes"] for v in per.values())
    tot_us = sum(v["avg_us"] for v in per.values())
    achieved = tot_bytes / (tot_us * 1e3)
    # what a plain streaming read of the same three sizes takes, same timing
    fl = read_floor_fixed()
    floor = {"us_per_set": round(sum(fl.values()), 2), "launches_us": fl,
             "frac": round(tot_bytes / (sum(fl.values()) * 1e3) / HBM_PEAK_GBS, 4),
             "set_vs_floor": round(sum(fl.values()) / tot_us, 4)}
    # the PMC traffic figure counts only when it was measured on this build's
    # kernel sources (profiles/q4_gemv_traffic.json records their hash)
    traffic = None
    tf = ROOT / "profiles" / "q4_gemv_traffic.json"
    if tf.exists():
        rec = json.loads(tf.read_text())
        if rec.get("csrc_sha256") == csrc_hash():
            traffic = rec.get("hbm_bytes_per_set")
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "kernel": "q4_gemv_mfma_kernel (six-linear set, 3 launches, GEMV layout)",
            "bytes_per_set": tot_bytes, "us_per_set": round(tot_us, 2), "launches": per,
            "read_floor": floor}


def profile_gemv(iters):
    """Only the GEMV launches plus a 256 MiB copy (for rocprofv3 --pmc passes)."""
    import torch
    sets, launches = gemv_sets()
    for name, fn, _ in launches:
        for i in range(iters):
            fn(sets[i % len(sets)])
    a = torch.empty(64 * 2**20, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"profile": "gemv", "iters": iters, "copy_bytes_read": a.numel() * 4}))


FLOOR_GEOMETRY = {"qkv": (14176256, 2, 8), "gate_up": (66125824, 8, 8), "down": (33067008, 8, 8)}


def read_floor_fixed():
    """The plain-read floor at the best geometry ``read_floor`` found per
    launch (MI355X): bytes, workgroups per CU, loads in flight."""
    import torch
    from lokahi_amd import _abi
    from lokahi_amd.ops import _ctx, _stream
    lib = _abi.load()
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    res = {}
    for name, (nbytes, wpc, u) in FLOOR_GEOMETRY.items():
        bufs = [torch.empty(nbytes // 4, dtype=torch.int32, device="cuda").fill_(i + 1)
                for i in range(6)]

        def fn(i):
            _abi.check(lib.strata_bench_read(_ctx(0), bufs[i % 6].data_ptr(), nbytes, wpc, u,
                                             sink.data_ptr(), _stream(0)))
        res[name] = round(graph_time_us(fn, 48), 3)
        del bufs
    return res


def read_floor():
    """Plain-read floor of the six-linear set's three launches: the library's
    streaming-read helper (``strata_bench_read``) over buffers of the
    launches' sizes, 6 copies cycled (past the last-level cache), graph-timed
    like the roofline leg, best over 2-8 workgroups per CU and 4-16 loads in
    flight per lane."""
    import torch
    from lokahi_amd import _abi
    from lokahi_amd.ops import _ctx, _stream
    lib = _abi.load()
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    res = {}
    for name, nbytes in (("qkv", 14176256), ("gate_up", 66125824), ("down", 33067008)):
        bufs = [torch.empty(nbytes // 4, dtype=torch.int32, device="cuda").fill_(i + 1)
                for i in range(6)]
        best = None
        for wpc in (2, 4, 8):
            for u in (4, 8, 16):
                def fn(i, wpc=wpc, u=u):
                    _abi.check(lib.strata_bench_read(_ctx(0), bufs[i % 6].data_ptr(), nbytes, wpc,
                                                     u, sink.data_ptr(), _stream(0)))
                us = graph_time_us(fn, 48)
                if best is None or us < best[0]:
                    best = (us, wpc, u)
        res[name] = {"bytes": nbytes, "us": round(best[0], 2), "wg_per_cu": best[1],
                     "loads_in_flight": best[2], "GBps": round(nbytes / best[0] / 1e3, 1)}
        del bufs
    res["set_us"] = round(sum(v["us"] for v in res.values() if isinstance(v, dict)), 2)
    res["set_frac_hbm"] = round(113369088 / res["set_us"] / 1e3 / HBM_PEAK_GBS, 4)
    return res


def profile_prefill(iters=3):
    """Config 5's kernels alone (for rocprofv3 passes): the causal bf16
    attention at 8192 tokens and the 8B gate projection at M = 8192 (weight
    re-layout + fused-dequant MFMA GEMM), each ``iters`` times."""
    import torch
    from lokahi_amd import ops
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(5)
    L = 8192
    q = torch.randn((1, 32, L, 128), generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn((1, 8, L, 128), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((1, 8, L, 128), generator=g, device=dev).to(torch.bfloat16)
    for _ in range(iters):
        ops.attention(q, k, v, causal=True)
    x = torch.randn((L, 4096), generator=g, device=dev).to(torch.bfloat16)
    w = ops.quantize(torch.randn((14336, 4096), generator=g, device=dev) * 0.02)
    for _ in range(iters):
        ops.linear(x, *w)
    torch.cuda.synchronize()
    print(json.dumps({"profile": "prefill", "iters": iters,
                      "attention_flops": 4 * 32 * 128 * L * (L + 1) // 2,
                      "gate_gemm_flops": 2 * L * 14336 * 4096}))


def profile_midrows(rows=(128, 200), iters=3):
    """The 8B layer's prefill linears as the engine launches them (q/k/v
    together, o, gate/up together, down) at a few mid-size row counts, each
    ``iters`` times (for rocprofv3 kernel traces of the split-K GEMM)."""
    import torch
    from lokahi_amd import ops
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(5)
    groups = [("qkv", (4096, 1024, 1024), 4096), ("o", (4096,), 4096),
              ("gate_up", (14336, 14336), 4096), ("down", (4096,), 14336)]
    ws = {name: [ops.quantize(torch.randn((n, k), generator=g, device=dev) * 0.02) for n in ns]
          for name, ns, k in groups}
    for M in rows:
        for name, ns, k in groups:
            x = torch.randn((M, k), generator=g, device=dev).to(torch.bfloat16)
            outs = [torch.empty((M, n), dtype=torch.bfloat16, device=dev) for n in ns]
            for _ in range(iters):
                ops.linear_multi(x, ws[name], outs=outs)
    torch.cuda.synchronize()
    print(json.dumps({"profile": "midrows", "rows": list(rows), "iters": iters}))


def attention_decode():
    """Config 3: Hq32/Hkv8, D128, bf16 KV.  Times the attend step over a cache
    that already holds the appended token (L + 1 keys); the append itself is
    one O(1) row write per layer and head (`strata_kv_append`), not timed
    here."""
    import torch
    from lokahi_amd import ops
    dev = torch.device("cuda", 0)
    res = []
    for B, L in [(1, 1024), (1, 2048), (1, 8192), (1, 32768), (16, 1024), (16, 8192), (16, 32768)]:
        g = torch.Generator(device=dev).manual_seed(B * 7 + L)
        q = torch.randn((B, 32, 1, 128), generator=g, device=dev).to(torch.bfloat16)
        k = torch.randn((B, 8, L + 1, 128), generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn((B, 8, L + 1, 128), generator=g, device=dev).to(torch.bfloat16)
        us = graph_time_us(lambda i: ops.attention(q, k, v), 10)
        kv = B * 8 * (L + 1) * 128 * 2 * 2
        res.append({"batch": B, "context": L, "us": round(us, 2), "kv_bytes": kv,
                    "GBps": round(kv / (us * 1e3), 1),
                    "frac_hbm": round(kv / (us * 1e3) / HBM_PEAK_GBS, 4)})
        del q, k, v
    torch.cuda.empty_cache()
    return res


def prefill_8b():
    """Config 5: q4 GEMM at M=8192 over the seven 8B linears, launched as the
    engine's prefill launches them (q/k/v together, o, gate/up together,
    down), + causal GQA prefill."""
    import torch
    from lokahi_amd import ops
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(5)
    M = 8192
    launches = [("qkv", [("q", 4096), ("k", 1024), ("v", 1024)], 4096), ("o", [("o", 4096)], 4096),
                ("gate_up", [("gate", 14336), ("up", 14336)], 4096), ("down", [("down", 4096)], 14336)]
    x = torch.randn((M, 4096), generator=g, device=dev).to(torch.bfloat16)
    xd = torch.randn((M, 14336), generator=g, device=dev).to(torch.bfloat16)
    tot_us, flops = 0.0, 0
    per = {}
    for name, shapes, k in launches:
        ws = [ops.quantize(torch.randn((n, k), generator=g, device=dev) * 0.02) for _, n in shapes]
        outs = [torch.empty((M, n), dtype=torch.bfloat16, device=dev) for _, n in shapes]
        xi = xd if k == 14336 else x
        us = graph_time_us(lambda i: ops.linear_multi(xi, ws, outs=outs), 3, warm=1)
        f = sum(2 * M * n * k for _, n in shapes)
        per[name] = {"us": round(us, 1), "TFLOPs": round(f / us / 1e6, 1),
                     "frac_mfma_bf16": round(f / us / 1e6 / MFMA_BF16_PEAK_TFLOPS, 4)}
        tot_us += us
        flops += f
        del ws, outs
    gemm = flops / tot_us / 1e6
    q = torch.randn((1, 32, M, 128), generator=g, device=dev).to(torch.bfloat16)
    kk = torch.randn((1, 8, M, 128), generator=g, device=dev).to(torch.bfloat16)
    vv = torch.randn((1, 8, M, 128), generator=g, device=dev).to(torch.bfloat16)
    aus = graph_time_us(lambda i: ops.attention(q, kk, vv, q_block_size=512, k_block_size=512),
                        3, warm=1)
    aflops = 4 * 32 * 128 * (M * (M + 1) // 2)
    del q, kk, vv, x, xd
    torch.cuda.empty_cache()
    return {"tokens": M,
            "q4_gemm": {"us_per_layer": round(tot_us, 1), "TFLOPs": round(gemm, 1),
                        "frac_mfma_bf16": round(gemm / MFMA_BF16_PEAK_TFLOPS, 4),
                        "kernel": "q4_gemm_mfma_kernel (hand-written fused dequant, bf16 MFMA)",
                        "launches": per},
            "attention": {"us": round(aus, 1), "TFLOPs": round(aflops / aus / 1e6, 1),
                          "frac_mfma_bf16": round(aflops / aus / 1e6 / MFMA_BF16_PEAK_TFLOPS, 4)}}


def run_decode(cfg, prompt_len, new_tokens, seed, batch=1, warm_tokens=None):
    """Prefill `prompt_len` uniform-random ids per row, then time `new_tokens`
    greedy decode steps per row on the native engine.

    An untimed pass first runs the same prefill and `warm_tokens` decode steps
    (default: `new_tokens`); it also captures the step graph of each 256-key
    bucket it reaches.  A bucket the timed pass reaches first is captured
    inside the timed region.  Each decode step is one forward of one token
    per row (the first from the prefill's last prompt token)."""
    import torch
    from lokahi_amd.llama import DecoderEngine, HipLlamaForCausalLM, random_weights
    warm_tokens = new_tokens if warm_tokens is None else warm_tokens
    weights = random_weights(cfg, seed=seed)
    model = HipLlamaForCausalLM(cfg, weights)
    cache = model.new_cache(batch, prompt_len + max(new_tokens, warm_tokens) + 8)
    engine = DecoderEngine(model, cache, max_batch=batch, max_tokens=batch * prompt_len)
    gen = torch.Generator().manual_seed(seed)
    prompt = torch.randint(0, cfg.vocab_size, (batch, prompt_len), generator=gen)
    times = []
    for n in (warm_tokens, new_tokens):
        cache.clear()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        engine.forward(prompt[:, :-1])
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        toks = engine.generate(prompt[:, -1:], n) if n > 0 else None
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        times.append((t1 - t0, t2 - t1))
    prefill_s, decode_s = times[-1]
    del engine, model, weights, cache
    torch.cuda.empty_cache()
    return prefill_s, decode_s, toks


def decode_bytes(cfg, ctx_avg):
    lin = (cfg.hidden_size * cfg.hidden_size * 2  # q, o
           + 2 * cfg.hidden_size * cfg.num_key_value_heads * cfg.head_dim  # k, v
           + 3 * cfg.hidden_size * cfg.intermediate_size)  # gate, up, down
    q4 = lin // 2 + 4 * (lin // 64)
    kv = 2 * 2 * cfg.num_key_value_heads * cfg.head_dim * ctx_avg
    return cfg.num_hidden_layers * (q4 + kv) + cfg.vocab_size * cfg.hidden_size * 2


def decode_batch8():
    """Serving view (not a BASELINE config): the 8B shape decoding 8 sequences
    at once, 512-token prompts, 32 timed tokens per sequence; aggregate tok/s.
    The q4 linears then run the batched GEMV (8 rows share each weight read)."""
    from lokahi_amd.llama import LLAMA3_8B
    B, P, T = 8, 512, 33
    prefill_s, decode_s, _ = run_decode(LLAMA3_8B, P, T, seed=3, batch=B)
    return {"batch": B, "prompt": P, "new_tokens_per_row": T,
            "decode_tok_s": round(B * T / decode_s, 1),
            "ms_per_step": round(1e3 * decode_s / T, 3), "prefill_s": round(prefill_s, 3)}


def e2e_3b():
    """Config 4: Llama-3.2-3B-shaped greedy generation, 2048-token prompt + 256 tokens."""
    from lokahi_amd.llama import LLAMA32_3B
    n = 256
    prefill_s, decode_s, _ = run_decode(LLAMA32_3B, 2048, n, seed=77)
    tok_s = n / decode_s
    byts = decode_bytes(LLAMA32_3B, 2048 + n // 2)
    return {"model": "Llama-3.2-3B shape (28 layers, 3072/8192, 24q/8kv heads, vocab 128256)",
            "prompt": 2048, "new_tokens": n, "decode_tok_s": round(tok_s, 1),
            "prefill_s": round(prefill_s, 4), "bytes_per_token": byts,
            "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / byts, 1),
            "frac_of_roofline": round(tok_s * byts / (HBM_PEAK_GBS * 1e9), 4)}


def config1():
    """Config 1: B1, Hq8/Hkv2, D64, L512, chunks 128, RoPE theta 1e4, fp32."""
    import torch
    from lokahi_amd import ops
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(1)
    q = torch.randn((1, 8, 513, 64), generator=g, device=dev)
    k = torch.randn((1, 2, 513, 64), generator=g, device=dev)
    v = torch.randn((1, 2, 513, 64), generator=g, device=dev)
    pos = torch.arange(513, device=dev, dtype=torch.int32)[None]
    qp, kp, vp, posp = q[:, :, :512].contiguous(), k[:, :, :512].contiguous(), \
        v[:, :, :512].contiguous(), pos[:, :512].contiguous()
    qd = q[:, :, 512:].contiguous()
    posd = torch.tensor([[512]], dtype=torch.int32, device=dev)

    def pre(i):
        ops.rope(qp, kp, posp, 10000.0)
        ops.attention(qp, kp, vp, query_positions=posp, q_block_size=128, k_block_size=128)

    def dec(i):
        ops.attention(qd, k, v, query_positions=posd)
    return {"prefill_us": round(graph_time_us(pre, 20), 2),
            "decode_us": round(graph_time_us(dec, 20), 2)}


def _np_q4_linear(x, w, s, b):
    """NumPy lane: dequantize the q4 matrix to float32 on every call, then
    one BLAS matvec (q4 affine format: nibble j of word i is k = 8i + j)."""
    import numpy as np
    n, kw = w.shape
    shifts = np.arange(0, 32, 4, dtype=np.uint32)
    codes = ((w[:, :, None] >> shifts) & 0xF).astype(np.float32).reshape(n, -1, 64)
    sf = (s.astype(np.uint32) << 16).view(np.float32)
    bf = (b.astype(np.uint32) << 16).view(np.float32)
    wd = (codes * sf[:, :, None] + bf[:, :, None]).reshape(n, kw * 8)
    return wd @ x


def _np_decode_attn(q, kc, vc):
    """NumPy lane: one query per head against the whole cache (GQA groups)."""
    import numpy as np
    hq, d = q.shape
    hkv = kc.shape[0]
    k = (kc.astype(np.uint32) << 16).view(np.float32)
    v = (vc.astype(np.uint32) << 16).view(np.float32)
    qg = q.reshape(hkv, hq // hkv, d)
    sc = np.einsum("hgd,hld->hgl", qg, k) / np.sqrt(d)
    sc = np.exp(sc - sc.max(-1, keepdims=True))
    sc /= sc.sum(-1, keepdims=True)
    return np.einsum("hgl,hld->hgd", sc, v).reshape(hq, d)


def cpu_baseline(prompt):
    """CPU restatement timed on a bounded sample: one 8B layer's seven q4
    linears, decode attention at the prompt length for one layer, and 1/8 of
    the bf16 lm_head; scaled to one token (x32 layers, x8 lm_head).  Two
    lanes: the C restatement (OpenMP) and NumPy (dequantize + BLAS matmul per
    call); warmup, then timed repetitions reported as min/median/p95/mean."""
    import numpy as np
    lib_path = ROOT / "oracle" / "libstrata_oracle.so"
    lib = C.CDLL(str(lib_path))
    rng = np.random.default_rng(0)
    P = C.c_void_p
    shapes = [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (14336, 4096),
              (14336, 4096), (4096, 14336)]
    mats = []
    for n, k in shapes:
        w = rng.integers(0, 2**32, size=(n, k // 8), dtype=np.uint32)
        s = np.full((n, k // 64), 0x3c00, np.uint16)
        b = np.full((n, k // 64), 0xbc00, np.uint16)
        x = np.full(k, 0x3f80, np.uint16)
        y = np.zeros(n, np.uint16)
        mats.append((n, k, w, s, b, x, y))
    Hq, Hkv, D = 32, 8, 128
    q = rng.normal(size=(1, Hq, D)).astype(np.float32)
    kc = rng.integers(0, 2**16, size=(1, Hkv, prompt, D), dtype=np.uint16) & 0x3fff
    vc = kc.copy()
    ao = np.zeros((1, Hq, D), np.float32)
    V8 = 128256 // 8
    lw = rng.integers(0, 2**16, size=(V8, 4096), dtype=np.uint16) & 0x3fff
    lx = np.full(4096, 0x3f80, np.uint16)
    ly = np.zeros(V8, np.float32)

    def one_c():
        t0 = time.perf_counter()
        for n, k, w, s, b, x, y in mats:
            lib.oracle_q4_gemv_bf16(x.ctypes.data_as(P), C.c_int64(k), w.ctypes.data_as(P),
                                    s.ctypes.data_as(P), b.ctypes.data_as(P), C.c_int64(n),
                                    C.c_int(64), y.ctypes.data_as(P))
        t1 = time.perf_counter()
        lib.oracle_decode_attn(q.ctypes.data_as(P), kc.ctypes.data_as(P), vc.ctypes.data_as(P),
                               1, Hq, Hkv, prompt, D, ao.ctypes.data_as(P))
        t2 = time.perf_counter()
        lib.oracle_bf16_gemv(lx.ctypes.data_as(P), C.c_int64(4096), lw.ctypes.data_as(P),
                             C.c_int64(V8), ly.ctypes.data_as(P))
        t3 = time.perf_counter()
        return (t1 - t0) * 32 + (t2 - t1) * 32 + (t3 - t2) * 8

    xf = {k: np.ones(k, np.float32) for k in (4096, 14336)}

    def one_np():
        t0 = time.perf_counter()
        for n, k, w, s, b, x, y in mats:
            _np_q4_linear(xf[k], w, s, b)
        t1 = time.perf_counter()
        _np_decode_attn(q[0], kc[0], vc[0])
        t2 = time.perf_counter()
        ((lw.astype(np.uint32) << 16).view(np.float32)) @ xf[4096]
        t3 = time.perf_counter()
        return (t1 - t0) * 32 + (t2 - t1) * 32 + (t3 - t2) * 8

    def lane(fn, budget_s, max_reps):
        fn()  # warm
        times, t_start = [], time.perf_counter()
        while len(times) < 3 or (time.perf_counter() - t_start < budget_s
                                 and len(times) < max_reps):
            times.append(fn())
        return times

    tc = lane(one_c, 10.0, 50)
    tn = lane(one_np, 10.0, 20)
    med_c = sorted(tc)[len(tc) // 2]
    med_n = sorted(tn)[len(tn) // 2]
    omp = int(os.environ.get("OMP_NUM_THREADS", 0)) or os.cpu_count()
    sc, sn = rep_stats(tc), rep_stats(tn)
    sc["tok_s"], sn["tok_s"] = round(1.0 / med_c, 3), round(1.0 / med_n, 3)
    sn["cores"] = os.cpu_count()
    return {"value": round(1.0 / med_c, 3), "unit": "tok/s", "cores": omp, "kind": "port",
            "sample": ("C restatement (OpenMP) per token from one 8B layer's 7 q4 GEMVs + decode "
                       f"attention at L={prompt} (x32 layers) + 1/8 of the bf16 lm_head (x8); "
                       "value from the median repetition"),
            "lanes": {"c_openmp_per_token": sc, "numpy_dequant_matmul_per_token": sn}}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only (no multi-GPU path); "
                                   "run with --gpus 1"}))
        sys.exit(2)
    import torch
    if args.profile == "floor":
        print(json.dumps({"profile": "floor", "read_floor": read_floor()}))
        return
    if args.profile == "gemv":
        profile_gemv(args.gemv_iters)
        return
    if args.profile == "prefill":
        profile_prefill()
        return
    if args.profile == "midrows":
        profile_midrows()
        return
    from lokahi_amd.llama import LLAMA3_8B

    cfg = LLAMA3_8B
    K, W = args.steps, args.warmup  # timed and untimed decode steps (one token each)
    if K < 1:
        raise SystemExit("--steps must be at least 1")
    prefill_s, decode_s, _ = run_decode(cfg, args.prompt, K, seed=1234, warm_tokens=W)
    tok_s = K / decode_s
    ms_per_step = 1e3 * decode_s / K
    token_bytes = decode_bytes(cfg, args.prompt + K // 2)

    roof = gemv_roofline(args.gemv_iters)
    line = {
        "metric": "decode tok/s, Llama-3-8B-shape q4 bs=1; q4 GEMV HBM GB/s (% of peak)",
        "value": round(tok_s, 3), "unit": "tok/s", "n_gpus": 1, "steps": K,
        "warmup": W, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16 activations, q4 weights, fp32 accumulate",
        "data": "synthetic (random-init weights N(0,0.02) quantized on device; uniform-random prompt ids)",
        "config": {"workload": "llama3-8b-shape q4 greedy decode, batch 1, after 2048-token prefill "
                               "(native engine, decode steps launched from C++)",
                   "model": "Llama-3-8B shape (32 layers, 4096/14336, 32q/8kv heads, vocab 128256)",
                   "global_batch": 1, "seq_len": args.prompt, "parallelism": "single GPU"},
        "decode_bandwidth": {"bytes_per_token": token_bytes,
                             "achieved_GBps": round(token_bytes * tok_s / 1e9, 1),
                             "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / token_bytes, 1),
                             "frac_of_roofline": round(token_bytes * tok_s / (HBM_PEAK_GBS * 1e9), 4)},
        "prefill_s": round(prefill_s, 3),
        "roofline": roof,
    }
    if not args.no_extra:
        line["attention_decode"] = attention_decode()
        line["prefill"] = prefill_8b()
        line["e2e_3b"] = e2e_3b()
        line["config1"] = config1()
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.prompt)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
