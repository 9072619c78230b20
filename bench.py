"""Benchmark: Llama-3-8B-shaped q4 decode at batch 1 on one MI355X.

One "step" = one greedy decode token through the full 32-layer 8B-shaped
model (q4 group-64 linears, bf16 embedding / lm_head, bf16 KV cache, RoPE
theta 5e5) after a 2048-token prefill, with every input already resident in
HBM.  ``value`` is decode tokens/s.

The same run measures the dominant kernel, the q4 GEMV, on the BASELINE
config-2 six-linear set ([4096->4096], [4096->1024] x2, [4096->14336] x2,
[14336->4096]) as the decode driver launches it (q/k/v in one launch,
gate/up in one launch, down alone), timing every launch with HIP events on
the stream it runs on -> ``roofline``; and times the CPU restatement
(oracle/libstrata_oracle.so, OpenMP on all host cores) on a bounded sample
of the same per-token work -> ``cpu_baseline``.
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
PROMPT = 2048


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=64)
    p.add_argument("--warmup", type=int, default=8)
    p.add_argument("--prompt", type=int, default=PROMPT)
    p.add_argument("--gemv-iters", type=int, default=50)
    p.add_argument("--no-cpu", action="store_true")
    return p.parse_args()


def q4_bytes(n, k, m=1):
    return n * k // 2 + 2 * 2 * n * (k // 64) + 2 * k * m + 2 * n * m


def gemv_roofline(iters):
    """Time the decode-layer q4 GEMV launches with HIP events on their stream."""
    import torch
    from lokahi_amd import ops
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(7)

    def q4(n, k):
        return ops.quantize(torch.randn((n, k), generator=g, device=dev) * 0.02)

    # Six copies of the six-linear set (680 MB) are cycled so that no launch
    # finds its weights in the 256 MB last-level (Infinity) cache.
    copies = 6
    sets = [{"q": q4(4096, 4096), "k": q4(1024, 4096), "v": q4(1024, 4096),
             "gate": q4(14336, 4096), "up": q4(14336, 4096), "down": q4(4096, 14336)}
            for _ in range(copies)]
    x = torch.randn((1, 4096), generator=g, device=dev).to(torch.bfloat16)
    xd = torch.randn((1, 14336), generator=g, device=dev).to(torch.bfloat16)
    outs = {n: torch.empty((1, sets[0][n][0].shape[0]), dtype=torch.bfloat16, device=dev)
            for n in sets[0]}
    launches = [
        ("qkv", lambda W: ops.linear_multi(x, [W["q"], W["k"], W["v"]],
                                           outs=[outs["q"], outs["k"], outs["v"]]),
         q4_bytes(4096, 4096) + 2 * q4_bytes(1024, 4096) - 2 * 2 * 4096),  # x read once
        ("gate_up", lambda W: ops.linear_multi(x, [W["gate"], W["up"]],
                                               outs=[outs["gate"], outs["up"]]),
         2 * q4_bytes(14336, 4096) - 2 * 4096),
        ("down", lambda W: ops.linear_multi(xd, [W["down"]], outs=[outs["down"]]),
         q4_bytes(4096, 14336)),
    ]
    stream = torch.cuda.current_stream(dev)
    for _, fn, _ in launches:
        for c in range(copies):
            fn(sets[c])
    torch.cuda.synchronize()
    per = {}
    for name, fn, nbytes in launches:
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(iters)]
        # A spin kernel holds the stream while the host enqueues every timed
        # launch, so the event pairs bracket back-to-back kernels, not host
        # launch latency.
        torch.cuda._sleep(200_000_000)
        for it, (a, b) in enumerate(evs):
            a.record(stream)
            fn(sets[it % copies])
            b.record(stream)
        torch.cuda.synchronize()
        ms = sorted(a.elapsed_time(b) for a, b in evs)
        per[name] = {"bytes": nbytes, "avg_us": 1e3 * sum(ms) / len(ms),
                     "median_us": 1e3 * ms[len(ms) // 2]}
    tot_bytes = sum(v["bytes"] for v in per.values())
    tot_us = sum(v["avg_us"] for v in per.values())
    for v in per.values():
        v["GBps"] = v["bytes"] / (v["avg_us"] * 1e3)
    achieved = tot_bytes / (tot_us * 1e3)
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": "q4_gemv_kernel (six-linear set, 3 launches)",
            "bytes_per_set": tot_bytes, "us_per_set": round(tot_us, 2),
            "launches": {k: {kk: round(vv, 3) if isinstance(vv, float) else vv
                             for kk, vv in v.items()} for k, v in per.items()}}


def cpu_baseline(prompt):
    """CPU restatement timed on a bounded sample: one 8B layer's seven q4
    linears, decode attention at the prompt length for one layer, and 1/8 of
    the bf16 lm_head; scaled to one token (x32 layers, x8 lm_head)."""
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

    def one():
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

    one()  # warm
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < 10.0 and len(times) < 50):
        times.append(one())
    times.sort()
    per_token = times[len(times) // 2]
    cores = int(os.environ.get("OMP_NUM_THREADS", 0)) or os.cpu_count()
    return {"value": round(1.0 / per_token, 3), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": (f"C restatement (OpenMP), median of {len(times)} reps of: one 8B layer's "
                       f"7 q4 GEMVs + decode attention at L={prompt} (x32 layers) + 1/8 of the "
                       f"bf16 lm_head (x8)")}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; run with --gpus 1"}))
        sys.exit(2)
    import torch
    from lokahi_amd.llama import LLAMA3_8B, DecoderEngine, HipLlamaForCausalLM, random_weights
    from lokahi_amd import ops

    cfg = LLAMA3_8B
    torch.manual_seed(0)
    weights = random_weights(cfg, seed=1234)
    model = HipLlamaForCausalLM(cfg, weights)
    K = args.steps + 1  # tokens per timed generate call (first one is host-launched)
    cache = model.new_cache(1, args.prompt + 2 * K + 8)
    engine = DecoderEngine(model, cache, max_batch=1, max_tokens=args.prompt)
    gen = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, cfg.vocab_size, (1, args.prompt), generator=gen)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    logits = engine.forward(prompt[:, :-1])  # prefill prompt[:-1]
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    # warmup: one full generate call of K tokens (captures the decode-step
    # HIP graph, which the timed call replays)
    toks = engine.generate(prompt[:, -1:], K)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    toks = engine.generate(toks[:, -1:], K)  # K greedy decode steps, graph-replayed
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = 1e3 * elapsed / K
    tok_s = K / elapsed
    del logits

    roof = gemv_roofline(args.gemv_iters)
    # bytes one decode token must stream at this context (weights + KV + lm_head)
    lin = sum(q4_bytes(n, k) for n, k in [(4096, 4096), (1024, 4096), (1024, 4096),
                                          (4096, 4096), (14336, 4096), (14336, 4096),
                                          (4096, 14336)])
    ctx = args.prompt + K + K // 2
    token_bytes = cfg.num_hidden_layers * (lin + 2 * 2 * 8 * 128 * ctx) + cfg.vocab_size * 4096 * 2
    line = {
        "metric": "decode tok/s, Llama-3-8B-shape q4 bs=1; q4 GEMV HBM GB/s (% of peak)",
        "value": round(tok_s, 3), "unit": "tok/s", "n_gpus": 1, "steps": K,
        "warmup": K, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16 activations, q4 weights, fp32 accumulate",
        "data": "synthetic (random-init weights N(0,0.02) quantized on device; uniform-random prompt ids)",
        "config": {"workload": "llama3-8b-shape q4 greedy decode, batch 1, after 2048-token prefill "
                               "(native engine, HIP-graph decode step)",
                   "model": "Llama-3-8B shape (32 layers, 4096/14336, 32q/8kv heads, vocab 128256)",
                   "global_batch": 1, "seq_len": args.prompt, "parallelism": "single GPU"},
        "decode_bandwidth": {"bytes_per_token": token_bytes,
                             "achieved_GBps": round(token_bytes * tok_s / 1e9, 1),
                             "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / token_bytes, 1),
                             "frac_of_roofline": round(token_bytes * tok_s / (HBM_PEAK_GBS * 1e9), 4)},
        "prefill_s": round(prefill_s, 3),
        "roofline": roof,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.prompt)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
