// Chunked causal grouped-query attention for gfx950.
//
// Semantics follow online_chunked_grouped_attention_mx
// (src/ollm/backends/mlx_ops.py:32-152): scores = (q . k) * D^-1/2, key t is
// visible to a query at absolute position p iff t <= p (causal), softmax is
// accumulated online in fp32, out = wv / max(s, eps) in q's dtype.  Query
// positions default to bottom-right alignment arange(Lk - Lq, Lk) (69-72).
//
// Kernels:
//   * attn_decode_kernel : Lq == 1.  Split-K over the key axis; each workgroup
//     streams one key chunk of one KV head for its query heads (the whole
//     group G = Hq/Hkv, K/V read once, or half of it when the grid would not
//     fill the GPU), keeps per-16-lane online-softmax state in registers,
//     merges its lanes through LDS and writes (m, s, o[D]) partials;
//     attn_decode_merge combines the chunks.
//   * attn_decode_mfma : Lq == 1, bf16 q/k/v, batched heads (B * Hkv >= 64).
//     One wave per (b, KV head, key chunk); the G query heads are the columns
//     of 32x32x16 MFMAs, K/V tiles stream through a wave-private LDS ring;
//     partials merged by attn_decode_merge.
//   * attn_prefill_mfma32 : Lq > 1, bf16 q/k/v, D in {64, 128}.  Flash-style
//     on 32x32x16 MFMA: 32-key K and V tiles streamed straight from global
//     memory into LDS (two stages), S^T = K Q^T and O^T += V^T P^T, every
//     lane owns one query row and all softmax state is in-lane; V^T
//     operands come from row-major V through the LDS transpose read.  Key
//     tiles past the causal limit of the workgroup's query tile are skipped.
//   * attn_prefill_f32 : the same for fp32 inputs on 16x16x4 fp32 MFMA.
//   * attn_generic : any other shape (e.g. tiny head dims), one wave per query.
#include <algorithm>
#include <type_traits>
#include <cstdlib>

#include "strata_common.h"

namespace {

constexpr float kLog2e = 1.4426950408889634f;

template <typename T>
__device__ __forceinline__ void load_vec16(const T* p, float* out);  // 16 bytes -> floats

template <>
__device__ __forceinline__ void load_vec16<bf16_t>(const bf16_t* p, float* out) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    out[2 * c] = __uint_as_float(u[c] << 16);
    out[2 * c + 1] = __uint_as_float(u[c] & 0xffff0000u);
  }
}
template <>
__device__ __forceinline__ void load_vec16<float>(const float* p, float* out) {
  const float4 v = *reinterpret_cast<const float4*>(p);
  out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
}

// Load n (4 or 8) consecutive elements of V as floats.
template <typename T, int N>
__device__ __forceinline__ void load_elems(const T* p, float* out) {
  if constexpr (sizeof(T) * N == 16) {
    load_vec16<T>(p, out);
  } else if constexpr (sizeof(T) == 2 && N == 4) {  // bf16 x4 = 8 bytes
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    out[0] = __uint_as_float(v.x << 16); out[1] = __uint_as_float(v.x & 0xffff0000u);
    out[2] = __uint_as_float(v.y << 16); out[3] = __uint_as_float(v.y & 0xffff0000u);
  } else {  // f32 x8 = 32 bytes
    load_vec16<float>(reinterpret_cast<const float*>(p), out);
    load_vec16<float>(reinterpret_cast<const float*>(p) + 4, out + 4);
  }
}

// N consecutive elements of a K or V row held as raw bits (converted to
// floats only when used), so a pipelined loop can keep the next sweep's
// loads in flight in few registers.
template <typename T, int N>
struct Raw {
  static constexpr int W = N * (int)sizeof(T) / 4;  // 32-bit words
  uint32_t u[W];
  __device__ __forceinline__ void load(const T* p) {
    if constexpr (W % 4 == 0) {
#pragma unroll
      for (int i = 0; i < W / 4; ++i) {
        const uint4 v = reinterpret_cast<const uint4*>(p)[i];
        u[4 * i] = v.x; u[4 * i + 1] = v.y; u[4 * i + 2] = v.z; u[4 * i + 3] = v.w;
      }
    } else {
      const uint2 v = *reinterpret_cast<const uint2*>(p);
      u[0] = v.x; u[1] = v.y;
    }
  }
  __device__ __forceinline__ void to_float(float* out) const {
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int i = 0; i < W; ++i) {
        out[2 * i] = __uint_as_float(u[i] << 16);
        out[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int i = 0; i < W; ++i) out[i] = __uint_as_float(u[i]);
    }
  }
};

// --------------------------------------------------------------- decode (Lq=1)
// grid (nsplit, Hkv, B), block 256.  Each workgroup reduces one key chunk of
// one KV head for its G query heads to (m, s, o[D]) per head.  With several
// chunks the partials go to `part` and attn_decode_merge combines them (the
// kernel boundary orders the partials' writes before the merge's reads on
// every XCD).  Partials of one (b, hq), part_stride(nsplit, D) floats apart:
// o[nsplit][D], then (m, s)[nsplit] as float2 (16-byte aligned blocks, so the
// merge fetches them with wide loads in one round trip).
constexpr int kMaxDecodeSplits = 256;

// Everything the first K/V and q loads need leads the argument list (16
// dwords, preloaded into SGPRs with the dispatch).
template <typename TQ, typename TK, typename TV, int D, int G>
__global__ __launch_bounds__(256) void attn_decode_kernel(
    const TQ* __restrict__ q, const TK* __restrict__ k, const TV* __restrict__ v,
    int64_t kv_bs, int64_t kv_hs, int Lk, int chunk, int gfull, int Hq,
    const int32_t* __restrict__ qpos, const int* __restrict__ dlen, int causal, int nsplit,
    float scale, float eps, float* __restrict__ part, TQ* __restrict__ out) {
  constexpr int EPL = 16 / sizeof(TK);          // key elements per lane
  constexpr int LPK = D / EPL;                  // lanes per key
  constexpr int KPW = 64 / LPK;                 // keys per wave step
  constexpr int J = 4;                          // keys per stream per step
  static_assert(LPK <= 64 && 64 % LPK == 0, "unsupported head dim");

  // blockIdx.y = (kv head, slice): the workgroup serves G of the gfull query
  // heads of its KV head, hq0 .. hq0 + G - 1.
  const int split = blockIdx.x, b = blockIdx.z;
  const int hslices = gfull / G;
  const int hkv = blockIdx.y / hslices;
  const int hq0 = hkv * gfull + (blockIdx.y - hkv * hslices) * G;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / LPK, part_idx = lane % LPK;
  const int e0 = part_idx * EPL;
  const int t0 = split * chunk;
  // Keys [t0, tcap) exist in memory; the first sweep's K/V loads are issued
  // from that range before the key count is known, so they do not wait for
  // the count to arrive.
  const int tcap = min(Lk, t0 + chunk);
  const TK* kb = k + (int64_t)b * kv_bs + (int64_t)hkv * kv_hs;
  const TV* vb = v + (int64_t)b * kv_bs + (int64_t)hkv * kv_hs;
  // Keys t == sub (mod KPW) of each wave's sweeps: a sweep covers J groups
  // of KPW consecutive keys per wave (KPW * D * sizeof(TK) contiguous bytes
  // per group), the 4 waves interleave, consecutive sweeps are 4*KPW*J keys
  // apart.  Two register sets alternate so the loads of sweep i+1 are in
  // flight while sweep i is computed.
  using RK = Raw<TK, EPL>;
  using RV = Raw<TV, EPL>;
  RK ka[J], kb2[J];
  RV va[J], vb2[J];
  const int sweep = 4 * KPW * J;
  const int first = t0 + wave * KPW;
  auto fetch = [&](RK* kr, RV* vr, int base, int tl) {
#pragma unroll
    for (int jj = 0; jj < J; ++jj) {
      const int t = max(min(base + jj * 4 * KPW + sub, tl - 1), 0);  // clamped, masked later
      kr[jj].load(kb + (int64_t)t * D + e0);
      vr[jj].load(vb + (int64_t)t * D + e0);
    }
  };
  fetch(ka, va, first, tcap);
  // A graph-replayed decode step reads the current key count from memory
  // (Lk is then the captured capacity); chunks past it publish s = 0.
  if (dlen) Lk = *dlen;

  int kend = Lk;
  if (causal) {
    const int p = qpos ? qpos[b] : Lk - 1;
    kend = min(Lk, p + 1);
  }
  const int t1 = min(kend, t0 + chunk);

  // bf16 q and K: q stays packed and q.k runs on v_dot2_f32_bf16 over the
  // raw K words (no K conversion, half the q registers); otherwise fp32 FMAs.
  constexpr bool kDot2 = sizeof(TQ) == 2 && sizeof(TK) == 2;
  float qv[G][kDot2 ? 1 : EPL];
  uint32_t qw[G][kDot2 ? EPL / 2 : 1];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const TQ* qp = q + ((int64_t)b * Hq + hq0 + g) * D + e0;
    if constexpr (kDot2) {
      Raw<TQ, EPL> r;
      r.load(qp);
#pragma unroll
      for (int w = 0; w < EPL / 2; ++w) qw[g][w] = r.u[w];
    } else {
      load_elems<TQ, EPL>(qp, qv[g]);
    }
  }

  float m[G], s[G], o[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    s[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) o[g][e] = 0.f;
  }

  const float sl2 = scale * kLog2e;
  auto consume = [&](const RK* kr, const RV* vr, int base) {
    float kx[J][kDot2 ? 1 : EPL], vx[J][EPL];
#pragma unroll
    for (int jj = 0; jj < J; ++jj) {
      if constexpr (!kDot2) kr[jj].to_float(kx[jj]);
      vr[jj].to_float(vx[jj]);
      // Keys past the count were fetched speculatively (any bits, NaN
      // included): their weight is 0, and 0 * NaN must not reach o.
      if (base + jj * 4 * KPW + sub >= t1) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) vx[jj][e] = 0.f;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float sc[J];
      float mb = -INFINITY;
#pragma unroll
      for (int jj = 0; jj < J; ++jj) {
        float d = 0.f;
        if constexpr (kDot2) {
#pragma unroll
          for (int w = 0; w < EPL / 2; ++w)
            d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, kr[jj].u[w]),
                                                __builtin_bit_cast(bf16x2_t, qw[g][w]), d, false);
        } else {
#pragma unroll
          for (int e = 0; e < EPL; ++e) d = fmaf(qv[g][e], kx[jj][e], d);
        }
        d = group_sum<LPK>(d);
        sc[jj] = (base + jj * 4 * KPW + sub < t1) ? d * sl2 : -INFINITY;  // log2 domain
        mb = fmaxf(mb, sc[jj]);
      }
      const float mn = fmaxf(m[g], mb);
      // v_exp_f32 directly: exp2(-inf) = 0, results below 2^-126 flush to 0
      if (mn != -INFINITY) {
        const float alpha = __builtin_amdgcn_exp2f(m[g] - mn);
        float ps = 0.f;
        float pj[J];
#pragma unroll
        for (int jj = 0; jj < J; ++jj) { pj[jj] = __builtin_amdgcn_exp2f(sc[jj] - mn); ps += pj[jj]; }
        s[g] = fmaf(s[g], alpha, ps);
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          float acc = o[g][e] * alpha;
#pragma unroll
          for (int jj = 0; jj < J; ++jj) acc = fmaf(pj[jj], vx[jj][e], acc);
          o[g][e] = acc;
        }
        m[g] = mn;
      }
    }
  };
  for (int base = first; base < t1; base += 2 * sweep) {
    if (base + sweep < t1) fetch(kb2, vb2, base + sweep, t1);
    consume(ka, va, base);
    if (base + sweep >= t1) break;
    if (base + 2 * sweep < t1) fetch(ka, va, base + 2 * sweep, t1);
    consume(kb2, vb2, base + sweep);
  }

  // ---- merge the 4*KPW streams of the workgroup in LDS: every stream
  // (wave, sub) publishes its (m, s, o[D]) per head, then all threads
  // combine them, GB heads per round.
  constexpr int NS = 4 * KPW;
  constexpr int GB = G <= 4 ? G : (G % 4 == 0 ? 4 : G / 2);  // heads per LDS round
  static_assert(G % GB == 0, "head rounds must tile the group");
  __shared__ float2 sm_ms[NS][GB];  // (m, s) per stream and head
  __shared__ float sm_o[NS][GB][D];
  const int stream = wave * KPW + sub;
#pragma unroll
  for (int g0 = 0; g0 < G; g0 += GB) {
#pragma unroll
    for (int gl = 0; gl < GB; ++gl) {
      const int g = g0 + gl;
#pragma unroll
      for (int e = 0; e < EPL; ++e) sm_o[stream][gl][e0 + e] = o[g][e];
      if (part_idx == 0) sm_ms[stream][gl] = make_float2(m[g], s[g]);
    }
    __syncthreads();
    // All LDS reads of a thread are issued before any is used (one LDS
    // latency, not one per stream); streams that saw no key have s = 0.
    for (int idx = threadIdx.x; idx < GB * D; idx += 256) {
      const int gl = idx / D, d = idx - gl * D;
      float2 ms[NS];
      float ov[NS];
#pragma unroll
      for (int w = 0; w < NS; ++w) {
        ms[w] = sm_ms[w][gl];
        ov[w] = sm_o[w][gl][d];
      }
      float mx = -INFINITY;
#pragma unroll
      for (int w = 0; w < NS; ++w) mx = fmaxf(mx, ms[w].y > 0.f ? ms[w].x : -INFINITY);
      float ss = 0.f, oo = 0.f;
#pragma unroll
      for (int w = 0; w < NS; ++w) {
        const float f = ms[w].y > 0.f ? __builtin_amdgcn_exp2f(ms[w].x - mx) : 0.f;
        ss = fmaf(ms[w].y, f, ss);
        oo = fmaf(ov[w], f, oo);
      }
      const int hq = hq0 + g0 + gl;
      if (nsplit == 1) {
        Elem<TQ>::store(out, ((int64_t)b * Hq + hq) * D + d, oo / fmaxf(ss, eps));
      } else {
        float* pp = part + ((int64_t)b * Hq + hq) * part_stride(nsplit, D);
        pp[split * D + d] = oo;
        if (d == 0)
          *reinterpret_cast<float2*>(pp + nsplit * D + 2 * split) = make_float2(mx, ss);
      }
    }
    if (g0 + GB < G) __syncthreads();
  }
}

// grid (B*Hq), block 256: combine the nsplit partials of one (b, hq), 64
// splits per round.  Lane l of every wave reads (m, s) of split base + l (the
// max and the sum are wave reductions); thread t reads head-dim entries
// 4*(t%32)..+4 of the splits base + t/32 + 8r, r < 8, and takes their
// weights from the owning lanes with a shuffle.  All loads of a round are
// issued before any is used.  D <= 128.
template <typename TQ>
__global__ __launch_bounds__(256) void attn_decode_merge(const float* __restrict__ part,
                                                         int nsplit, int D, float eps,
                                                         TQ* __restrict__ out) {
  __shared__ float4 red[4][32];
  const int bh = blockIdx.x;
  const float* pp = part + (int64_t)bh * part_stride(nsplit, D);
  const float2* ms = reinterpret_cast<const float2*>(pp + (int64_t)nsplit * D);
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int c4 = t & 31, ig = t >> 5;
  const int col = 4 * c4 < D ? 4 * c4 : 0;
  float mx = -INFINITY, ss = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int base = 0; base < nsplit; base += 64) {
    // indices clamped, values masked afterwards: no load behind a branch
    float2 my = ms[min(base + lane, nsplit - 1)];
    if (base + lane >= nsplit) my.y = 0.f;
    float4 ov[8];
#pragma unroll
    for (int r = 0; r < 8; ++r)
      ov[r] = *reinterpret_cast<const float4*>(pp + (int64_t)min(base + ig + 8 * r, nsplit - 1) * D + col);
    // keep every load of the round ahead of the first use (one round trip)
    asm volatile("" : "+v"(my.x), "+v"(my.y));
#pragma unroll
    for (int r = 0; r < 8; ++r) asm volatile("" : "+v"(ov[r].x), "+v"(ov[r].y), "+v"(ov[r].z), "+v"(ov[r].w));
    // Branch-free (a branch here lets the compiler sink the o loads past
    // it): with no key seen yet mb stays -inf and every weight below is 0.
    const float mb = fmaxf(mx, wave_max(my.y > 0.f ? my.x : -INFINITY));
    const float mref = mb == -INFINITY ? 0.f : mb;
    const float alpha = mx == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mx - mref);
    const float w = my.y > 0.f ? __builtin_amdgcn_exp2f(my.x - mref) : 0.f;  // 0 for splits past nsplit
    ss = fmaf(ss, alpha, wave_sum(my.y * w));
    acc.x *= alpha; acc.y *= alpha; acc.z *= alpha; acc.w *= alpha;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const float wr = __shfl(w, ig + 8 * r, 64);
      acc.x = fmaf(ov[r].x, wr, acc.x);
      acc.y = fmaf(ov[r].y, wr, acc.y);
      acc.z = fmaf(ov[r].z, wr, acc.z);
      acc.w = fmaf(ov[r].w, wr, acc.w);
    }
    mx = mb;
  }
  // lanes t and t+32 of a wave hold the same columns
  acc.x = xor_sum<32>(acc.x);
  acc.y = xor_sum<32>(acc.y);
  acc.z = xor_sum<32>(acc.z);
  acc.w = xor_sum<32>(acc.w);
  if (lane < 32) red[wave][c4] = acc;
  __syncthreads();
  if (t < 32 && 4 * c4 < D) {
    const float inv = 1.f / fmaxf(ss, eps);
    const float4 a0 = red[0][c4], a1 = red[1][c4], a2 = red[2][c4], a3 = red[3][c4];
    const int64_t o0 = (int64_t)bh * D + 4 * c4;
    Elem<TQ>::store(out, o0 + 0, ((a0.x + a1.x) + (a2.x + a3.x)) * inv);
    Elem<TQ>::store(out, o0 + 1, ((a0.y + a1.y) + (a2.y + a3.y)) * inv);
    Elem<TQ>::store(out, o0 + 2, ((a0.z + a1.z) + (a2.z + a3.z)) * inv);
    Elem<TQ>::store(out, o0 + 3, ((a0.w + a1.w) + (a2.w + a3.w)) * inv);
  }
}

// grid (B*Hq), one wave: the same combination for D in {64, 128} and at
// most NS splits.  Lane l holds split l's (m, s) and its weight; it reads
// head-dim entries C*l .. C*l+C-1 of every split (all loads issued first)
// and takes each split's weight by a constant-lane read.  No LDS, no barrier.
template <typename TQ, int D, int NS>
__global__ __launch_bounds__(64) void attn_decode_merge_w(const float* __restrict__ part,
                                                          int nsplit, float eps,
                                                          TQ* __restrict__ out) {
  constexpr int C = D / 64;
  const int bh = blockIdx.x, lane = threadIdx.x;
  const float* pp = part + (int64_t)bh * part_stride(nsplit, D);
  const float2* ms = reinterpret_cast<const float2*>(pp + (int64_t)nsplit * D);
  float2 my = ms[min(lane, nsplit - 1)];
  float ov[NS][C];
#pragma unroll
  for (int sp = 0; sp < NS; ++sp) {
    const float* row = pp + (int64_t)min(sp, nsplit - 1) * D + C * lane;
    if constexpr (C == 2) {
      const float2 t = *reinterpret_cast<const float2*>(row);
      ov[sp][0] = t.x;
      ov[sp][1] = t.y;
    } else {
      ov[sp][0] = *row;
    }
  }
  if (lane >= nsplit) my.y = 0.f;
  const float mb = wave_max(my.y > 0.f ? my.x : -INFINITY);
  const float mref = mb == -INFINITY ? 0.f : mb;
  const float w = my.y > 0.f ? __builtin_amdgcn_exp2f(my.x - mref) : 0.f;  // 0 past nsplit
  const float ss = wave_sum(my.y * w);
  float acc[C] = {};
#pragma unroll
  for (int sp = 0; sp < NS; ++sp) {
    const float ws = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), sp));
#pragma unroll
    for (int c = 0; c < C; ++c) acc[c] = fmaf(ov[sp][c], ws, acc[c]);
  }
  const float inv = 1.f / fmaxf(ss, eps);
#pragma unroll
  for (int c = 0; c < C; ++c) Elem<TQ>::store(out, (int64_t)bh * D + C * lane + c, acc[c] * inv);
}

// The merge launch for nsplit > 1 partials of B*Hq rows.
template <typename TQ>
void launch_decode_merge(const float* part, int nsplit, int D, int rows, float eps, TQ* out,
                         hipStream_t st) {
#define STRATA_MW(DD, NN)                                                                    \
  hipLaunchKernelGGL((attn_decode_merge_w<TQ, DD, NN>), dim3(rows), dim3(64), 0, st, part,  \
                     nsplit, eps, out)
  // (NS in steps of 8 up to 48: the loads past nsplit repeat the last split)
#define STRATA_MWD(DD)                                                  \
  if (nsplit <= 16) STRATA_MW(DD, 16);                                  \
  else if (nsplit <= 24) STRATA_MW(DD, 24);                             \
  else if (nsplit <= 32) STRATA_MW(DD, 32);                             \
  else if (nsplit <= 40) STRATA_MW(DD, 40);                             \
  else if (nsplit <= 48) STRATA_MW(DD, 48);                             \
  else STRATA_MW(DD, 64);
  if ((D == 64 || D == 128) && nsplit <= 64) {
    if (D == 128) {
      STRATA_MWD(128)
    } else {
      STRATA_MWD(64)
    }
  } else {
    hipLaunchKernelGGL((attn_decode_merge<TQ>), dim3(rows), dim3(256), 0, st, part, nsplit, D,
                       eps, out);
  }
#undef STRATA_MWD
#undef STRATA_MW
}

// ----------------------------------------------------------- prefill on MFMA
// Workgroup wg of the prefill grid -> (query tile, b, kv head, query head).
// remap: workgroups are dealt to the 8 XCDs round-robin (wg % 8); a group
// gi of the G query heads of one (query tile, b, kv head) goes to XCD
// gi % 8 in G consecutive slots of that XCD, groups ordered longest causal
// query tile first (measured 1.5x on the bf16 two-block kernel at 8k
// causal).  Otherwise the order is query tile fastest, then head, then
// batch.  Returns false for the padding of the last round.
constexpr int kXcds = 8;
__host__ __device__ inline int prefill_grid(int nqt, int B, int Hkv, int G) {
  const int groups = nqt * B * Hkv;
  return (groups + kXcds - 1) / kXcds * kXcds * G;
}
__device__ inline bool prefill_item(bool remap, int wg, int nqt, int B, int Hkv, int G, int* qt,
                                    int* b, int* hkv, int* hq) {
  if (!remap) {
    if (wg >= nqt * B * Hkv * G) return false;
    *qt = wg % nqt;
    *hq = (wg / nqt) % (Hkv * G);
    *b = wg / (nqt * Hkv * G);
    *hkv = *hq / G;
    return true;
  }
  const int xcd = wg % kXcds, slot = wg / kXcds;
  const int g = slot % G, gi = (slot / G) * kXcds + xcd;
  if (gi >= nqt * B * Hkv) return false;
  const int per_tile = B * Hkv;
  *qt = nqt - 1 - gi / per_tile;
  const int rest = gi % per_tile;
  *b = rest / Hkv;
  *hkv = rest % Hkv;
  *hq = *hkv * G + g;
  return true;
}
__device__ __forceinline__ f32x4_t mfma_f32(float a, float b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Two floats -> packed bf16 pair, round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// fp32 prefill.  1-D grid, block 256; workgroup -> (query tile qt, b, hq)
// in plain order (prefill_item without the remap); wave w owns the 16 query
// rows qt*64 + 16w + 0..15.  S^T = K Q^T and O^T += V P^T on 16x16x4 fp32
// MFMAs; one LDS stage of K and V tiles (64 keys, row-major, padded rows).
// MFMA 16x16x4 layouts (wave64): A (16 x 4): lane l holds row l%16, k l/16;
// B (4 x 16): lane l holds column l%16, k l/16; C (16 x 16): lane l holds
// column l%16, rows 4(l/16) + 0..3.
template <int D>
__global__ __launch_bounds__(256) void attn_prefill_f32(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    int64_t kv_bs, int64_t kv_hs, const int32_t* __restrict__ qpos, int B, int Hq, int Hkv,
    int Lq, int Lk, int causal, float scale, float eps, int out_tm, float* __restrict__ out) {
  constexpr int KT = 64;                 // keys per tile
  constexpr int PAD = 4;                 // LDS row padding (elements)
  constexpr int RS = D + PAD;            // LDS row stride
  __shared__ __attribute__((aligned(16))) float ks[KT * RS];
  __shared__ __attribute__((aligned(16))) float vs[KT * RS];
  __shared__ int s_kmax;

  const int G = Hq / Hkv;
  int qt, b, hkv, hq;
  if (!prefill_item(false, blockIdx.x, (Lq + 63) / 64, B, Hkv, G, &qt, &b, &hkv, &hq))
    return;  // grid padding
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int row = qt * 64 + 16 * wave + col;  // this lane's query row
  const bool row_ok = row < Lq;
  const int qp = row_ok ? (causal ? (qpos ? qpos[(int64_t)b * Lq + row] : Lk - Lq + row) : Lk - 1)
                        : -1;
  // keys every row of the wave sees (no mask below) and keys any row needs
  int kfull = row_ok ? (causal ? qp + 1 : Lk) : 0;
  int wave_need = qp + 1;
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) {
    kfull = min(kfull, __shfl_xor(kfull, off, 64));
    wave_need = max(wave_need, __shfl_xor(wave_need, off, 64));
  }
  if (threadIdx.x == 0) s_kmax = 0;
  __syncthreads();
  if (lane == 0) atomicMax(&s_kmax, wave_need);
  __syncthreads();
  const int kmax = causal ? min(Lk, s_kmax) : Lk;

  const float* kbase = k + (int64_t)b * kv_bs + (int64_t)hkv * kv_hs;
  const float* vbase = v + (int64_t)b * kv_bs + (int64_t)hkv * kv_hs;
  // Q fragments as the B operand of S^T: column = query row, k = head dim 4s + grp.
  constexpr int QF = D / 4;
  float qf[QF];
  {
    const float* qrow = q + (((int64_t)b * Hq + hq) * Lq + (row_ok ? row : 0)) * D;
#pragma unroll
    for (int s = 0; s < QF; ++s) qf[s] = row_ok ? qrow[4 * s + grp] : 0.f;
  }
  constexpr int DT = D / 16;  // output d tiles
  f32x4_t acc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  const float sl2 = scale * kLog2e;

  // Tiles: 16-byte chunks, chunk c of the tile -> (key t, element d0); keys
  // past Lk read key Lk - 1 (finite; their scores are masked, their
  // weights 0).  Tile t+1's loads are issued before tile t's math.
  constexpr int NCH = KT * D / 4 / 256;  // chunks per thread per tile
  static_assert(KT * D / 4 % 256 == 0, "tile chunks must divide over the block");
  uint4 kreg[NCH], vreg[NCH];
  auto fetch = [&](int kb) {
#pragma unroll
    for (int u = 0; u < NCH; ++u) {
      const int c = threadIdx.x + 256 * u;
      const int t = c / (D / 4), d0 = 4 * (c % (D / 4));
      const int key = min(kb + t, Lk - 1);
      kreg[u] = *reinterpret_cast<const uint4*>(kbase + (int64_t)key * D + d0);
      vreg[u] = *reinterpret_cast<const uint4*>(vbase + (int64_t)key * D + d0);
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int u = 0; u < NCH; ++u) {
      const int c = threadIdx.x + 256 * u;
      const int t = c / (D / 4), d0 = 4 * (c % (D / 4));
      *reinterpret_cast<uint4*>(&ks[t * RS + d0]) = kreg[u];
      *reinterpret_cast<uint4*>(&vs[t * RS + d0]) = vreg[u];
    }
  };
  if (kmax > 0) {
    fetch(0);
    stage();
  }
  __syncthreads();
  for (int kb0 = 0; kb0 < kmax; kb0 += KT) {
    const bool more = kb0 + KT < kmax;
    if (more) fetch(kb0 + KT);
    if (__builtin_amdgcn_readfirstlane((int)(kb0 < wave_need))) {
      // st[j][i] = score(this lane's row, key kb0 + 16j + 4 grp + i)
      f32x4_t st[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        st[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < QF; ++s)
          st[j] = mfma_f32(ks[(16 * j + col) * RS + 4 * s + grp], qf[s], st[j]);
      }
      if (kb0 + KT > kfull) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = kb0 + 16 * j + 4 * grp + i;
            const bool ok = key < Lk && (!causal || key <= qp) && row_ok;
            st[j][i] = ok ? st[j][i] : -INFINITY;
          }
      }
      // online softmax (log2 domain, raw scores kept, sl2 > 0)
      float mb = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) mb = fmaxf(mb, st[j][i]);
      mb = xor_max<16>(mb);
      mb = xor_max<32>(mb);
      const float mn = fmaxf(m_run, mb * sl2);
      const bool none = mn == -INFINITY;  // no visible key yet: weights 0, alpha 1
      const float alpha = none ? 1.f : __builtin_amdgcn_exp2f(m_run - mn);
      const float nmn = none ? 0.f : -mn;
      float ps = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = __builtin_amdgcn_exp2f(fmaf(st[j][i], sl2, nmn));
          st[j][i] = p;
          ps += p;
        }
      l_run = fmaf(l_run, alpha, ps);
      m_run = mn;
      if (__any(alpha != 1.f)) {
#pragma unroll
        for (int i = 0; i < DT; ++i) acc[i] *= alpha;
      }
      // O^T += V^T P^T, one key per MFMA k-slot
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = 16 * j + 4 * grp + i;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt)
            acc[dt] = mfma_f32(vs[key * RS + dt * 16 + col], st[j][i], acc[dt]);
        }
    }
    __syncthreads();  // every wave is done with the tile
    if (more) {
      stage();
      __syncthreads();
    }
  }

  float l_tot = l_run;
  l_tot = xor_sum<16>(l_tot);
  l_tot = xor_sum<32>(l_tot);
  if (row_ok) {
    const float inv = 1.f / fmaxf(l_tot, eps);
    // out_tm: token-major [B, Lq, Hq, D] (the o_proj input); else [B, Hq, Lq, D]
    float* orow = out + (out_tm ? (((int64_t)b * Lq + row) * Hq + hq) * D
                                : (((int64_t)b * Hq + hq) * Lq + row) * D);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) orow[dt * 16 + 4 * grp + i] = acc[dt][i] * inv;
  }
}

// ------------------------------------------------- bf16 prefill, 32x32 tiles
typedef float f32x16_t __attribute__((ext_vector_type(16)));
__device__ __forceinline__ f32x16_t mfma32_bf16(const bf16x8_t& a, const bf16x8_t& b,
                                                f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// bf16 prefill on 32x32x16 MFMA tiles.  Workgroup = NW waves = 32 NW query
// rows of one (b, query head) (grid order as prefill_item); wave w owns rows
// qt*32NW + 32w + 0..31.  S^T = K Q^T and O^T += V^T P^T run as 32x32x16
// MFMAs whose 32-cycle issue leaves room for other waves' softmax on the
// SIMD; the P^T operand is the S^T accumulator itself (no shuffles).
// K and V tiles (KT keys) are streamed by direct global -> LDS loads into a
// ring of NST stages, row-major with XOR-swizzled 16-byte chunks: the loads
// of tile t + NST - 1 are issued at the top of tile t, and no register holds
// them.  V^T operands come from row-major V through the LDS transpose read
// (ds_read_b64_tr_b16: in each 16-lane group, lane l' receives element
// (l' & 3) of the 4-element rows addressed by lanes 4k + (l' >> 2), k < 4).
// MFMA 32x32x16 layouts (wave64): A (32 x 16): lane l holds row l%32, k
// 8(l/32) .. +8; B (16 x 32): lane l holds column l%32, the same k; C (32 x
// 32): lane l holds column l%32, rows 8(i/4) + 4(l/32) + i%4 for i < 16.
typedef short v4i16_t __attribute__((ext_vector_type(4)));
constexpr float kRescaleSlack = 8.f;
template <int D, int NW, int NST, int KT>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(KT == 32 ? 3 : 2)))
void attn_prefill_mfma32(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    int64_t kv_bs, int64_t kv_hs, const int32_t* __restrict__ qpos, int B, int Hq, int Hkv,
    int Lq, int Lk, int causal, float scale, float eps, int out_tm, bf16_t* __restrict__ out) {
  constexpr int KB = KT / 32;         // 32-key score blocks per tile
  constexpr int ROW = D * 2;          // bytes per K / V row
  constexpr int NCHK = D / 8;         // 16-byte chunks per row
  constexpr int TILE = KT * ROW;      // bytes of one K or V tile
  constexpr int STAGE = 2 * TILE;     // K tile, then V tile
  constexpr int AHEAD = NST - 1;      // tiles in flight ahead of the one computed
  constexpr int QR = 32 * NW;         // query rows per workgroup
  constexpr int NI = KT * NCHK / (64 * NW);  // 16-byte loads per thread per tile and operand
  static_assert(NI >= 1 && KT * NCHK % (64 * NW) == 0, "tile loads must divide over the workgroup");
  __shared__ __attribute__((aligned(16))) uint8_t lds[NST * STAGE];
  __shared__ int s_kmax;

  const int G = Hq / Hkv;
  int qt, b, hkv, hq;
  if (!prefill_item(true, blockIdx.x, (Lq + QR - 1) / QR, B, Hkv, G, &qt, &b, &hkv, &hq))
    return;  // grid padding
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c32 = lane & 31, h = lane >> 5;
  const int row = qt * QR + 32 * wave + c32;  // this lane's query row
  const bool row_ok = row < Lq;
  const int qp = row_ok ? (causal ? (qpos ? qpos[(int64_t)b * Lq + row] : Lk - Lq + row) : Lk - 1)
                        : -1;
  // Keys every row of the wave sees (tiles below need no mask) and keys any
  // row of it needs (tiles from there on are skipped); lanes l and l + 32
  // hold the same row.
  int kfull = row_ok ? (causal ? qp + 1 : Lk) : 0;
  int wave_need = qp + 1;
#pragma unroll
  for (int off = 1; off < 32; off <<= 1) {
    kfull = min(kfull, __shfl_xor(kfull, off, 64));
    wave_need = max(wave_need, __shfl_xor(wave_need, off, 64));
  }
  if (threadIdx.x == 0) s_kmax = 0;
  __syncthreads();
  if (lane == 0) atomicMax(&s_kmax, wave_need);
  __syncthreads();
  const int kmax = causal ? min(Lk, s_kmax) : Lk;

  // Buffer descriptors of this head's K and V rows: keys at or past Lk
  // read as zero.
  const v4i32_t rk = rsrc(k + (int64_t)b * kv_bs + (int64_t)hkv * kv_hs, (uint32_t)Lk * ROW);
  const v4i32_t rv = rsrc(v + (int64_t)b * kv_bs + (int64_t)hkv * kv_hs, (uint32_t)Lk * ROW);
  const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) uint8_t*)lds);
  // Chunk swizzles.  K: the 16 lanes reading one 16-byte column of 16 rows
  // meet 16 distinct chunk slots per 256 bytes of rows.  V: a transpose
  // read's half-wave (4 rows, two 32-byte column pairs per row) meets 8
  // distinct pairs per 256 bytes of rows.
  auto fk = [](int key) { return (key / (256 / ROW)) & (NCHK - 1); };
  auto fv = [](int key) { return (key * (NCHK / 4)) & (NCHK - 1); };
  // Load i of this thread fills 16-byte slot (wave * NI + i) * 64 + lane of
  // a tile: key slot / NCHK, chunk slot % NCHK holding source chunk
  // (slot % NCHK) ^ swizzle(key).
  uint32_t kvo[NI], vvo[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int slot = (wave * NI + i) * 64 + lane;
    const int key = slot / NCHK, cp = slot % NCHK;
    kvo[i] = key * ROW + 16 * (cp ^ fk(key));
    vvo[i] = key * ROW + 16 * (cp ^ fv(key));
  }
  auto issue = [&](int kb, int st) {
    const uint32_t base = lds0 + st * STAGE;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      dma16(base + (wave * NI + i) * 1024, kvo[i], rk, (uint32_t)kb * ROW);
      dma16(base + TILE + (wave * NI + i) * 1024, vvo[i], rv, (uint32_t)kb * ROW);
    }
  };

  // Q^T fragments (the B operand of S^T): column = this lane's row, k = the
  // head dims 16 s + 8 h .. +8.
  constexpr int QS = D / 16;
  bf16x8_t qf[QS];
  {
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(q) +
                           (((int64_t)b * Hq + hq) * Lq + (row_ok ? row : 0)) * D;
#pragma unroll
    for (int s = 0; s < QS; ++s) {
      uint4 u = make_uint4(0, 0, 0, 0);
      if (row_ok) u = *reinterpret_cast<const uint4*>(qrow + s * 16 + 8 * h);
      qf[s] = __builtin_bit_cast(bf16x8_t, u);
    }
  }
  constexpr int DB = D / 32;  // 32-row head-dim blocks of O^T
  f32x16_t acc[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const float sl2 = scale * kLog2e;

  // This lane's LDS byte offsets inside a stage, fixed for the kernel: the
  // swizzles depend only on the lane's part of the row index (32 kb and
  // 16 s4 + 8 j leave fk and fv unchanged), so the per-tile and per-step
  // parts are immediate offsets.
  // K operand of S^T block kb, step s: row 32 kb + c32, chunk 2s + h.
  int k_off[QS];
#pragma unroll
  for (int s = 0; s < QS; ++s) k_off[s] = c32 * ROW + 16 * ((2 * s + h) ^ fk(c32));
  // V^T operand (transpose read) of 16-key step s4, half j (keys 16 s4 + 8j
  // + 4h + 0..3) and head-dim block db: this lane addresses key
  // 16 s4 + 8j + 4h + (l' >> 2), head dims 32 db + 16 (g & 1) + 4 (l' & 3)
  // .. +3, g = lane / 16, l' = lane % 16.
  const int lp = lane & 15, g = lane >> 4;
  const int v_key = 4 * h + (lp >> 2);            // plus 16 s4 + 8 j
  const int v_col = 16 * (g & 1) + 4 * (lp & 3);  // plus 32 db (elements)
  int v_off[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    const int col = 32 * db + v_col;
    v_off[db] = TILE + v_key * ROW + 16 * ((col / 8) ^ fv(v_key)) + 2 * (col % 8);
  }
  static_assert(NST == 2 || NST == 3, "the tile loop cycles two or three stages");

  // Wait until at most n tiles' loads (2 NI each) of this thread are in flight.
  auto wait_tiles = [&](int n) {
    if (n <= 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else if (n == 1) asm volatile("s_waitcnt vmcnt(%0)" :: "n"(2 * NI) : "memory");
    else if (n == 2) asm volatile("s_waitcnt vmcnt(%0)" :: "n"(4 * NI) : "memory");
    else asm volatile("s_waitcnt vmcnt(%0)" :: "n"(6 * NI) : "memory");
  };
  static_assert(AHEAD <= 3, "wait_tiles covers up to three tiles in flight");
  const int nt = (kmax + KT - 1) / KT;
  // prologue: tiles 0 .. AHEAD - 1 in flight, tile 0 complete
  for (int t = 0; t < AHEAD && t < nt; ++t) issue(t * KT, t);
  wait_tiles(min(nt, AHEAD) - 1);
  __syncthreads();
  // one tile on stage ST (a compile-time constant, so every LDS address is a
  // lane offset plus an immediate)
  auto tile = [&](int t, auto STC) {
    constexpr int ST = decltype(STC)::value;
    const int kb0 = t * KT;
    if (t + AHEAD < nt) issue((t + AHEAD) * KT, (ST + AHEAD) % NST);  // the stage tile t - 1 used
    const uint8_t* ks = lds + ST * STAGE;
    // Waves whose rows see no key of the tile skip its math (one scalar
    // branch); rows of a live wave that see none are masked to p = 0.
    if (__builtin_amdgcn_readfirstlane((int)(kb0 < wave_need))) {
      __builtin_amdgcn_s_setprio(1);
      // st[kb][i] = score(this lane's row, key kb0 + 32 kb + 8(i/4) + 4h + i%4)
      f32x16_t sc[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[kb][r] = 0.f;
#pragma unroll
      for (int s = 0; s < QS; ++s)
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          const uint4 a = *reinterpret_cast<const uint4*>(ks + k_off[s] + 32 * kb * ROW);
          sc[kb] = mfma32_bf16(__builtin_bit_cast(bf16x8_t, a), qf[s], sc[kb]);
        }
      __builtin_amdgcn_s_setprio(0);
      // online softmax in the log2 domain (raw scores kept; the scale is
      // folded into the exponent's FMA, sl2 > 0)
      if (kb0 + KT > kfull) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = kb0 + 32 * kb + 8 * (i / 4) + 4 * h + i % 4;
            const bool ok = key < Lk && (!causal || key <= qp) && row_ok;
            sc[kb][i] = ok ? sc[kb][i] : -INFINITY;
          }
      }
      float mb = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) mb = fmaxf(mb, sc[kb][i]);
      mb = xor_max<32>(mb);
      // The reference maximum moves only when the tile's maximum exceeds it
      // by more than kRescaleSlack (log2 units): the exponentials stay below
      // 2^kRescaleSlack (exact in fp32, bf16's relative precision when
      // packed), o / l is unchanged, and O is rescaled far less often
      // (8k causal: 612-619 -> 579-585 us).
      const float mt = mb * sl2;
      const float mn = mt > m_run + kRescaleSlack ? mt : m_run;
      // rows with no visible key yet keep mn = -inf (weights 0, alpha 1)
      const bool none = mn == -INFINITY;
      const float alpha = none ? 1.f : __builtin_amdgcn_exp2f(m_run - mn);
      const float nmn = none ? 0.f : -mn;
      float ps = 0.f;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float p = __builtin_amdgcn_exp2f(fmaf(sc[kb][i], sl2, nmn));  // exp2(-inf) = 0
          sc[kb][i] = p;
          ps += p;
        }
      l_run = fmaf(l_run, alpha, ps);
      m_run = mn;
      if (__any(alpha != 1.f)) {
#pragma unroll
        for (int i = 0; i < DB; ++i) acc[i] *= alpha;
      }
      __builtin_amdgcn_s_setprio(1);
      // O^T += V^T P^T over 16-key steps: the P^T operand of step s4 (keys
      // 16 s4 .. +16) is sc[s4 / 2][8 (s4 % 2) .. +8]: lane half h holds keys
      // 16 s4 + 4h + 0..3 and 16 s4 + 8 + 4h + 0..3, and the V^T operand
      // takes the same keys for its head dim.
#pragma unroll
      for (int s4 = 0; s4 < KT / 16; ++s4) {
        const int kb = s4 / 2, i0 = 8 * (s4 % 2);
        uint4 pu;
        pu.x = pack_bf16x2(sc[kb][i0 + 0], sc[kb][i0 + 1]);
        pu.y = pack_bf16x2(sc[kb][i0 + 2], sc[kb][i0 + 3]);
        pu.z = pack_bf16x2(sc[kb][i0 + 4], sc[kb][i0 + 5]);
        pu.w = pack_bf16x2(sc[kb][i0 + 6], sc[kb][i0 + 7]);
        const bf16x8_t pb = __builtin_bit_cast(bf16x8_t, pu);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          v4i16_t vv[2];
#pragma unroll
          for (int j = 0; j < 2; ++j)
            vv[j] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) v4i16_t*)(lds0 + ST * STAGE + v_off[db] +
                                                               (16 * s4 + 8 * j) * ROW));
          uint4 au;
          au.x = (uint16_t)vv[0][0] | ((uint32_t)(uint16_t)vv[0][1] << 16);
          au.y = (uint16_t)vv[0][2] | ((uint32_t)(uint16_t)vv[0][3] << 16);
          au.z = (uint16_t)vv[1][0] | ((uint32_t)(uint16_t)vv[1][1] << 16);
          au.w = (uint16_t)vv[1][2] | ((uint32_t)(uint16_t)vv[1][3] << 16);
          acc[db] = mfma32_bf16(__builtin_bit_cast(bf16x8_t, au), pb, acc[db]);
        }
      }
      __builtin_amdgcn_s_setprio(0);
    }
    // tile t + 1 complete in this thread (later tiles' loads may remain in
    // flight), then in every thread
    wait_tiles(min(nt - 1, t + AHEAD) - (t + 1));
    __syncthreads();
  };
  for (int t = 0; t < nt; t += NST) {
    tile(t, std::integral_constant<int, 0>{});
    if (t + 1 >= nt) break;
    tile(t + 1, std::integral_constant<int, 1>{});
    if constexpr (NST == 3) {
      if (t + 2 >= nt) break;
      tile(t + 2, std::integral_constant<int, 2 % NST>{});
    }
  }

  const float l_tot = xor_sum<32>(l_run);
  if (row_ok) {
    const float inv = 1.f / fmaxf(l_tot, eps);
    // out_tm: token-major [B, Lq, Hq, D] (the o_proj input); else [B, Hq, Lq, D]
    uint16_t* orow = reinterpret_cast<uint16_t*>(out) +
                     (out_tm ? (((int64_t)b * Lq + row) * Hq + hq) * D
                             : (((int64_t)b * Hq + hq) * Lq + row) * D);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const uint2 o2 = make_uint2(pack_bf16x2(acc[db][4 * g4] * inv, acc[db][4 * g4 + 1] * inv),
                                    pack_bf16x2(acc[db][4 * g4 + 2] * inv, acc[db][4 * g4 + 3] * inv));
        *reinterpret_cast<uint2*>(orow + 32 * db + 8 * g4 + 4 * h) = o2;
      }
  }
}

// ---------------------------------------------------- batched decode on MFMA
// One wave per (b, KV head, key chunk).  The G query heads of the KV head are
// the columns of S^T = K Q^T on 32x32x16 MFMAs (columns past G hold zero q and
// are ignored), so the online softmax is in-lane per head exactly as in the
// prefill kernel; O^T += V^T P^T takes P^T straight from the S^T accumulator
// and V^T through the LDS transpose read.  K and V tiles of 32 keys stream
// through a ring of NST stages private to the wave (direct global -> LDS
// loads, no barrier).  Partials (m, s, o[D]) per head go to `part` for
// attn_decode_merge, or the output is finalised when there is one chunk.
// The arguments the first K/V loads need lead the list (16 preloaded dwords).
template <int D, int NST, int WPG>
__global__ __launch_bounds__(64 * WPG) void attn_decode_mfma(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    int64_t kv_bs, int64_t kv_hs, int B, int Hq, int Hkv, int Lk, int chunk, int nsplit,
    const int32_t* __restrict__ qpos, const int* __restrict__ dlen, int causal, float scale,
    float eps, float* __restrict__ part, bf16_t* __restrict__ out) {
  constexpr int KT = 32;
  constexpr int ROW = D * 2;
  constexpr int NCHK = D / 8;
  constexpr int TILE = KT * ROW;
  constexpr int STAGE = 2 * TILE;
  constexpr int AHEAD = NST - 1;
  constexpr int NI = KT * NCHK / 64;   // 16-byte loads per lane per tile and operand
  constexpr int QS = D / 16;
  constexpr int DB = D / 32;
  static_assert(NST == 2 || NST == 3, "two or three stages");
  __shared__ __attribute__((aligned(16))) uint8_t lds_all[WPG * NST * STAGE];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int item = blockIdx.x * WPG + wave;
  if (item >= B * Hkv * nsplit) return;  // wave-uniform; the kernel has no barrier
  const int split = item % nsplit, bh = item / nsplit;
  const int hkv = bh % Hkv, b = bh / Hkv;
  const int G = Hq / Hkv;
  const int c32 = lane & 31, h = lane >> 5;
  const bool head_ok = c32 < G;
  const int hq = hkv * G + (head_ok ? c32 : 0);
  const int t0 = split * chunk;
  const int tcap = min(Lk, t0 + chunk);  // keys in memory (the capacity in graph mode)
  const bf16_t* kb = k + (int64_t)b * kv_bs + (int64_t)hkv * kv_hs;
  const bf16_t* vb = v + (int64_t)b * kv_bs + (int64_t)hkv * kv_hs;
  const v4i32_t rk = rsrc(kb, (uint32_t)max(tcap, 0) * ROW);
  const v4i32_t rv = rsrc(vb, (uint32_t)max(tcap, 0) * ROW);
  uint8_t* lds = lds_all + wave * NST * STAGE;
  const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) uint8_t*)lds);
  auto fk = [](int key) { return (key / (256 / ROW)) & (NCHK - 1); };
  auto fv = [](int key) { return (key * (NCHK / 4)) & (NCHK - 1); };
  uint32_t kvo[NI], vvo[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int slot = i * 64 + lane;
    const int key = slot / NCHK, cp = slot % NCHK;
    kvo[i] = key * ROW + 16 * (cp ^ fk(key));
    vvo[i] = key * ROW + 16 * (cp ^ fv(key));
  }
  auto issue = [&](int kb0, int st) {
    const uint32_t base = lds0 + st * STAGE;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      dma16(base + i * 1024, kvo[i], rk, (uint32_t)kb0 * ROW);
      dma16(base + TILE + i * 1024, vvo[i], rv, (uint32_t)kb0 * ROW);
    }
  };
  const int nt = tcap > t0 ? (tcap - t0 + KT - 1) / KT : 0;
  for (int t = 0; t < AHEAD && t < nt; ++t) issue(t0 + t * KT, t);
  // Q^T fragments: column = this lane's head, k = head dims 16 s + 8 h .. +8
  bf16x8_t qf[QS];
  {
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(q) + ((int64_t)b * Hq + hq) * D;
#pragma unroll
    for (int s = 0; s < QS; ++s) {
      uint4 u = *reinterpret_cast<const uint4*>(qrow + s * 16 + 8 * h);
      if (!head_ok) u = make_uint4(0, 0, 0, 0);
      qf[s] = __builtin_bit_cast(bf16x8_t, u);
    }
  }
  // Visible keys: [0, kend), read after the first tiles' loads are issued.
  int cnt = Lk;
  if (dlen) cnt = *dlen;
  int kend = cnt;
  if (causal) {
    const int p = qpos ? qpos[b] : cnt - 1;
    kend = min(cnt, p + 1);
  }
  const int t1 = min(kend, t0 + chunk);
  int k_off[QS];
#pragma unroll
  for (int s = 0; s < QS; ++s) k_off[s] = c32 * ROW + 16 * ((2 * s + h) ^ fk(c32));
  const int lp = lane & 15, gq = lane >> 4;
  const int v_key = 4 * h + (lp >> 2);
  const int v_col = 16 * (gq & 1) + 4 * (lp & 3);
  int v_off[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    const int col = 32 * db + v_col;
    v_off[db] = TILE + v_key * ROW + 16 * ((col / 8) ^ fv(v_key)) + 2 * (col % 8);
  }
  f32x16_t acc[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const float sl2 = scale * kLog2e;
  auto wait_tiles = [&](int n) {
    if (n <= 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else if (n == 1) asm volatile("s_waitcnt vmcnt(%0)" :: "n"(2 * NI) : "memory");
    else asm volatile("s_waitcnt vmcnt(%0)" :: "n"(4 * NI) : "memory");
  };
  // tiles past the visible keys are loaded (issued before the count was
  // known) but not computed
  const int ntv = t1 > t0 ? (t1 - t0 + KT - 1) / KT : 0;
  auto tile = [&](int t, auto STC) {
    constexpr int ST = decltype(STC)::value;
    const int kb0 = t0 + t * KT;
    if (t + AHEAD < nt) issue(kb0 + AHEAD * KT, (ST + AHEAD) % NST);
    wait_tiles(min(nt - 1, t + AHEAD) - t);
    const uint8_t* ks = lds + ST * STAGE;
    if (kb0 + KT > t1) {
      // V rows of keys past the visible ones may hold any bits (unwritten
      // cache slots): zero them, so that p = 0 times them stays 0.
      uint8_t* vt = lds + ST * STAGE + TILE;
      const int r0 = max(t1 - kb0, 0);
      for (int c = lane; c < (KT - r0) * NCHK; c += 64)
        *reinterpret_cast<uint4*>(vt + r0 * ROW + 16 * c) = make_uint4(0, 0, 0, 0);
    }
    __builtin_amdgcn_s_setprio(1);
    f32x16_t sc;
#pragma unroll
    for (int r = 0; r < 16; ++r) sc[r] = 0.f;
#pragma unroll
    for (int s = 0; s < QS; ++s) {
      const uint4 a = *reinterpret_cast<const uint4*>(ks + k_off[s]);
      sc = mfma32_bf16(__builtin_bit_cast(bf16x8_t, a), qf[s], sc);
    }
    __builtin_amdgcn_s_setprio(0);
    if (kb0 + KT > t1) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = kb0 + 8 * (i / 4) + 4 * h + i % 4;
        sc[i] = key < t1 ? sc[i] : -INFINITY;
      }
    }
    float mb = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) mb = fmaxf(mb, sc[i]);
    mb = xor_max<32>(mb);
    const float mt = mb * sl2;
    const float mn = mt > m_run + kRescaleSlack ? mt : m_run;
    const bool none = mn == -INFINITY;
    const float alpha = none ? 1.f : __builtin_amdgcn_exp2f(m_run - mn);
    const float nmn = none ? 0.f : -mn;
    float ps = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float p = __builtin_amdgcn_exp2f(fmaf(sc[i], sl2, nmn));
      sc[i] = p;
      ps += p;
    }
    l_run = fmaf(l_run, alpha, ps);
    m_run = mn;
    if (__any(alpha != 1.f)) {
#pragma unroll
      for (int i = 0; i < DB; ++i) acc[i] *= alpha;
    }
    __builtin_amdgcn_s_setprio(1);
    // P enters the MFMA as bf16 hi + lo parts (p - bf16(p) is exact in fp32),
    // so P V keeps about 16 significant bits of each weight, close to the
    // fp32 weights of attn_decode_kernel, at twice the P V MFMAs (the kernel
    // is bound by the K/V stream, not by the matrix cores).
#pragma unroll
    for (int s4 = 0; s4 < KT / 16; ++s4) {
      const int i0 = 8 * s4;
      uint32_t ph[4], pl[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float p0 = sc[i0 + 2 * c], p1 = sc[i0 + 2 * c + 1];
        ph[c] = pack_bf16x2(p0, p1);
        pl[c] = pack_bf16x2(p0 - __uint_as_float(ph[c] << 16),
                            p1 - __uint_as_float(ph[c] & 0xffff0000u));
      }
      const bf16x8_t pb = __builtin_bit_cast(bf16x8_t, make_uint4(ph[0], ph[1], ph[2], ph[3]));
      const bf16x8_t pbl = __builtin_bit_cast(bf16x8_t, make_uint4(pl[0], pl[1], pl[2], pl[3]));
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        v4i16_t vv[2];
#pragma unroll
        for (int j = 0; j < 2; ++j)
          vv[j] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) v4i16_t*)(lds0 + ST * STAGE + v_off[db] +
                                                             (16 * s4 + 8 * j) * ROW));
        uint4 au;
        au.x = (uint16_t)vv[0][0] | ((uint32_t)(uint16_t)vv[0][1] << 16);
        au.y = (uint16_t)vv[0][2] | ((uint32_t)(uint16_t)vv[0][3] << 16);
        au.z = (uint16_t)vv[1][0] | ((uint32_t)(uint16_t)vv[1][1] << 16);
        au.w = (uint16_t)vv[1][2] | ((uint32_t)(uint16_t)vv[1][3] << 16);
        acc[db] = mfma32_bf16(__builtin_bit_cast(bf16x8_t, au), pb, acc[db]);
        acc[db] = mfma32_bf16(__builtin_bit_cast(bf16x8_t, au), pbl, acc[db]);
      }
    }
    __builtin_amdgcn_s_setprio(0);
  };
  for (int t = 0; t < ntv; t += NST) {
    tile(t, std::integral_constant<int, 0>{});
    if (t + 1 < ntv) tile(t + 1, std::integral_constant<int, 1>{});
    if constexpr (NST == 3)
      if (t + 2 < ntv) tile(t + 2, std::integral_constant<int, 2 % NST>{});
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no load into LDS outlives the wave
  const float l_tot = xor_sum<32>(l_run);
  if (!head_ok) return;
  // O^T accumulator: lane (c32, h) holds head c32, dims 32 db + 8 (i / 4) + 4 h + i % 4
  if (nsplit == 1) {
    const float inv = 1.f / fmaxf(l_tot, eps);
    bf16_t* orow = out + ((int64_t)b * Hq + hq) * D;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        Elem<bf16_t>::store(orow, 32 * db + 8 * (i / 4) + 4 * h + i % 4, acc[db][i] * inv);
  } else {
    float* pp = part + ((int64_t)b * Hq + hq) * part_stride(nsplit, D);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; i += 4)
        *reinterpret_cast<float4*>(pp + split * D + 32 * db + 8 * (i / 4) + 4 * h) =
            make_float4(acc[db][i], acc[db][i + 1], acc[db][i + 2], acc[db][i + 3]);
    if (h == 0)
      *reinterpret_cast<float2*>(pp + nsplit * D + 2 * split) =
          make_float2(l_tot > 0.f ? m_run : -INFINITY, l_tot);
  }
}

// ------------------------------------------------------------------ generic
// One wave per (b, hq, query row); any D <= 256, any dtype mix.  Pass 1 finds
// the row max and sum with lanes over keys; pass 2 has lanes over head dims.
template <typename TQ, typename TK, typename TV>
__global__ __launch_bounds__(64) void attn_generic(
    const TQ* __restrict__ q, const TK* __restrict__ k, const TV* __restrict__ v, int64_t kv_bs,
    int64_t kv_hs, const int32_t* __restrict__ qpos, int Hq, int Hkv, int Lq, int Lk, int D,
    int causal, float scale, float eps, TQ* __restrict__ out) {
  const int row = blockIdx.x, hq = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x;
  const int hkv = hq / (Hq / Hkv);
  __shared__ float qs[256];
  const int64_t qoff = (((int64_t)b * Hq + hq) * Lq + row) * D;
  for (int d = lane; d < D; d += 64) qs[d] = Elem<TQ>::load(q, qoff + d);
  __syncthreads();
  int kend = Lk;
  if (causal) {
    const int p = qpos ? qpos[(int64_t)b * Lq + row] : Lk - Lq + row;
    kend = max(0, min(Lk, p + 1));
  }
  const TK* kb = k + (int64_t)b * kv_bs + (int64_t)hkv * kv_hs;
  const TV* vb = v + (int64_t)b * kv_bs + (int64_t)hkv * kv_hs;
  float m = -INFINITY, s = 0.f;
  for (int t = lane; t < kend; t += 64) {
    float d = 0.f;
    for (int e = 0; e < D; ++e) d = fmaf(qs[e], Elem<TK>::load(kb, (int64_t)t * D + e), d);
    d *= scale;
    const float mn = fmaxf(m, d);
    s = s * __expf(m - mn) + __expf(d - mn);
    m = mn;
  }
  float mx = m;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  float sum = (s > 0.f) ? s * __expf(m - mx) : 0.f;
  sum = wave_sum(sum);
  for (int d0 = 0; d0 < D; d0 += 64) {
    const int d = d0 + lane;
    float o = 0.f;
    if (d < D) {
      for (int t = 0; t < kend; ++t) {
        float sc = 0.f;
        for (int e = 0; e < D; ++e) sc = fmaf(qs[e], Elem<TK>::load(kb, (int64_t)t * D + e), sc);
        o = fmaf(__expf(sc * scale - mx), Elem<TV>::load(vb, (int64_t)t * D + d), o);
      }
      Elem<TQ>::store(out, qoff + d, o / fmaxf(sum, eps));
    }
  }
}

// Key-axis split of the decode kernel for `Lcap` keys: enough workgroups to
// cover the GPU about 4x, at least 64 keys (one 4-wave sweep) per split
// below 3072 keys and 128 from there on, at most kMaxDecodeSplits splits.
// At batch 1 the kernel is bound by each wave's dependent chain, so short
// splits (more waves) win up to ~2.3k keys (2k: 7.6 us against 8.2 us); from
// 4k keys two sweeps per split halve the merge's work (4k: 10.1 us against
// 11.4 us; 8k: 15.5 us against 17.4 us).
constexpr int kLongSplitKeys = 3072;    // 128-key minimum split from here
constexpr int kLongContextKeys = 6144;  // few heads: 2 splits per CU from here
constexpr int kBatchedShortKeys = 2048; // batched heads: 2 per CU up to here
constexpr int kBatchedLongKeys = 16384; // batched heads: 6 per CU from here
void decode_split_geometry(int num_cus, int B, int Hkv, int Lcap, int* nsplit_out, int* chunk_out,
                           bool whole_group = false) {
  // A query group that cannot be halved over workgroups (odd G > 1, e.g.
  // Llama-3.2-3B's G = 3) also takes 128-key splits at short contexts
  // (3B decode at ~2k keys: 963 -> 971 tok/s; G = 4 keeps 64: 8B 649
  // against 629 tok/s with 128).
  int min_chunk = (Lcap >= kLongSplitKeys || whole_group) ? 128 : 64;
  // Batched heads (B*Hkv >= 64, e.g. 16 x 8): short contexts prefer longer
  // splits (1k keys: 21.6 us at 2 per CU against 24.0 at 4), very long ones
  // more of them (32k keys: 371 us at 6 against 378 at 4).  Few heads (batch
  // 1): from 6k keys longer splits (8k: 13.9 us at 2 per CU against 16.0;
  // 16k: 21.3 against 24.3; 32k: 30.0 against 34.4; below 8k the 128-key
  // minimum already bounds the count).  strata_attn_decode_splits takes the maximum
  // over these regimes' boundaries for the partials sizing.
  int per_cu = 4;
  if (B * Hkv >= 64)
    per_cu = Lcap <= kBatchedShortKeys ? 2 : (Lcap >= kBatchedLongKeys ? 6 : 4);
  else if (Lcap >= kLongContextKeys)
    per_cu = 2;
  int want = (num_cus * per_cu + B * Hkv - 1) / (B * Hkv);
  if (want > kMaxDecodeSplits) want = kMaxDecodeSplits;
  int nsplit = (Lcap + min_chunk - 1) / min_chunk;
  if (nsplit > want) nsplit = want;
  if (nsplit < 1) nsplit = 1;
  int chunk = (Lcap + nsplit - 1) / nsplit;
  if (chunk < 1) chunk = 1;
  nsplit = (Lcap + chunk - 1) / chunk;
  if (nsplit < 1) nsplit = 1;
  *nsplit_out = nsplit;
  *chunk_out = chunk;
}

// bf16 decode over many (row, KV head, key) triples runs attn_decode_mfma:
// batched heads (B * Hkv >= 64), or at least 64 Ki key-heads (batch 1 with 8
// KV heads from 8k keys).  Below that the latency-bound vector kernel wins
// (MI355X, Hq32/Hkv8 D128, MFMA against vector: B1/L2k 9.0 against 8.1 us,
// B1/L8k 12.0 against 13.9, B1/L32k 27.1 against 30.5, B4/L8k 26.3 against
// 30.7).  One wave per (b, KV head, key chunk), about 4 waves per CU in all,
// chunks a multiple of the 32-key tile and at least 64 keys.
constexpr int kMfmaDecodeMinHeads = 64;
constexpr int64_t kMfmaDecodeMinKeyHeads = 65536;
inline bool mfma_decode(int B, int Hkv, int64_t L) {
  static const bool vector_only = getenv("STRATA_ATTN_DECODE_VECTOR") != nullptr;
  static const bool mfma_always = getenv("STRATA_ATTN_DECODE_MFMA") != nullptr;
  if (vector_only) return false;
  return mfma_always || B * Hkv >= kMfmaDecodeMinHeads || (int64_t)B * Hkv * L >= kMfmaDecodeMinKeyHeads;
}
constexpr int kMfmaDecodeWaves = 4;  // waves per workgroup (each with its own LDS ring)
void decode_mfma_geometry(int num_cus, int B, int Hkv, int Lcap, int* nsplit_out, int* chunk_out) {
  int per_cu = 4;
  int ns = (num_cus * per_cu + B * Hkv - 1) / (B * Hkv);
  ns = std::max(1, std::min(ns, std::min(kMaxDecodeSplits, (Lcap + 63) / 64)));
  int chunk = (Lcap + ns - 1) / ns;
  chunk = std::max(32, (chunk + 31) / 32 * 32);
  *nsplit_out = std::max(1, (Lcap + chunk - 1) / chunk);
  *chunk_out = chunk;
}

template <typename TQ, typename TK, typename TV, int D>
int launch_decode(strata_ctx* ctx, const void* q, const void* k, const void* v, int64_t kv_bs,
                  int64_t kv_hs, const int32_t* qpos, int B, int Hq, int Hkv, int Lk, int causal,
                  float scale, float eps, void* out, const AttnExtra& ex, hipStream_t stream) {
  const int G = Hq / Hkv;
  if constexpr (sizeof(TQ) == 2 && sizeof(TK) == 2 && sizeof(TV) == 2) {
    // (STRATA_ATTN_DECODE_VECTOR / STRATA_ATTN_DECODE_MFMA force either kernel)
    if (G <= 32 && mfma_decode(B, Hkv, Lk)) {
      // (B16 Hq32/Hkv8 D128 on MI355X against attn_decode_kernel: 1k keys
      // 21.4 -> 17.3-18.0 us, 8k 113 -> 102 us, 32k 387 -> 370 us)
      constexpr int WPG = kMfmaDecodeWaves;
      int ns, ch;
      decode_mfma_geometry(ctx->num_cus, B, Hkv, Lk, &ns, &ch);
      float* pt = nullptr;
      if (ns > 1) {
        if (ex.part) {
          if (ex.part_splits < ns)
            return strata_set_error(STRATA_EINVAL, "decode attention: partials buffer too small");
          pt = ex.part;
        } else {
          void* p = nullptr;
          const int rc = strata_ctx_scratch(ctx, (size_t)B * Hq * part_stride(ns, D) * sizeof(float), &p, stream);
          if (rc) return rc;
          pt = reinterpret_cast<float*>(p);
        }
      }
      const int items = B * Hkv * ns;
      hipLaunchKernelGGL((attn_decode_mfma<D, 2, WPG>), dim3((items + WPG - 1) / WPG), dim3(64 * WPG),
                         0, stream, (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, kv_bs,
                         kv_hs, B, Hq, Hkv, Lk, ch, ns, qpos, ex.dlen, causal, scale, eps, pt,
                         (bf16_t*)out);
      STRATA_HIP_CHECK(hipGetLastError());
      if (ns > 1) {
        launch_decode_merge<TQ>(pt, ns, D, B * Hq, eps, (TQ*)out, stream);
        STRATA_HIP_CHECK(hipGetLastError());
      }
      return STRATA_OK;
    }
  }
  int nsplit, chunk;
  decode_split_geometry(ctx->num_cus, B, Hkv, Lk, &nsplit, &chunk, G > 1 && G % 2 != 0);
  float* part = nullptr;
  if (nsplit > 1) {
    if (ex.part) {  // decoder-owned partials (graph-safe: no allocation)
      if (ex.part_splits < nsplit)
        return strata_set_error(STRATA_EINVAL, "decode attention: partials buffer too small");
      part = ex.part;
    } else {
      void* p = nullptr;
      const int rc = strata_ctx_scratch(ctx, (size_t)B * Hq * part_stride(nsplit, D) * sizeof(float), &p, stream);
      if (rc) return rc;
      part = reinterpret_cast<float*>(p);
    }
  }
  // Query heads per workgroup: the whole group reads K/V once; while the grid
  // has fewer than two workgroups per CU the group is halved, so each wave's
  // chain is shorter (batch 1: 1k keys 1 head, 2k-4k keys 2 heads per
  // workgroup: 2k 8.6 -> 7.6 us, 4k 10.7 -> 10.1 us; 8k+ and batch 16 keep
  // the full group, which reads K/V once).
  int HG = G;
  while (HG % 2 == 0 && (int64_t)nsplit * B * Hkv * (G / HG) < 2 * ctx->num_cus) HG /= 2;
  dim3 grid(nsplit, Hkv * (G / HG), B);
#define STRATA_DEC(GV)                                                                        \
  if (HG == GV)                                                                               \
    hipLaunchKernelGGL((attn_decode_kernel<TQ, TK, TV, D, GV>), grid, dim3(256), 0, stream,   \
                       (const TQ*)q, (const TK*)k, (const TV*)v, kv_bs, kv_hs, Lk, chunk, G,  \
                       Hq, qpos, ex.dlen, causal, nsplit, scale, eps, part, (TQ*)out);
  STRATA_DEC(1) else STRATA_DEC(2) else STRATA_DEC(3) else STRATA_DEC(4) else STRATA_DEC(6) else
  STRATA_DEC(8) else
    return strata_set_error(STRATA_ENOTSUP, "decode attention: group size %d not in {1,2,3,4,6,8}",
                            G);
#undef STRATA_DEC
  STRATA_HIP_CHECK(hipGetLastError());
  if (nsplit > 1) {
    launch_decode_merge<TQ>(part, nsplit, D, B * Hq, eps, (TQ*)out, stream);
    STRATA_HIP_CHECK(hipGetLastError());
  }
  return STRATA_OK;
}

template <typename TQ, typename TK, typename TV>
int launch_generic(const void* q, const void* k, const void* v, int64_t kv_bs, int64_t kv_hs,
                   const int32_t* qpos, int B, int Hq, int Hkv, int Lq, int Lk, int D, int causal,
                   float scale, float eps, void* out, hipStream_t stream) {
  hipLaunchKernelGGL((attn_generic<TQ, TK, TV>), dim3(Lq, Hq, B), dim3(64), 0, stream,
                     (const TQ*)q, (const TK*)k, (const TV*)v, kv_bs, kv_hs, qpos, Hq, Hkv, Lq, Lk,
                     D, causal, scale, eps, (TQ*)out);
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}

template <typename TQ, typename TK, typename TV>
int dispatch_types(strata_ctx* ctx, const void* q, const void* k, const void* v, int64_t kv_bs,
                   int64_t kv_hs, const int32_t* qpos, int B, int Hq, int Hkv, int Lq, int Lk,
                   int D, int causal, float scale, float eps, void* out, const AttnExtra& ex,
                   hipStream_t stream) {
  const int G = Hq / Hkv;
  const bool g_ok = G == 1 || G == 2 || G == 3 || G == 4 || G == 6 || G == 8;
  if (Lq == 1 && g_ok && (D == 64 || D == 128)) {
    if (D == 64)
      return launch_decode<TQ, TK, TV, 64>(ctx, q, k, v, kv_bs, kv_hs, qpos, B, Hq, Hkv, Lk,
                                           causal, scale, eps, out, ex, stream);
    return launch_decode<TQ, TK, TV, 128>(ctx, q, k, v, kv_bs, kv_hs, qpos, B, Hq, Hkv, Lk, causal,
                                          scale, eps, out, ex, stream);
  }
  if constexpr (sizeof(TQ) == sizeof(TK) && sizeof(TK) == sizeof(TV)) {
    if (Lq > 1 && (D == 64 || D == 128)) {
      if constexpr (sizeof(TQ) == 2) {
        // 4 waves (128 query rows) per workgroup, two LDS stages of 32-key
        // tiles (32 KB): three workgroups per CU (160 VGPRs), whose waves
        // share each SIMD without sharing a barrier (8k causal: 586-602 us;
        // 64-key tiles, two workgroups per CU: 606-628 us; 8 waves in one
        // workgroup per CU: 683-696 us; a third stage: no gain)
        constexpr int NWV = 4, NSTV = 2, KTV = 32;
        const dim3 grid(prefill_grid((Lq + 32 * NWV - 1) / (32 * NWV), B, Hkv, Hq / Hkv));
        if (D == 64)
          hipLaunchKernelGGL((attn_prefill_mfma32<64, NWV, NSTV, KTV>), grid, dim3(64 * NWV), 0,
                             stream, (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, kv_bs,
                             kv_hs, qpos, B, Hq, Hkv, Lq, Lk, causal, scale, eps, ex.out_tm,
                             (bf16_t*)out);
        else
          hipLaunchKernelGGL((attn_prefill_mfma32<128, NWV, NSTV, KTV>), grid, dim3(64 * NWV), 0,
                             stream, (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, kv_bs,
                             kv_hs, qpos, B, Hq, Hkv, Lq, Lk, causal, scale, eps, ex.out_tm,
                             (bf16_t*)out);
      } else {
        // fp32: 16x16x4 MFMA tiles, 64 query rows per workgroup
        const dim3 grid(prefill_grid((Lq + 63) / 64, B, Hkv, Hq / Hkv));
        if (D == 64)
          hipLaunchKernelGGL((attn_prefill_f32<64>), grid, dim3(256), 0, stream,
                             (const float*)q, (const float*)k, (const float*)v, kv_bs, kv_hs, qpos,
                             B, Hq, Hkv, Lq, Lk, causal, scale, eps, ex.out_tm, (float*)out);
        else
          hipLaunchKernelGGL((attn_prefill_f32<128>), grid, dim3(256), 0, stream,
                             (const float*)q, (const float*)k, (const float*)v, kv_bs, kv_hs, qpos,
                             B, Hq, Hkv, Lq, Lk, causal, scale, eps, ex.out_tm, (float*)out);
      }
      STRATA_HIP_CHECK(hipGetLastError());
      return STRATA_OK;
    }
  }
  return launch_generic<TQ, TK, TV>(q, k, v, kv_bs, kv_hs, qpos, B, Hq, Hkv, Lq, Lk, D, causal,
                                    scale, eps, out, stream);
}

}  // namespace

int strata_attn_decode_splits(strata_ctx* ctx, int B, int Hkv, int Lcap) {
  int nsplit, chunk;
  decode_split_geometry(ctx->num_cus, B, Hkv, Lcap, &nsplit, &chunk);
  if (mfma_decode(B, Hkv, Lcap)) {  // the MFMA kernel's count grows with Lcap
    int n2;
    decode_mfma_geometry(ctx->num_cus, B, Hkv, Lcap, &n2, &chunk);
    nsplit = std::max(nsplit, n2);
  }
  // The split count grows with the capacity within each regime of the
  // geometry (minimum chunk, splits per CU); the last capacity before a
  // regime boundary may need more splits than Lcap.
  const int bounds[] = {kBatchedShortKeys, kLongSplitKeys - 1, kLongContextKeys - 1,
                        kBatchedLongKeys - 1};
  for (int bnd : bounds) {
    if (Lcap > bnd) {
      int n2;
      decode_split_geometry(ctx->num_cus, B, Hkv, bnd, &n2, &chunk);
      nsplit = std::max(nsplit, n2);
    }
  }
  return nsplit;
}

int strata_attention_dispatch(strata_ctx* ctx, const void* q, int qd, const void* k, int kd,
                              const void* v, int vd, int64_t kv_bs, int64_t kv_hs,
                              const int32_t* qpos, int B, int Hq, int Hkv, int Lq, int Lk, int D,
                              int causal, float eps, void* out, const AttnExtra& ex,
                              void* stream) {
  const float scale = 1.0f / sqrtf(static_cast<float>(D));
  hipStream_t s = as_stream(stream);
#define STRATA_T(c) std::conditional_t<(c) == STRATA_BF16, bf16_t, float>
#define STRATA_CASE(A, Bc, C)                                                                  \
  if (qd == A && kd == Bc && vd == C)                                                          \
    return dispatch_types<STRATA_T(A), STRATA_T(Bc), STRATA_T(C)>(                             \
        ctx, q, k, v, kv_bs, kv_hs, qpos, B, Hq, Hkv, Lq, Lk, D, causal, scale, eps, out, ex, s);
  STRATA_CASE(STRATA_BF16, STRATA_BF16, STRATA_BF16)
  STRATA_CASE(STRATA_F32, STRATA_F32, STRATA_F32)
  STRATA_CASE(STRATA_F32, STRATA_F32, STRATA_BF16)
  STRATA_CASE(STRATA_BF16, STRATA_F32, STRATA_BF16)
  STRATA_CASE(STRATA_F32, STRATA_BF16, STRATA_BF16)
#undef STRATA_CASE
#undef STRATA_T
  return strata_set_error(STRATA_ENOTSUP, "attention: unsupported dtype combination q=%d k=%d v=%d",
                          qd, kd, vd);
}
