// Decode q4 GEMV on the matrix cores, over a load-time weight layout.
//
//   y[m, n] = sum_k x[m, k] * (s[n, k/64] * q[n, k] + b[n, k/64]),  M <= 4
//   (mx.quantized_matmul(transpose=True) of the decode step,
//    src/ollm/llama_mlx.py:53-74; callers 257-268, 313-316, 393-408)
//
// Why the matrix cores: at batch 1 every code is used once, so the cost per
// weight byte is the VALU work that turns codes into bf16 operands plus the
// dot.  A 4-bit code pair becomes a bf16 pair (128 + q) with one AND-OR of
// the magic 0x43004300 (3 shifts + 4 AND-ORs per 8 codes); the dot itself
// goes to a 16x16x32 bf16 MFMA instead of 16 v_dot2 per 32 codes.  The x
// operand carries each k-octet in the MFMA column of its group, so one
// accumulator tile collects 16 rows x 16 separate group dots and the
// per-group affine terms are applied once per 1024 codes:
//   acc += s * sum_k x (128 + q) + (b - 128 s) * sum_k x.
//
// Layout ("GEMV layout", built once by q4_gemv_pack_kernel from the MLX
// layout; one buffer per group of linears launched together):
//   * packed rows come in blocks of 16 (a block is one workgroup); K is
//     padded to Kp = 1024 * nt and split into nt tasks of 16 groups, one per
//     wave of the workgroup;
//   * task (rb, t), wave-load w (0..7), lane l = 16 j + m:
//       codes[((rb * nt + t) * 8 + w) * 64 + l]  (uint4) = packed row m of the
//       block, group g = 16 t + 4 (w / 2) + j, codes 32 (w % 2) .. +31 of the
//       group (16 contiguous bytes of the MLX row), each 8-code word with its
//       nibbles re-ordered so that (word >> 4c) & 0x000f000f is the pair of
//       codes (2c, 2c + 1): the x operand is then x itself, in order;
//   * sb[((rb * nt + t) * 64 + L) * 4 + i] (u32) = s | b << 16 of packed row
//     4 (L / 16) + i, group 16 t + L % 16 (zero for padding).
//   Word p of wave-load w (MFMA step 4 w + p) is the A operand of phase
//   a = w / 2 (groups 16 t + 4 a + j), octet o = 4 (w % 2) + p.
//   The B operand of that step: lane (j, n) holds x[octet o of group
//   16 t + 4 a + j] when n == 4 a + j and zeros otherwise (M = 1), so
//   C[m][n] accumulates group 16 t + n of row m over the 32 steps.  For
//   2 <= M <= 4, column n = 4 b + j' carries batch row b and group
//   4 a + j', and the affine terms are applied after each phase.
// Rows may be permuted inside a block so that epilogue pairs share it:
//   perm 1 (gate/up): block rows 0-7 are gate rows 8 lb .. +7, rows 8-15 the
//     up rows of the same indices;
//   perm 2 (q/k/v with RoPE): inside head h, block b' holds head rows
//     8 b' .. +7 and D/2 + 8 b' .. +7 (the rotate-half pairs).
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "strata_internal.h"

namespace {

constexpr uint32_t kMagic2 = 0x43004300u;  // bf16 pair (128.0, 128.0)

// (w & 0x000f000f) | 0x43004300: one v_and_or_b32 with the mask in a VGPR
// (mask_v) and the magic in an SGPR.  Plain C, not inline assembly: the
// result feeds the matrix cores, and the compiler must see the VALU write to
// keep the VALU -> MFMA operand hazard wait states.
__device__ __forceinline__ uint32_t code_pair(uint32_t w, uint32_t mask_v) {
  return (w & mask_v) | kMagic2;
}

__device__ __forceinline__ f32x4_t mfma16(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

template <int CTRL>
__device__ __forceinline__ float dppv(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}

struct GvProblem {
  void* y;       // output [M, n] (RESID: the residual stream, updated in place)
  int64_t n;     // output rows
  int rb0;       // first row block of the problem in the layout
};

struct GvArgs {
  const uint4* codes;
  const uint4* sb;
  int M, K, nt;
  int count;
  GvProblem p[kGvMaxProblems];
  int rb_end[kGvMaxProblems];
  int nrb;   // row blocks of the layout
  int pair;  // MP 1, 5-8 rows: both 4-row halves of every row block in one grid
  // RoPE / KV append (EPI_ROPE)
  int head_dim, n_heads, n_kv_heads, lmax, pos0;
  const int* dpos;            // device position (graph-replayed step) or null
  const float2* rope_table;   // [lmax][D/2]
  const float2* rope_cur;     // with dpos: (cos, sin) row of *dpos
  uint16_t* q_out;            // [M, Hq, 1, D]
  uint16_t* kc;               // cache layer [M, Hkv, lmax, D]
  uint16_t* vc;
  const uint16_t* norm_w;     // RMSNorm prologue weight [K] (NORM)
  float eps;
};

enum { GV_STORE = 0, GV_SILU = 1, GV_ROPE = 2, GV_RESID = 3 };

// Per-wave LDS: staged x [MM][1024] bf16, a zero block, group sums [MM][16].
template <int MM>
constexpr int kWaveLds = MM * 2048 + 256 + MM * 64;

// Occupancy: the batch-1 store / SiLU / residual kernels fit 72 VGPRs, so
// seven 4-wave workgroups share a CU and the 8B gate/up launch (1792 blocks)
// is resident at once; the RoPE kernel (one block per 16 q/k/v rows, fewer
// than two per CU) and the batched kernels get more registers instead.
template <int MP, int EPI>
constexpr int kGvWavesPerEu = MP != 0 ? 2 : (EPI == 2 ? 4 : 7);

// NTC: the K task count when known at compile time (4: the 8B hidden width,
// 14: the 8B FFN width, 3 and 8: the 3B widths), 0 for any (up to 16).
// HT: waves per K task.  With HT = 2 (batch 1, launches too small to fill
// the GPU) each wave takes half a task, 4 of its 8 weight loads and 2 of its
// 4 phases, so the block has twice the waves, each with half the chain.
template <int MP, int EPI, bool NORM, typename YT, int NTC, int HT = 1>
__global__ __launch_bounds__(NTC ? 64 * NTC * HT : 1024) __attribute__((amdgpu_waves_per_eu(kGvWavesPerEu<MP, EPI>)))
void q4_gemv_mfma_kernel(const uint16_t* __restrict__ x, const uint4* __restrict__ codes,
                         const uint4* __restrict__ sbp, const uint16_t* __restrict__ nw, int Ma,
                         int K, int nta, GvArgs a) {
  static_assert(HT == 1 || (HT == 2 && MP == 0), "half tasks are batch-1 only");
  constexpr int MM = MP == 0 ? 1 : 4;  // staged batch rows
  constexpr int NE = 2 / HT;           // x uint4 per lane of the wave's (half) task
  constexpr int NWL = 8 / HT;          // weight loads per lane
  extern __shared__ uint4 smem[];
  // x, the weights, the norm weights and the shape lead the argument list:
  // the dispatch preloads them into SGPRs, so the first loads issue without
  // waiting for the argument segment.
  const int nt = NTC ? NTC : nta;
  // a.pair (MP 1, 5-8 rows): workgroups 16 i + c and 16 i + 8 + c take batch
  // rows 0-3 and 4-7 of row block 8 i + c.  Both run on XCD c, one soon
  // after the other, so the second finds the block's weights in that L2.
  int rb = blockIdx.x, ro = 0;
  if constexpr (MP == 1) {
    if (a.pair) {
      const int slot = rb >> 3;
      ro = 4 * (slot & 1);
      rb = (slot >> 1) * 8 + (rb & 7);
      if (rb >= a.nrb) return;  // grid padding (whole workgroup)
    }
  }
  const int M = MP == 1 ? min(4, Ma - ro) : Ma;  // rows of this workgroup
  const uint16_t* const xp = x + (int64_t)ro * K;
  const int lane = threadIdx.x & 63, j = lane >> 4, n = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t = HT == 2 ? wave >> 1 : wave;  // this wave's K task
  const int hh = HT == 2 ? wave & 1 : 0;     // and its half (HT = 2)
  const int nw_ = nt * HT;                   // waves of the block
  char* base = reinterpret_cast<char*>(smem);
  uint4* xw = reinterpret_cast<uint4*>(base + wave * kWaveLds<MM>);
  uint4* zero = xw + MM * 128;
  float* xs = reinterpret_cast<float*>(zero + 16);
  float* red = reinterpret_cast<float*>(base + nw_ * kWaveLds<MM>);  // [waves][MM][16]
  float* nred = red + nw_ * MM * 16;                                  // [waves][MM]

  // x of the task: uint4 u (0..127) = x[8u .. 8u+7] of the task, group u / 8.
  // (HT = 2: the wave's half hh holds u = 64 hh + lane, one per lane)
  uint4 xv[MM][NE], wn[NE];
#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int ee = 0; ee < NE; ++ee) {
      const int e = HT == 2 ? hh : ee;
      const int k = 1024 * t + 8 * (lane + 64 * e);
      const int mc = min(m, M - 1);
      xv[m][ee] = k < K ? *reinterpret_cast<const uint4*>(xp + (int64_t)mc * K + k)
                        : make_uint4(0, 0, 0, 0);
    }
  if constexpr (NORM) {
#pragma unroll
    for (int ee = 0; ee < NE; ++ee) {
      const int e = HT == 2 ? hh : ee;
      const int k = 1024 * t + 8 * (lane + 64 * e);
      wn[ee] = k < K ? *reinterpret_cast<const uint4*>(nw + k) : make_uint4(0, 0, 0, 0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // weights and affine terms of the task, all issued before any math
  uint4 wb[NWL];
  uint4 sbv[MP == 0 ? 1 : 4];
  {
    const int64_t tb = (int64_t)rb * nt + t;
    if constexpr (MP == 0) {
      sbv[0] = load_nt(sbp + tb * 64 + lane);
    } else {
#pragma unroll
      for (int ph = 0; ph < 4; ++ph) sbv[ph] = load_nt(sbp + tb * 64 + 16 * j + 4 * ph + (lane & 3));
    }
#pragma unroll
    for (int w = 0; w < NWL; ++w) wb[w] = load_nt(codes + (tb * 8 + 4 * hh + w) * 64 + lane);
  }
  __builtin_amdgcn_sched_barrier(0);

  // The block's problem (output linear) and the epilogue threads' roles.
  // Looked up only now: its dependent scalar loads would otherwise hold back
  // the weight stream.
  int pi = 0;
#pragma unroll
  for (int q = 1; q < kGvMaxProblems; ++q)
    if (q < a.count && rb >= a.p[q].rb0) pi = q;
  const int lb = rb - a.p[pi].rb0;
  const int em = threadIdx.x >> 4, er = threadIdx.x & 15;  // epilogue thread: batch row, block row
  const int eb = em + ro;  // its row of the whole batch
  const bool eth = wave == 0 && em < M;
  // epilogue operands, fetched now (they return with the weights); the
  // residual values are loaded by every lane at an in-bounds index
  uint16_t hpre = 0;
  if constexpr (EPI == GV_RESID) {
    const int64_t nl = min(16 * (int64_t)lb + er, a.p[pi].n - 1);
    hpre = reinterpret_cast<const uint16_t*>(a.p[pi].y)[(int64_t)(min(em, M - 1) + ro) * a.p[pi].n + nl];
  }
  int pos = a.pos0;
  float2 cs = make_float2(0.f, 0.f);
  if constexpr (EPI == GV_ROPE) {
    if (eth && a.dpos) {
      using gint = const __attribute__((address_space(1))) int;
      int zv;
      asm volatile("v_mov_b32 %0, 0" : "=v"(zv));
      pos = ((gint*)a.dpos)[zv];
    }
    if (eth && er < 8 && pi < 2) {
      const int D = a.head_dim, i = 8 * (lb % (D >> 4)) + er;
      cs = a.dpos ? a.rope_cur[i] : a.rope_table[(int64_t)a.pos0 * (D >> 1) + i];
    }
  }

  // RMSNorm prologue (llama_mlx.py:77-92): r = 1/sqrt(mean(x^2) + eps) over
  // the whole row (the block's waves together hold it), then
  // x <- bf16(w * (x * r)) with each product rounded, in registers.
  if constexpr (NORM) {
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      float sq = 0.f;
#pragma unroll
      for (int ee = 0; ee < NE; ++ee) {
        const uint32_t u[4] = {xv[m][ee].x, xv[m][ee].y, xv[m][ee].z, xv[m][ee].w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float lo = __uint_as_float(u[c] << 16), hi = __uint_as_float(u[c] & 0xffff0000u);
          sq = fmaf(lo, lo, sq);
          sq = fmaf(hi, hi, sq);
        }
      }
      sq = wave_sum(sq);
      if (lane == 0) nred[wave * MM + m] = sq;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      float tot = 0.f;
      for (int w = 0; w < nw_; ++w) tot += nred[w * MM + m];
      const float r = 1.0f / sqrtf(tot / static_cast<float>(K) + a.eps);
#pragma unroll
      for (int ee = 0; ee < NE; ++ee) {
        uint32_t* u = reinterpret_cast<uint32_t*>(&xv[m][ee]);
        const uint32_t wu[4] = {wn[ee].x, wn[ee].y, wn[ee].z, wn[ee].w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float lo = mul_rn(mul_rn(__uint_as_float(u[c] << 16), r), __uint_as_float(wu[c] << 16));
          const float hi = mul_rn(mul_rn(__uint_as_float(u[c] & 0xffff0000u), r),
                                  __uint_as_float(wu[c] & 0xffff0000u));
          u[c] = static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
        }
      }
    }
  }
  // stage x in the wave's own LDS region (no barrier: only this wave reads
  // it) and take its group sums from the registers
#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int ee = 0; ee < NE; ++ee) {
      const int e = HT == 2 ? hh : ee;
      const uint4 v = m < M ? xv[m][ee] : make_uint4(0, 0, 0, 0);
      xw[m * 128 + lane + 64 * e] = v;
      const uint32_t u[4] = {v.x, v.y, v.z, v.w};
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) s += __uint_as_float(u[c] << 16) + __uint_as_float(u[c] & 0xffff0000u);
      s += dppv<0xB1>(s);   // quad_perm [1,0,3,2]
      s += dppv<0x4E>(s);   // quad_perm [2,3,0,1]
      s += dppv<0x141>(s);  // row_half_mirror: 8 lanes = one group
      if ((lane & 7) == 0) xs[m * 16 + 8 * e + (lane >> 3)] = s;
    }
  if (lane < 16) zero[lane] = make_uint4(0, 0, 0, 0);
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  uint32_t mask = 0x000f000fu;
  asm volatile("" : "+v"(mask));  // the AND-OR mask lives in a VGPR
  auto a_op = [&](int p) {
    const uint4 w4 = wb[p >> 2];
    const uint32_t wd = (p & 3) == 0 ? w4.x : (p & 3) == 1 ? w4.y : (p & 3) == 2 ? w4.z : w4.w;
    u32x4_t av;
    av.x = code_pair(wd, mask);
    av.y = code_pair(wd >> 4, mask);
    av.z = code_pair(wd >> 8, mask);
    av.w = code_pair(wd >> 12, mask);
    return av;
  };
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if constexpr (MP == 0) {
    // the wave's phases: 4 (HT = 1), or 2 hh .. 2 hh + 1 (HT = 2)
    constexpr int NPH = 4 / HT;
    const uint4* bb[NPH];
#pragma unroll
    for (int q = 0; q < NPH; ++q) {
      const int ph = NPH * hh + q;
      bb[q] = (n == 4 * ph + j) ? xw + (4 * ph + j) * 8 : zero;
    }
    f32x4_t c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < 8 * NPH; ++p) {
      const u32x4_t av = a_op(p);
      const uint4 bv = bb[p >> 3][p & 7];
      const u32x4_t bq = {bv.x, bv.y, bv.z, bv.w};
      if (p & 1) c1 = mfma16(av, bq, c1);
      else c0 = mfma16(av, bq, c0);
    }
    // group column n belongs to phase n / 4: columns of the other half's
    // phases hold no product and get no affine term
    const float X = (HT == 1 || (n >> 3) == hh) ? xs[n] : 0.f;
    const uint32_t sw[4] = {sbv[0].x, sbv[0].y, sbv[0].z, sbv[0].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float sc = __uint_as_float(sw[i] << 16), bc = __uint_as_float(sw[i] & 0xffff0000u);
      acc[i] = sc * (c0[i] + c1[i]) + fmaf(-128.f, sc, bc) * X;
    }
    // sum the 16 group columns of each row (one DPP row)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = acc[i];
      v += dppv<0x121>(v);  // row_ror:1
      v += dppv<0x122>(v);  // row_ror:2
      v += dppv<0x124>(v);  // row_ror:4
      v += dppv<0x128>(v);  // row_ror:8
      acc[i] = v;
    }
    if (n == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) red[wave * 16 + 4 * j + i] = acc[i];
    }
  } else {
    // column n = 4 b + j': batch row b, group 4 ph + j' of the phase
    const int bm = n >> 2, jg = n & 3;
    const bool act = jg == j && bm < M;
#pragma unroll
    for (int ph = 0; ph < 4; ++ph) {
      const uint4* bb = act ? xw + bm * 128 + (4 * ph + j) * 8 : zero;
      f32x4_t c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int o = 0; o < 8; ++o) {
        const u32x4_t av = a_op(8 * ph + o);
        const uint4 bv = bb[o];
        const u32x4_t bq = {bv.x, bv.y, bv.z, bv.w};
        if (o & 1) c1 = mfma16(av, bq, c1);
        else c0 = mfma16(av, bq, c0);
      }
      const float X = xs[min(bm, MM - 1) * 16 + 4 * ph + jg];
      const uint32_t sw[4] = {sbv[ph].x, sbv[ph].y, sbv[ph].z, sbv[ph].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float sc = __uint_as_float(sw[i] << 16), bc = __uint_as_float(sw[i] & 0xffff0000u);
        acc[i] += sc * (c0[i] + c1[i]) + fmaf(-128.f, sc, bc) * X;
      }
    }
    // sum the 4 group columns of each batch row (one lane quad)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = acc[i];
      v += dppv<0xB1>(v);
      v += dppv<0x4E>(v);
      acc[i] = v;
    }
    if (jg == 0 && bm < M) {
#pragma unroll
      for (int i = 0; i < 4; ++i) red[(wave * MM + bm) * 16 + 4 * j + i] = acc[i];
    }
  }
  __syncthreads();
  if (!eth) return;
  // the K tasks of the block summed in task order (deterministic)
  auto total = [&](int row) {
    float s = 0.f;
    for (int w = 0; w < nw_; ++w) s += red[(w * MM + (MP == 0 ? 0 : em)) * 16 + row];
    return s;
  };
  const GvProblem& P = a.p[pi];
  if constexpr (EPI == GV_STORE || EPI == GV_RESID) {
    const int64_t nl = 16 * (int64_t)lb + er;
    if (nl >= P.n) return;
    const float v = total(er);
    if constexpr (EPI == GV_RESID) {
      uint16_t* hp = reinterpret_cast<uint16_t*>(P.y) + (int64_t)eb * P.n + nl;
      *hp = f32_to_bf16(bf16_to_f32(hpre) + bf16_to_f32(f32_to_bf16(v)));
    } else {
      Elem<YT>::store(reinterpret_cast<YT*>(P.y), (int64_t)eb * P.n + nl, v);
    }
  } else if constexpr (EPI == GV_SILU) {
    // act = bf16(silu(bf16(gate)) * bf16(up))   (llama_mlx.py:399-407)
    const int64_t nl = 8 * (int64_t)lb + er;
    if (er >= 8 || nl >= P.n) return;
    const float g = bf16_to_f32(f32_to_bf16(total(er)));
    const float u = bf16_to_f32(f32_to_bf16(total(er + 8)));
    const float sg = g / (1.0f + expf(-g));
    reinterpret_cast<uint16_t*>(P.y)[(int64_t)eb * P.n + nl] = f32_to_bf16(mul_rn(sg, u));
  } else {
    // q/k/v: RoPE on q and k at the step's position, k and v into the cache
    // (llama_mlx.py:271-297; values rounded to bf16 before the rotation)
    if (er >= 8) return;
    const int D = a.head_dim, half = D >> 1, D16 = D >> 4;
    const int h = lb / D16, i = 8 * (lb - h * D16) + er;
    const float a0 = bf16_to_f32(f32_to_bf16(total(er)));
    const float a1 = bf16_to_f32(f32_to_bf16(total(er + 8)));
    if (pi == 2) {
      const int64_t co = (((int64_t)eb * a.n_kv_heads + h) * a.lmax + pos) * D;
      a.vc[co + i] = f32_to_bf16(a0);
      a.vc[co + i + half] = f32_to_bf16(a1);
    } else {
      float o1, o2;
      rotate_pair(a0, a1, cs.x, cs.y, &o1, &o2);
      if (pi == 0) {
        const int64_t qo = ((int64_t)eb * a.n_heads + h) * D;
        a.q_out[qo + i] = f32_to_bf16(o1);
        a.q_out[qo + i + half] = f32_to_bf16(o2);
      } else {
        const int64_t co = (((int64_t)eb * a.n_kv_heads + h) * a.lmax + pos) * D;
        a.kc[co + i] = f32_to_bf16(o1);
        a.kc[co + i + half] = f32_to_bf16(o2);
      }
    }
  }
}

// ---------------------------------------------------------------- packing
struct GvPackArgs {
  const uint32_t* w[kGvMaxProblems];
  const uint16_t* s[kGvMaxProblems];
  const uint16_t* b[kGvMaxProblems];
  int64_t n[kGvMaxProblems];
  int rb0[kGvMaxProblems + 1];
  int count;  // packed problems
  int perm, head_dim, K, nt, nrb;
};

// Source (weight index, row) of packed row pr of packed problem p; row < 0
// for padding.
__device__ __forceinline__ void gv_source(const GvPackArgs& a, int p, int pr, int* wi, int64_t* row) {
  const int lb = pr >> 4, r = pr & 15;
  if (a.perm == 1) {  // gate/up pairs
    *wi = r < 8 ? 0 : 1;
    const int64_t rr = 8 * (int64_t)lb + (r & 7);
    *row = rr < a.n[0] ? rr : -1;
  } else if (a.perm == 2) {  // rotate-half pairs inside each head
    const int D = a.head_dim, D16 = D >> 4;
    const int h = lb / D16, bq = lb - h * D16;
    const int hr = r < 8 ? 8 * bq + r : (D >> 1) + 8 * bq + (r - 8);
    *wi = p;
    const int64_t rr = (int64_t)h * D + hr;
    *row = rr < a.n[p] ? rr : -1;
  } else {
    *wi = p;
    *row = pr < a.n[p] ? pr : -1;
  }
}

__device__ __forceinline__ int gv_problem(const GvPackArgs& a, int rb) {
  int p = 0;
  for (int q = 1; q < a.count; ++q)
    if (rb >= a.rb0[q]) p = q;
  return p;
}

__global__ void q4_gemv_pack_codes(GvPackArgs a, uint4* __restrict__ codes) {
  const int64_t total = (int64_t)a.nrb * a.nt * 512;
  const int G = a.K >> 6;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int lane = idx & 63, w = (idx >> 6) & 7;
    const int64_t tb = idx >> 9;
    const int t = tb % a.nt, rb = tb / a.nt;
    const int p = gv_problem(a, rb);
    int wi;
    int64_t row;
    gv_source(a, p, 16 * (rb - a.rb0[p]) + (lane & 15), &wi, &row);
    const int g = 16 * t + 4 * (w >> 1) + (lane >> 4);
    uint32_t o[4] = {0, 0, 0, 0};
    if (row >= 0 && g < G) {
      const uint32_t* src = a.w[wi] + row * (a.K >> 3) + 8 * g + 4 * (w & 1);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t v = src[q];
        uint32_t r = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c)
          r |= ((v >> (8 * c)) & 0xfu) << (4 * c) | ((v >> (8 * c + 4)) & 0xfu) << (16 + 4 * c);
        o[q] = r;
      }
    }
    codes[idx] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

__global__ void q4_gemv_pack_sb(GvPackArgs a, uint32_t* __restrict__ sb) {
  const int64_t total = (int64_t)a.nrb * a.nt * 256;
  const int G = a.K >> 6;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int i = idx & 3, L = (idx >> 2) & 63;
    const int64_t tb = idx >> 8;
    const int t = tb % a.nt, rb = tb / a.nt;
    const int p = gv_problem(a, rb);
    int wi;
    int64_t row;
    gv_source(a, p, 16 * (rb - a.rb0[p]) + 4 * (L >> 4) + i, &wi, &row);
    const int g = 16 * t + (L & 15);
    uint32_t v = 0;
    if (row >= 0 && g < G) {
      const int64_t si = row * G + g;
      v = (uint32_t)a.s[wi][si] | ((uint32_t)a.b[wi][si] << 16);
    }
    sb[idx] = v;
  }
}

// Batch-1 launches with fewer than kGvHalfTaskWaves task waves run half
// tasks (HT = 2): twice the waves, each with half the load-to-store chain.
constexpr int64_t kGvHalfTaskWaves = 4096;

template <int MP, int EPI, bool NORM, typename YT, int NTC, int HT>
void launch_one(const uint16_t* x, const GvArgs& a, int nrb, hipStream_t st) {
  constexpr int MM = MP == 0 ? 1 : 4;
  const int waves = a.nt * HT;
  const size_t lds = (size_t)waves * (kWaveLds<MM> + MM * 64 + MM * 4);
  const int grid = a.pair ? 2 * ((nrb + 7) / 8 * 8) : nrb;
  hipLaunchKernelGGL((q4_gemv_mfma_kernel<MP, EPI, NORM, YT, NTC, HT>), dim3(grid), dim3(64 * waves),
                     lds, st, x, a.codes, a.sb, NORM ? a.norm_w : nullptr, a.M, a.K, a.nt, a);
}

template <int MP, int EPI, bool NORM, typename YT>
void launch_gv(const uint16_t* x, const GvArgs& a, int nrb, hipStream_t st) {
  const bool half = MP == 0 && (int64_t)nrb * a.nt < kGvHalfTaskWaves;
  if (a.nt == 4) {
    if (half) launch_one<MP, EPI, NORM, YT, 4, MP == 0 ? 2 : 1>(x, a, nrb, st);
    else launch_one<MP, EPI, NORM, YT, 4, 1>(x, a, nrb, st);
    return;
  }
  if (a.nt == 14 && !NORM) {
    launch_one<MP, EPI, NORM, YT, 14, 1>(x, a, nrb, st);
    return;
  }
  // the 3B widths (3072, and 8192 for down); the batched kernels need the
  // small block's register budget too (the generic 1024-thread bound spills)
  if (a.nt == 3) {
    if (half) launch_one<MP, EPI, NORM, YT, 3, MP == 0 ? 2 : 1>(x, a, nrb, st);
    else launch_one<MP, EPI, NORM, YT, 3, 1>(x, a, nrb, st);
    return;
  }
  if (a.nt == 8 && !NORM) {
    if (half) launch_one<MP, EPI, NORM, YT, 8, MP == 0 ? 2 : 1>(x, a, nrb, st);
    else launch_one<MP, EPI, NORM, YT, 8, 1>(x, a, nrb, st);
    return;
  }
  launch_one<MP, EPI, NORM, YT, 0, 1>(x, a, nrb, st);
}

template <int EPI, bool NORM, typename YT>
void launch_gv_m(const uint16_t* x, const GvArgs& a, int nrb, hipStream_t st) {
  if (a.M == 1) {
    launch_gv<0, EPI, NORM, YT>(x, a, nrb, st);
  } else if (a.M <= 4) {
    launch_gv<1, EPI, NORM, YT>(x, a, nrb, st);
  } else {  // 5-8 rows: paired 4-row workgroups
    GvArgs b = a;
    b.pair = 1;
    launch_gv<1, EPI, NORM, YT>(x, b, nrb, st);
  }
}

}  // namespace

bool strata_gemv_layout_fits(int K, int M) {
  return K > 0 && K % 64 == 0 && K <= 16384 && M >= 1 && M <= kGvMaxRows;
}

int strata_gemv_layout_build(const strata_q4_weight* ws, int count, int K, int perm, int head_dim,
                             GemvLayout* out, void* stream) {
  STRATA_REQUIRE(ws && out && count >= 1 && count <= kGvMaxProblems, "GEMV layout: bad arguments");
  STRATA_REQUIRE(K > 0 && K % 64 == 0 && K <= 16384, "GEMV layout: K=%d must be a multiple of 64, at most 16384", K);
  GvPackArgs pa{};
  GemvLayout L{};
  L.K = K;
  L.nt = (K + 1023) / 1024;
  L.perm = perm;
  L.head_dim = head_dim;
  int rbs = 0;
  if (perm == 1) {
    STRATA_REQUIRE(count == 2 && ws[0].N == ws[1].N, "GEMV layout: gate/up pairs need two equal linears");
    L.count = 1;
    L.N[0] = ws[0].N;
    L.rb0[0] = 0;
    rbs = (int)((ws[0].N + 7) / 8);
  } else {
    if (perm == 2)
      STRATA_REQUIRE(head_dim % 16 == 0 && head_dim > 0, "GEMV layout: head_dim %d must be a multiple of 16", head_dim);
    L.count = count;
    for (int i = 0; i < count; ++i) {
      if (perm == 2) STRATA_REQUIRE(ws[i].N % head_dim == 0, "GEMV layout: rows must be whole heads");
      L.rb0[i] = rbs;
      L.N[i] = ws[i].N;
      rbs += (int)((ws[i].N + 15) / 16);
    }
  }
  L.rb0[L.count] = rbs;
  L.nrb = rbs;
  for (int i = 0; i < count; ++i) {
    STRATA_REQUIRE(ws[i].w && ws[i].scales && ws[i].biases, "GEMV layout: null weight");
    pa.w[i] = ws[i].w;
    pa.s[i] = ws[i].scales;
    pa.b[i] = ws[i].biases;
    pa.n[i] = ws[i].N;
  }
  for (int i = 0; i <= L.count; ++i) pa.rb0[i] = L.rb0[i];
  pa.count = L.count;
  pa.perm = perm;
  pa.head_dim = head_dim;
  pa.K = K;
  pa.nt = L.nt;
  pa.nrb = L.nrb;
  L.code_bytes = (size_t)L.nrb * L.nt * 512 * 16;
  L.sb_bytes = (size_t)L.nrb * L.nt * 256 * 4;
  if (hipMalloc(&L.buf, L.code_bytes + L.sb_bytes) != hipSuccess) {
    (void)hipGetLastError();
    return strata_set_error(STRATA_ENOMEM, "GEMV layout: allocation of %zu bytes failed",
                            L.code_bytes + L.sb_bytes);
  }
  hipStream_t st = as_stream(stream);
  uint4* codes = static_cast<uint4*>(L.buf);
  uint32_t* sb = reinterpret_cast<uint32_t*>(static_cast<char*>(L.buf) + L.code_bytes);
  hipLaunchKernelGGL(q4_gemv_pack_codes, dim3(2048), dim3(256), 0, st, pa, codes);
  hipLaunchKernelGGL(q4_gemv_pack_sb, dim3(1024), dim3(256), 0, st, pa, sb);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    (void)hipFree(L.buf);
    return strata_set_error(STRATA_EHIP, "GEMV layout: pack launch failed: %s", hipGetErrorString(e));
  }
  *out = L;
  return STRATA_OK;
}

void strata_gemv_layout_free(GemvLayout* L) {
  if (L && L->buf) (void)hipFree(L->buf);
  if (L) L->buf = nullptr;
}

int strata_gemv_layout_run(const GemvLayout& L, const void* x, int M, void* const* ys, int y_dtype,
                           const GemvEpilogue* e, void* stream) {
  STRATA_REQUIRE(L.buf != nullptr, "GEMV layout: not built");
  STRATA_REQUIRE(M >= 1 && M <= kGvMaxRows, "GEMV layout: M=%d outside 1..%d", M, kGvMaxRows);
  STRATA_REQUIRE(x != nullptr && ys != nullptr, "GEMV layout: null x/y");
  GvArgs a{};
  a.codes = static_cast<const uint4*>(L.buf);
  a.sb = reinterpret_cast<const uint4*>(static_cast<const char*>(L.buf) + L.code_bytes);
  a.M = M;
  a.K = L.K;
  a.nt = L.nt;
  a.nrb = L.nrb;
  a.count = L.count;
  for (int i = 0; i < L.count; ++i) {
    a.p[i].y = ys[i];
    a.p[i].n = L.N[i];
    a.p[i].rb0 = L.rb0[i];
  }
  const int mode = e ? e->mode : 0;
  const bool norm = e && e->norm_w;
  if (e) {
    a.head_dim = e->head_dim;
    a.n_heads = e->n_heads;
    a.n_kv_heads = e->n_kv_heads;
    a.lmax = e->lmax;
    a.pos0 = e->pos0;
    a.dpos = e->dpos;
    a.rope_table = e->rope_table;
    a.rope_cur = e->rope_cur;
    a.q_out = e->q_out;
    a.kc = e->kc;
    a.vc = e->vc;
    a.norm_w = e->norm_w;
    a.eps = e->eps;
  }
  STRATA_REQUIRE(mode == 0 || y_dtype == STRATA_BF16,
                 "GEMV layout: the fused epilogues write bf16 (y_dtype %d)", y_dtype);
  STRATA_REQUIRE((mode == 1) == (L.perm == 1) && (mode == 2) == (L.perm == 2),
                 "GEMV layout: epilogue %d does not match the layout's row order %d", mode, L.perm);
  if (mode == 2)
    STRATA_REQUIRE(L.count == 3 && a.head_dim == L.head_dim && a.rope_table &&
                       (a.dpos == nullptr || a.rope_cur != nullptr),
                   "GEMV layout: RoPE epilogue needs q/k/v and the (cos, sin) table");
  const uint16_t* xx = static_cast<const uint16_t*>(x);
  hipStream_t st = as_stream(stream);
  const int nrb = L.nrb;
  if (mode == 0 && y_dtype == STRATA_F32) {
    if (norm) launch_gv_m<GV_STORE, true, float>(xx, a, nrb, st);
    else launch_gv_m<GV_STORE, false, float>(xx, a, nrb, st);
  } else if (mode == 0) {
    if (norm) launch_gv_m<GV_STORE, true, bf16_t>(xx, a, nrb, st);
    else launch_gv_m<GV_STORE, false, bf16_t>(xx, a, nrb, st);
  } else if (mode == 1) {
    if (norm) launch_gv_m<GV_SILU, true, bf16_t>(xx, a, nrb, st);
    else launch_gv_m<GV_SILU, false, bf16_t>(xx, a, nrb, st);
  } else if (mode == 2) {
    if (norm) launch_gv_m<GV_ROPE, true, bf16_t>(xx, a, nrb, st);
    else launch_gv_m<GV_ROPE, false, bf16_t>(xx, a, nrb, st);
  } else {
    STRATA_REQUIRE(!norm, "GEMV layout: no RMSNorm prologue on the residual epilogue");
    launch_gv_m<GV_RESID, false, bf16_t>(xx, a, nrb, st);
  }
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}
