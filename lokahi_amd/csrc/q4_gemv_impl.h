// Kernel templates and launchers of the q4 / bf16 GEMV (included by the
// q4_gemv*.hip translation units, which instantiate disjoint subsets).
#pragma once
// Decode-side quantized (q4 affine, group 64) and bf16 matrix-vector kernels.
//
// y[m, n] = sum_k x[m, k] * (s[n, k/64] * q[n, k] + b[n, k/64])
// (mx.quantized_matmul(transpose=True), src/ollm/llama_mlx.py:53-74)
//
// Design (HBM-bound streaming, gfx950 wave64):
//   * x for MT batch rows is staged once per workgroup into LDS, already
//     rearranged into bf16 pairs (x[8j+c], x[8j+c+4]) so that one AND-OR of a
//     packed word with the magic 0x43004300 yields the matching bf16 pair
//     (128+q[8j+c], 128+q[8j+c+4]) exactly; v_dot2_f32_bf16 then accumulates
//     x*(128+q) in fp32.  Per 32-element half group the offset is removed
//     with the precomputed LDS sum X = sum x:
//         acc += s * D + (b - 128 s) * X
//   * every lane streams one 16-byte uint4 (32 codes) per row per step, so a
//     wave reads 1 KiB contiguous per row per step (fully coalesced), R rows
//     at once to keep R*16 B per lane in flight and reuse the x reads;
//   * one workgroup per row block; every lane issues all of its weight loads
//     for a K chunk before it touches LDS, so thousands of waves keep the HBM
//     queues full; several linears that share x (q/k/v, gate/up) are one
//     launch ("problems" concatenated by row).
//   * lanes reduce with xor-butterflies at the end; results are deterministic.
#include <algorithm>
#include <cstdlib>

#include "strata_internal.h"

namespace {

constexpr int kMaxProblems = 8;
constexpr uint32_t kMagicPair = 0x43004300u;  // bf16 (128.0, 128.0)

struct Q4Problem {
  const uint4* w;      // [n, K/32] uint4  (== uint32 [n, K/8])
  const uint16_t* s;   // [n, K/64] bf16
  const uint16_t* b;   // [n, K/64] bf16
  void* y;             // [M, n]
  int n;
  int row0;
};

// Epilogues (decode engine), chosen by Q4Batch::epi:
//   EPI_STORE     : y[m, n] = bf16/fp32(acc)
//   EPI_SILU_PAIR : problems 0/1 = gate/up with rows interleaved (row 2n is
//                   gate n, row 2n+1 is up n, both in one wave); writes
//                   y0[m, n] = bf16(silu(bf16(gate)) * bf16(up))
//                   (llama_mlx.py:399-407) - the gate/up outputs never
//                   leave registers;
//   EPI_ROPE_KV   : problems 0/1/2 = q/k/v; inside each head the rows are
//                   ordered (0, D/2, 1, D/2+1, ...) so a wave holds a RoPE
//                   pair; writes rotated q head-major to q_out, rotated k and
//                   v into the KV cache at the step's position
//                   (llama_mlx.py:271-297; values are rounded to bf16 before
//                   RoPE, as the separate kernels do).
//   EPI_RESID     : the single problem's y is the residual stream h [M, n]:
//                   h[m, n] = bf16(h[m, n] + bf16(acc)) in place
//                   (llama_mlx.py:647, 653); only the lane that owns row n
//                   touches h[m, n] in the launch.
//   EPI_ROPE_KV_DEV: EPI_ROPE_KV with the position in device memory (dpos,
//                   graph-replayed steps) and its (cos, sin) row staged in
//                   rope_cur; a separate kernel, so the position load needs
//                   no runtime branch.
enum { EPI_STORE = 0, EPI_SILU_PAIR = 1, EPI_ROPE_KV = 2, EPI_RESID = 3, EPI_ROPE_KV_DEV = 4 };
template <int EPI>
constexpr bool kRopeEpi = EPI == EPI_ROPE_KV || EPI == EPI_ROPE_KV_DEV;

// Optional RMSNorm prologue (llama_mlx.py:77-92): x is replaced by
// bf16(w * (x * r)), r = 1/sqrt(mean(x^2) + eps) per batch row, before it is
// staged.
struct NormArgs {
  const uint16_t* w;  // [K] bf16
  float eps;
};

struct Q4Batch {
  Q4Problem p[kMaxProblems];
  int count;
  int total_rows;
  int epi;
  // EPI_ROPE_KV
  int head_dim, n_heads, n_kv_heads, lmax, pos0;
  const int* dpos;  // device position (graph-replayed step) or nullptr
  // with dpos: (cos, sin) [head_dim/2] of the position *dpos, staged by the
  // step that advanced it, so the RoPE operands need no dependent load
  const float2* rope_cur;
  float theta;
  const float2* rope_table;  // [lmax][head_dim/2] (cos, sin) of every cache position
  uint16_t* q_out;  // [M, Hq, 1, D] bf16
  uint16_t* kc;     // cache layer [M, Hkv, lmax, D] bf16
  uint16_t* vc;
};

// (w & 0x000f000f) | 0x43004300 as one v_and_or_b32: gfx9 VOP3 reads at most
// one scalar/literal operand, so the mask is passed in a VGPR (`mask_v`,
// hoisted out of the loops) and the magic as the scalar operand; written
// in C the pair becomes a separate AND and OR.
__device__ __forceinline__ uint32_t nib_pair(uint32_t w, uint32_t mask_v) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(w), "v"(mask_v), "s"(kMagicPair));
  return r;
}

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

template <typename YT>
__device__ __forceinline__ void store_y(void* y, int64_t idx, float v) {
  Elem<YT>::store(reinterpret_cast<YT*>(y), idx, v);
}

// Stage MT rows of x (bf16 or f32) into LDS.
//   bf16: xq[(mm*4 + j) * nv + i] = uint4 of the 4 bf16 pairs of word 4i+j,
//         xs[mm * nv + i]         = sum of the 32 x values of uint4 i.
//   f32 : xf[(mm*8 + c) * nv + i] = float4 of elements 32i+4c .. 32i+4c+3,
//         xs as above.
template <typename XT, int MT>
__device__ __forceinline__ void stage_x(const XT* __restrict__ x, int M, int K, int m0,
                                        uint4* smem, int nv) {
  float* xs;
  if constexpr (sizeof(XT) == 2) {
    uint4* xq = smem;
    xs = reinterpret_cast<float*>(smem + MT * 4 * nv);
    for (int idx = threadIdx.x; idx < MT * nv; idx += blockDim.x) {
      const int mm = idx / nv, i = idx - mm * nv;
      const int m = m0 + mm;
      float sum = 0.f;
      // rows past M read row M-1 (in bounds) and are zeroed after the loads
      const uint4* xr = reinterpret_cast<const uint4*>(x) + ((int64_t)min(m, M - 1) * K + (int64_t)i * 32) / 8;
      uint4 vv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) vv[j] = xr[j];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 v = m < M ? vv[j] : make_uint4(0, 0, 0, 0);
        uint4 pr;
        pr.x = (v.x & 0xffffu) | (v.z << 16);
        pr.y = (v.x >> 16) | (v.z & 0xffff0000u);
        pr.z = (v.y & 0xffffu) | (v.w << 16);
        pr.w = (v.y >> 16) | (v.w & 0xffff0000u);
        xq[(mm * 4 + j) * nv + i] = pr;
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int c = 0; c < 4; ++c)
          sum += __uint_as_float(u[c] << 16) + __uint_as_float(u[c] & 0xffff0000u);
      }
      xs[mm * nv + i] = sum;
    }
  } else {
    float4* xf = reinterpret_cast<float4*>(smem);
    xs = reinterpret_cast<float*>(smem + MT * 8 * nv);
    for (int idx = threadIdx.x; idx < MT * nv; idx += blockDim.x) {
      const int mm = idx / nv, i = idx - mm * nv;
      const int m = m0 + mm;
      float sum = 0.f;
      const float4* xr = reinterpret_cast<const float4*>(x + (int64_t)m * K + (int64_t)i * 32);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (m < M) v = xr[c];
        xf[(mm * 8 + c) * nv + i] = v;
        sum += (v.x + v.y) + (v.z + v.w);
      }
      xs[mm * nv + i] = sum;
    }
  }
}

// One workgroup = NW waves, persistent over row blocks (grid-stride).  x is
// staged into LDS once per workgroup behind the only barrier; after that each
// wave streams its rows with no synchronization: per row block it issues all
// R*U 16-byte weight loads (and their scales/biases, held in full 32-bit
// registers so no load waits on another), then computes.  The wave index is
// made wave-uniform (readfirstlane) so row/problem bookkeeping is scalar.
// bf16 x staging split in two so its global loads can be issued before the
// weight loads and written to LDS after them.  Thread t owns x items
// t, t + blockDim.x (XI of them); an item is the 32 x values of one weight
// uint4 position i of batch row mm.
template <int MT, int XI>
struct XStage {
  uint4 v[XI][4];
  uint4 wn[XI][4];  // RMSNorm weights of the same items (NORM kernels)
};

// x items (and, for the RMSNorm prologue, the norm weights of the same
// items) are loaded before the weight stream is issued: loads return in
// order, so anything issued after the weights would wait for all of them.
template <int MT, int XI, bool NORM = false>
__device__ __forceinline__ void xstage_load(XStage<MT, XI>& st, const uint16_t* __restrict__ x,
                                            int M, int K, int m0, int nv,
                                            const uint16_t* __restrict__ norm_w = nullptr) {
#pragma unroll
  for (int k = 0; k < XI; ++k) {
    const int raw = threadIdx.x + k * blockDim.x;
    const int idx = min(raw, MT * nv - 1);
    const int mm = idx / nv, i = idx - mm * nv;
    const int m = min(m0 + mm, M - 1);  // rows past M are zeroed at store time
    const uint4* xr = reinterpret_cast<const uint4*>(x + (int64_t)m * K + (int64_t)i * 32);
    // Without the RMSNorm prologue, threads without an item load nothing
    // (their staged values are unused, see xstage_store); the prologue reads
    // every thread's values unconditionally, which keeps its loads ahead of
    // the weight stream, and measured faster with all threads loading.
    if (NORM || raw < MT * nv) {
#pragma unroll
      for (int j = 0; j < 4; ++j) st.v[k][j] = xr[j];
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) st.v[k][j] = make_uint4(0, 0, 0, 0);
    }
    if constexpr (NORM) {
      const uint4* wr = reinterpret_cast<const uint4*>(norm_w) + i * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) st.wn[k][j] = wr[j];
    }
  }
}

// Without the RMSNorm prologue every thread stores: threads past the item
// count write into a per-lane sink after the staged x (kXSinkBytes), so no
// two lanes of a wave write one LDS address.  A conditional store would let
// the compiler sink the x loads into it, behind the weight loads (which
// return first: loads complete in order).  With the prologue the x values
// are consumed before the store, and threads past the item count skip it.
constexpr int kXSinkBytes = 16 + 64 * (4 * 16 + 4);  // alignment pad + per-lane sink
template <int MT, int XI, bool NORM>
__device__ __forceinline__ void xstage_store(const XStage<MT, XI>& st, int M, int m0, int nv,
                                             uint4* smem) {
  uint4* xq = smem;
  float* xs = reinterpret_cast<float*>(smem + MT * 4 * nv);
  uint4* sink_q = smem + MT * 4 * nv + (MT * nv + 3) / 4;  // first 16-byte slot after xs
  float* sink_s = reinterpret_cast<float*>(sink_q + 4 * 64);
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 0; k < XI; ++k) {
    const int raw = threadIdx.x + k * blockDim.x;
    const bool item = raw < MT * nv;
    if (NORM && !item) break;
    const int idx = min(raw, MT * nv - 1);
    const int mm = idx / nv, i = idx - mm * nv;
    const bool live = m0 + mm < M;
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint4 v = live ? st.v[k][j] : make_uint4(0, 0, 0, 0);
      uint4 pr;
      pr.x = (v.x & 0xffffu) | (v.z << 16);
      pr.y = (v.x >> 16) | (v.z & 0xffff0000u);
      pr.z = (v.y & 0xffffu) | (v.w << 16);
      pr.w = (v.y >> 16) | (v.w & 0xffff0000u);
      *(item ? &xq[(mm * 4 + j) * nv + i] : &sink_q[j * 64 + lane]) = pr;
      const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int c = 0; c < 4; ++c)
        sum += __uint_as_float(u[c] << 16) + __uint_as_float(u[c] & 0xffff0000u);
    }
    *(item ? &xs[mm * nv + i] : &sink_s[lane]) = sum;
  }
}

// RMSNorm of the staged x items held in registers (bf16 x, split staging).
// Every workgroup computes r for each of its batch rows (one block
// reduction) and rewrites its items as bf16(w * (x * r)); products are
// rounded one at a time, as in the standalone RMSNorm kernel.
template <int NW, int MT, int XI>
__device__ __forceinline__ void xstage_norm(XStage<MT, XI>& st, int M, int K, int m0, int nv,
                                            const NormArgs& na) {
  __shared__ float red[NW][MT];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float ss[MT];
#pragma unroll
  for (int mm = 0; mm < MT; ++mm) ss[mm] = 0.f;
#pragma unroll
  for (int k = 0; k < XI; ++k) {
    const int idx = threadIdx.x + k * blockDim.x;
    const int ic = min(idx, MT * nv - 1);
    const int mm = ic / nv;
    const bool live = idx < MT * nv && m0 + mm < M;
    float sq = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t u[4] = {st.v[k][j].x, st.v[k][j].y, st.v[k][j].z, st.v[k][j].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float lo = __uint_as_float(u[c] << 16), hi = __uint_as_float(u[c] & 0xffff0000u);
        sq = fmaf(lo, lo, sq);
        sq = fmaf(hi, hi, sq);
      }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t)
      if (live && t == mm) ss[t] += sq;
  }
#pragma unroll
  for (int mm = 0; mm < MT; ++mm) {
    const float t = wave_sum(ss[mm]);
    if (lane == 0) red[wave][mm] = t;
  }
  __syncthreads();
  float rr[MT];
#pragma unroll
  for (int mm = 0; mm < MT; ++mm) {
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) tot += red[w][mm];
    rr[mm] = 1.0f / sqrtf(tot / static_cast<float>(K) + na.eps);
  }
#pragma unroll
  for (int k = 0; k < XI; ++k) {
    const int idx = min((int)(threadIdx.x + k * blockDim.x), MT * nv - 1);
    const int mm = idx / nv;
    float r = rr[0];
#pragma unroll
    for (int t = 1; t < MT; ++t)
      if (t == mm) r = rr[t];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t* u = reinterpret_cast<uint32_t*>(&st.v[k][j]);
      const uint32_t wu[4] = {st.wn[k][j].x, st.wn[k][j].y, st.wn[k][j].z, st.wn[k][j].w};
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

// One workgroup = NW waves = one block of NW*R rows; wave w owns R rows.
// Order of work: x loads, then every weight/scale/bias load of the first K
// chunk (16-byte non-temporal loads, unconditional with clamped in-bounds
// addresses so none sits behind a branch), then x is written to LDS while the
// weights are still in flight, one barrier, the math, the store.
//
// Batch-1 kernels (MT == 1, bf16 x in one staging round) with short row
// chunks (U <= 2) in the shapes listed by kFiveWaves fit 96 VGPRs without
// spills: they are built for 5 waves per SIMD and launched 5 workgroups per
// CU (the extra wave per SIMD hides more load latency).  XI > 0
// selects that split staging (bf16 x); XI == 0 stages x up front (fp32 x).
// EPI picks the epilogue at compile time; NORM (XI > 0 only) applies the
// RMSNorm prologue to x.
template <int NW, int R, int U, int MT, int XI, int EPI, typename XT>
constexpr bool kFiveWaves = sizeof(XT) == 2 && XI == 1 && MT == 1 && U <= 2 &&
                            (R == 1 || (NW == 4 && R == 2 && (EPI == EPI_STORE || EPI == EPI_SILU_PAIR)));

template <int NW, int R, int U, int MT, int XI, int EPI, bool NORM, typename XT, typename YT>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(kFiveWaves<NW, R, U, MT, XI, EPI, XT> ? 5 : 1)))
void q4_gemv_kernel(const XT* __restrict__ x, int M, int K,
                                                          Q4Batch batch, NormArgs na) {
  static_assert(!NORM || XI > 0, "the RMSNorm prologue needs split bf16 staging");
  static_assert((EPI != EPI_SILU_PAIR && !kRopeEpi<EPI>) || R == 2,
                "pair epilogues need two rows per wave");
  extern __shared__ uint4 smem[];
  const int nv = K >> 5;  // uint4 (32 codes) per weight row
  const int m0 = blockIdx.y * MT;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const float* xs = reinterpret_cast<const float*>(smem + MT * (sizeof(XT) == 2 ? 4 : 8) * nv);

  const uint4* wp[R];
  const uint16_t* sp[R];
  const uint16_t* bp[R];
  int pid[R], nloc[R];
  bool valid[R];
  // Row block blk = NW*R rows: wave w owns rows (blk*NW + w)*R + r.
  const int nblk = (batch.total_rows + NW * R - 1) / (NW * R);
  int blk = blockIdx.x;
  // Epilogue operands are fetched with the block's weights, not at the tail:
  // the RoPE position and (cos, sin) of the block's pair, and the residual
  // values h[m, n] the RESID epilogue adds to.
  // EPI_ROPE_KV_DEV (graph-replayed step): the (cos, sin) pair comes from
  // the staged row rope_cur, and the position, needed only for the KV-append
  // address, is read after the weight loads are issued (load_rope_pos).  It
  // is a vector load from the global address space (a zero offset held in a
  // VGPR keeps it off the scalar path): a generic or scalar load counts on the
  // LDS wait counter too, so every wave would stall on it before issuing its
  // x and weight loads or in the RMSNorm prologue's LDS waits.
  // EPI_ROPE_KV: the position is the argument pos0.
  int rope_pos = 0;
  if constexpr (EPI == EPI_ROPE_KV) rope_pos = batch.pos0;
  auto load_rope_pos = [&]() {
    if constexpr (EPI == EPI_ROPE_KV_DEV) {
      using gint = const __attribute__((address_space(1))) int;
      int zero;
      asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
      rope_pos = ((gint*)batch.dpos)[zero];
    }
  };
  float2 cs_pre = make_float2(0.f, 0.f);
  uint16_t h_pre[R][MT];
  auto setup = [&](int b) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = (b * NW + wave) * R + r;
    valid[r] = row < batch.total_rows;
    int pi = 0, n = 0;
    if constexpr (EPI == EPI_SILU_PAIR) {
      pi = row & 1;
      n = valid[r] ? row >> 1 : 0;
    } else {
#pragma unroll
      for (int t = 1; t < kMaxProblems; ++t)
        if (t < batch.count && row >= batch.p[t].row0) pi = t;
      n = valid[r] ? row - batch.p[pi].row0 : 0;
      if constexpr (kRopeEpi<EPI>) {  // (h, 2p + w) -> h*D + p + w*D/2
        const int D = batch.head_dim, j = n % D;
        n = n - j + (j >> 1) + (j & 1) * (D >> 1);
      }
    }
    pid[r] = pi;
    nloc[r] = n;
    wp[r] = batch.p[pi].w + (int64_t)n * nv;
    sp[r] = batch.p[pi].s + (int64_t)n * (nv >> 1);
    bp[r] = batch.p[pi].b + (int64_t)n * (nv >> 1);
    if constexpr (EPI == EPI_RESID) {
#pragma unroll
      for (int mm = 0; mm < MT; ++mm) {
        const int m = min(m0 + mm, M - 1);
        h_pre[r][mm] = reinterpret_cast<const uint16_t*>(batch.p[pi].y)[(int64_t)m * batch.p[pi].n + n];
      }
    }
  }
  };
  // Issued after the block's weight loads, so they do not queue behind it.
  auto prefetch_rope = [&]() {
    if constexpr (kRopeEpi<EPI>) {
      const int D = batch.head_dim, i = min(nloc[0] % D, (D >> 1) - 1);  // pair (i, i + D/2)
      if constexpr (EPI == EPI_ROPE_KV_DEV)
        cs_pre = batch.rope_cur[i];
      else
        cs_pre = batch.rope_table[(int64_t)rope_pos * (D >> 1) + i];
    }
  };
  setup(blk);

  uint4 wv[R][U];
  uint32_t sv[R][U], bv[R][U];
  auto issue = [&](int c0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int ic = min(c0 + lane + 64 * u, nv - 1);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        wv[r][u] = load_nt(wp[r] + ic);
        sv[r][u] = sp[r][ic >> 1];
        bv[r][u] = bp[r][ic >> 1];
      }
    }
  };

  float acc[R][MT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) acc[r][mm] = 0.f;

  uint32_t nib_mask = 0x000f000fu;
  asm volatile("" : "+v"(nib_mask));  // keep the mask in a VGPR
  auto compute = [&](int c0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // A tail lane read a valid slot; zero scale and bias remove it.
      const bool tail = c0 + lane + 64 * u >= nv;
      const int i = min(c0 + lane + 64 * u, nv - 1);
#pragma unroll
      for (int mm = 0; mm < MT; ++mm) {
        const float xsum = xs[mm * nv + i];
        if constexpr (sizeof(XT) == 2) {
          const uint4* xq = smem;
          uint4 xa[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) xa[j] = xq[(mm * 4 + j) * nv + i];
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const uint32_t ww[4] = {wv[r][u].x, wv[r][u].y, wv[r][u].z, wv[r][u].w};
            float d = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const uint32_t w = ww[j];
              d = dot2_bf16(nib_pair(w, nib_mask), xa[j].x, d);
              d = dot2_bf16(nib_pair(w >> 4, nib_mask), xa[j].y, d);
              d = dot2_bf16(nib_pair(w >> 8, nib_mask), xa[j].z, d);
              d = dot2_bf16(nib_pair(w >> 12, nib_mask), xa[j].w, d);
            }
            const float sc = tail ? 0.f : __uint_as_float(sv[r][u] << 16);
            const float bc = tail ? 0.f : __uint_as_float(bv[r][u] << 16);
            acc[r][mm] = fmaf(sc, d, acc[r][mm]);
            acc[r][mm] = fmaf(fmaf(-128.f, sc, bc), xsum, acc[r][mm]);
          }
        } else {
          const float4* xf = reinterpret_cast<const float4*>(smem);
          float4 xa[8];
#pragma unroll
          for (int c = 0; c < 8; ++c) xa[c] = xf[(mm * 8 + c) * nv + i];
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const uint32_t ww[4] = {wv[r][u].x, wv[r][u].y, wv[r][u].z, wv[r][u].w};
            float d = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const uint32_t lo = ww[j] & 0x0f0f0f0fu;         // codes 0,2,4,6
              const uint32_t hi = (ww[j] >> 4) & 0x0f0f0f0fu;  // codes 1,3,5,7
              const float4 xa0 = xa[2 * j], xa1 = xa[2 * j + 1];
              d = fmaf(xa0.x, (float)(lo & 0xff), d);
              d = fmaf(xa0.y, (float)(hi & 0xff), d);
              d = fmaf(xa0.z, (float)((lo >> 8) & 0xff), d);
              d = fmaf(xa0.w, (float)((hi >> 8) & 0xff), d);
              d = fmaf(xa1.x, (float)((lo >> 16) & 0xff), d);
              d = fmaf(xa1.y, (float)((hi >> 16) & 0xff), d);
              d = fmaf(xa1.z, (float)(lo >> 24), d);
              d = fmaf(xa1.w, (float)(hi >> 24), d);
            }
            const float sc = tail ? 0.f : __uint_as_float(sv[r][u] << 16);
            const float bc = tail ? 0.f : __uint_as_float(bv[r][u] << 16);
            acc[r][mm] = fmaf(sc, d, acc[r][mm]);
            acc[r][mm] = fmaf(bc, xsum, acc[r][mm]);
          }
        }
      }
    }
  };

  if constexpr (XI > 0) {
    XStage<MT, XI> st;
    xstage_load<MT, XI, NORM>(st, reinterpret_cast<const uint16_t*>(x), M, K, m0, nv, na.w);
    issue(0);
    prefetch_rope();
    load_rope_pos();
    __builtin_amdgcn_sched_barrier(0);
    // x staging (and the RMSNorm) at raised wave priority: it gates every
    // wave's first compute, while the weights are still in flight
    // (GEMV set 30.7 -> 29.5 us, decode -2%)
    __builtin_amdgcn_s_setprio(1);
    if constexpr (NORM) xstage_norm<NW, MT, XI>(st, M, K, m0, nv, na);
    xstage_store<MT, XI, NORM>(st, M, m0, nv, smem);
    __builtin_amdgcn_s_setprio(0);
  } else {
    stage_x<XT, MT>(x, M, K, m0, smem, nv);
    issue(0);
    prefetch_rope();
    load_rope_pos();
  }
  __syncthreads();
  // Persistent over row blocks (grid-stride): x is staged once per
  // workgroup; the next block's first loads are issued before this block's
  // reduction and epilogue.
  for (;;) {
  compute(0);
  for (int c0 = 64 * U; c0 < nv; c0 += 64 * U) {
    __builtin_amdgcn_s_setprio(1);
    issue(c0);
    __builtin_amdgcn_s_setprio(0);
    compute(c0);
  }
  int e_pid[R], e_nloc[R];
  bool e_valid[R];
  uint16_t e_h[R][MT];
  const float2 e_cs = cs_pre;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    e_pid[r] = pid[r];
    e_nloc[r] = nloc[r];
    e_valid[r] = valid[r];
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) e_h[r][mm] = h_pre[r][mm];
  }
  const int next = blk + gridDim.x;
  const bool more = next < nblk;
  if (more) {
    // the next block's loads go out ahead of other waves' math on the SIMD
    __builtin_amdgcn_s_setprio(1);
    setup(next);
    issue(0);
    prefetch_rope();
    __builtin_amdgcn_s_setprio(0);
  }

#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) acc[r][mm] = wave_sum(acc[r][mm]);
  if constexpr (EPI == EPI_SILU_PAIR || kRopeEpi<EPI>) {
    {
#pragma unroll
      for (int mm = 0; mm < MT; ++mm) {
        const int m = m0 + mm;
        if (lane != mm || !e_valid[0] || m >= M) continue;
        const float a0 = bf16_to_f32(f32_to_bf16(acc[0][mm]));
        const float a1 = bf16_to_f32(f32_to_bf16(acc[1][mm]));
        if constexpr (EPI == EPI_SILU_PAIR) {
          const float sg = a0 / (1.0f + expf(-a0));
          const Q4Problem& p = batch.p[0];
          store_y<bf16_t>(p.y, (int64_t)m * p.n + e_nloc[0], mul_rn(sg, a1));
        } else {
          const int D = batch.head_dim, half = D >> 1;
          const int h = e_nloc[0] / D, i = e_nloc[0] - h * D;  // i < D/2: pair (i, i + D/2)
          const int pos = rope_pos;
          if (e_pid[0] == 2) {  // v: copy into the cache
            const int64_t co = (((int64_t)m * batch.n_kv_heads + h) * batch.lmax + pos) * D;
            batch.vc[co + i] = f32_to_bf16(a0);
            batch.vc[co + i + half] = f32_to_bf16(a1);
          } else {
            const float c = e_cs.x, sn = e_cs.y;
            float o1, o2;
            rotate_pair(a0, a1, c, sn, &o1, &o2);
            if (e_pid[0] == 0) {
              const int64_t qo = ((int64_t)m * batch.n_heads + h) * D;
              batch.q_out[qo + i] = f32_to_bf16(o1);
              batch.q_out[qo + i + half] = f32_to_bf16(o2);
            } else {
              const int64_t co = (((int64_t)m * batch.n_kv_heads + h) * batch.lmax + pos) * D;
              batch.kc[co + i] = f32_to_bf16(o1);
              batch.kc[co + i + half] = f32_to_bf16(o2);
            }
          }
        }
      }
    }
  } else {
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) {
      const int m = m0 + mm;
      if (lane == r * MT + mm && e_valid[r] && m < M) {
        const Q4Problem& p = batch.p[e_pid[r]];
        if constexpr (EPI == EPI_RESID) {
          uint16_t* hp = reinterpret_cast<uint16_t*>(p.y) + (int64_t)m * p.n + e_nloc[r];
          const float o = bf16_to_f32(f32_to_bf16(acc[r][mm]));
          *hp = f32_to_bf16(bf16_to_f32(e_h[r][mm]) + o);
        } else {
          store_y<YT>(p.y, (int64_t)m * p.n + e_nloc[r], acc[r][mm]);
        }
      }
    }
  }
  if (!more) break;
  blk = next;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) acc[r][mm] = 0.f;
  }
}

// Dense bf16-weight GEMV (lm_head): y[m,n] = sum_k x[m,k] * W[n,k]; same
// load-first structure, one uint4 = 8 weights per lane per step.  XI > 0:
// the MT*K/8 x items are exactly XI per thread and are loaded before the
// weight stream (loads return in order: x staged after the weights would
// wait for all of them); XI = 0 stages x after the first weight loads.
template <int NW, int R, int U, int MT, typename YT, int XI = 0>
__global__ __launch_bounds__(NW * 64) void bf16_gemv_kernel(const uint16_t* __restrict__ x, int M,
                                                            int K, const uint4* __restrict__ w,
                                                            int N, YT* __restrict__ y) {
  extern __shared__ uint4 smem[];
  const int nv = K >> 3;  // uint4 (8 bf16) per row
  const int m0 = blockIdx.y * MT;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * NW + wave) * R;
  float acc[R][MT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) acc[r][mm] = 0.f;
  uint4 xr[XI > 0 ? XI : 1];
  if constexpr (XI > 0) {
#pragma unroll
    for (int k = 0; k < XI; ++k) {
      const int idx = threadIdx.x + k * NW * 64;
      const int mm = idx / nv, i = idx - mm * nv;
      const int m = min(m0 + mm, M - 1);  // rows past M are zeroed at store time
      xr[k] = reinterpret_cast<const uint4*>(x + (int64_t)m * K)[i];
      if (m0 + mm >= M) xr[k] = make_uint4(0, 0, 0, 0);
    }
  }
  for (int c0 = 0; c0 < nv; c0 += 64 * U) {
    uint4 wv[R][U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = c0 + lane + 64 * u;
      const int ic = min(i, nv - 1);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        // unconditional, clamped load; rows past N are computed but never stored
        const uint4 t = load_nt(w + (int64_t)min(row0 + r, N - 1) * nv + ic);
        wv[r][u] = i < nv ? t : make_uint4(0, 0, 0, 0);
      }
    }
    if (c0 == 0) {
      if constexpr (XI > 0) {
#pragma unroll
        for (int k = 0; k < XI; ++k) smem[threadIdx.x + k * NW * 64] = xr[k];
      } else {
        for (int idx = threadIdx.x; idx < MT * nv; idx += blockDim.x) {
          const int mm = idx / nv, i = idx - mm * nv;
          const int m = m0 + mm;
          smem[idx] = (m < M) ? reinterpret_cast<const uint4*>(x + (int64_t)m * K)[i]
                              : make_uint4(0, 0, 0, 0);
        }
      }
      __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = min(c0 + lane + 64 * u, nv - 1);
#pragma unroll
      for (int mm = 0; mm < MT; ++mm) {
        const uint4 xa = smem[mm * nv + i];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float d = acc[r][mm];
          d = dot2_bf16(wv[r][u].x, xa.x, d);
          d = dot2_bf16(wv[r][u].y, xa.y, d);
          d = dot2_bf16(wv[r][u].z, xa.z, d);
          d = dot2_bf16(wv[r][u].w, xa.w, d);
          acc[r][mm] = d;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) acc[r][mm] = wave_sum(acc[r][mm]);
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) {
      const int m = m0 + mm;
      if (lane == r * MT + mm && row0 + r < N && m < M)
        Elem<YT>::store(y, (int64_t)m * N + row0 + r, acc[r][mm]);
    }
}

// Launch geometry of one GEMV: waves per workgroup, rows per wave, uint4 per
// lane per row per K chunk, batch rows per pass.
struct GemvShape {
  int nw, r, u, mt;
};

// Pick the geometry for `rows` output rows of `nv` uint4 each.  Aim: each
// lane holds ~8 outstanding 16-byte weight loads (R*U ~ 8) and the launch has
// several thousand waves; large-K rows use 8-wave workgroups so the x staged
// in LDS is shared by more rows.
GemvShape pick_shape(int nv, int rows, int M) {
  // Measured on MI355X (graph-replayed launches, weights cycled past the
  // 256 MB last-level cache): K=4096 rows prefer 4 waves x 2 rows with U=2,
  // small launches (< 8192 rows) 4 waves x 1 row (q/k/v 6.5 -> 5.8 us against
  // 8 waves x 1 row); batch-1 K=14336 prefers 8 waves x 1 row
  // with U=4 over two K chunks, one row block per workgroup (9.9 us against
  // 10.7 us for 4 waves with U=7 in one chunk).
  GemvShape g;
  const int chunks = (nv + 63) / 64;
  g.u = chunks <= 2 ? 2 : (chunks <= 4 ? 4 : (chunks <= 7 ? 7 : 8));
  g.mt = M >= 4 ? 4 : (M >= 2 ? 2 : 1);
  if (g.mt > 1) {
    g.r = 2;
    g.nw = 4;
  } else if (g.u == 2) {
    g.nw = 4;
    g.r = rows < 8192 ? 1 : 2;
  } else {
    g.nw = 8;
    g.r = 1;
    g.u = 4;
  }
  return g;
}

// Persistent grid size: workgroups per CU times CUs.  8-wave launches (small or long-row linears)
// get one row block per workgroup at the decode shapes; U >= 7 (batched
// long rows) runs three 4-wave workgroups per CU over several row blocks.
int g_num_cus = 256;
// Workgroups per CU of the persistent grid (five_waves: the kernel is built
// for 5 waves per SIMD).
int grid_cap(int nw, int u, bool norm, bool five_waves) {
  int per_cu = u >= 7 ? 3 : (nw >= 8 ? 6 : (five_waves ? 5 : 4));
  if (norm) {  // each workgroup normalizes x itself: 5 per CU measured best
    per_cu = 5;  // (with the prologue at raised wave priority; 4 before it)
  }
  return std::max(1, per_cu) * g_num_cus;
}

template <int NW, int R, int U, int MT, int XI, int EPI, bool NORM, typename XT, typename YT>
void launch_q4_x(const XT* x, int M, int K, const Q4Batch& batch, const NormArgs& na, size_t lds,
                 hipStream_t stream) {
  const int nblk = (batch.total_rows + NW * R - 1) / (NW * R);
  constexpr bool five = kFiveWaves<NW, R, U, MT, XI, EPI, XT>;
  dim3 grid(std::min(nblk, grid_cap(NW, U, NORM, five)), (M + MT - 1) / MT);
  hipLaunchKernelGGL((q4_gemv_kernel<NW, R, U, MT, XI, EPI, NORM, XT, YT>), grid, dim3(NW * 64),
                     lds, stream, x, M, K, batch, na);
}

template <int NW, int R, int U, int MT, int EPI, bool NORM, typename XT, typename YT>
void launch_q4_k(const void* x, int M, int K, const Q4Batch& batch, const NormArgs& na,
                 size_t lds, hipStream_t stream) {
  const int items = MT * (K / 32), threads = NW * 64;
  const XT* xx = reinterpret_cast<const XT*>(x);
  if (sizeof(XT) == 2 && items <= threads)
    launch_q4_x<NW, R, U, MT, 1, EPI, NORM, XT, YT>(xx, M, K, batch, na, lds, stream);
  else if (sizeof(XT) == 2 && items <= 2 * threads)
    launch_q4_x<NW, R, U, MT, 2, EPI, NORM, XT, YT>(xx, M, K, batch, na, lds, stream);
  else if constexpr (!NORM)
    launch_q4_x<NW, R, U, MT, 0, EPI, false, XT, YT>(xx, M, K, batch, na, lds, stream);
}

template <int NW, int R, int MT, int EPI, bool NORM, typename XT, typename YT>
bool launch_q4_u(const GemvShape& g, const void* x, int M, int K, const Q4Batch& batch,
                 const NormArgs& na, size_t lds, hipStream_t s) {
  // Kernels with the RMSNorm prologue or a pair epilogue run at the hidden
  // width only (K <= 8192, U <= 4); fp32 activations use U = 4.
  constexpr bool kSmall = NORM || EPI == EPI_SILU_PAIR || kRopeEpi<EPI>;
  constexpr bool kF32 = sizeof(XT) == 4;
  if (g.u == 2 && !kF32) {
    launch_q4_k<NW, R, 2, MT, EPI, NORM, XT, YT>(x, M, K, batch, na, lds, s);
    return true;
  }
  if (g.u == 4) {
    launch_q4_k<NW, R, 4, MT, EPI, NORM, XT, YT>(x, M, K, batch, na, lds, s);
    return true;
  }
  if constexpr (!kSmall && !kF32) {
    if (g.u == 7) {
      launch_q4_k<NW, R, 7, MT, EPI, NORM, XT, YT>(x, M, K, batch, na, lds, s);
      return true;
    }
    if (g.u == 8) {
      launch_q4_k<NW, R, 8, MT, EPI, NORM, XT, YT>(x, M, K, batch, na, lds, s);
      return true;
    }
  }
  return false;
}

// Geometry by shape (pick_shape); pair epilogues need R = 2 (4 waves); the
// RMSNorm prologue needs every staged x item in registers (<= 2 per thread).
template <int EPI, bool NORM, typename XT, typename YT>
int dispatch_q4(strata_ctx* ctx, const void* x, int M, int K, const Q4Batch& batch,
                const NormArgs& na, hipStream_t stream) {
  constexpr bool kPair = EPI == EPI_SILU_PAIR || kRopeEpi<EPI>;
  g_num_cus = ctx->num_cus;
  const int nv = K / 32;
  GemvShape g = pick_shape(nv, batch.total_rows, M);
  const size_t per_row = (size_t)nv * ((sizeof(XT) == 2 ? 64 : 128) + 4);
  while (g.mt > 1 && g.mt * per_row + kXSinkBytes > (size_t)ctx->max_lds_per_block) g.mt /= 2;
  const size_t lds = g.mt * per_row + kXSinkBytes;
  STRATA_REQUIRE((int64_t)lds <= ctx->max_lds_per_block,
                 "q4 GEMV: K=%d needs %zu B of LDS, device allows %d", K, lds,
                 ctx->max_lds_per_block);
  if (kPair || sizeof(XT) == 4 || g.mt > 1) {
    g.nw = 4;
    g.r = 2;
  }
  if (sizeof(XT) == 4) g.u = 4;
  if (NORM)
    STRATA_REQUIRE(g.mt * nv <= 2 * g.nw * 64,
                   "q4 GEMV: RMSNorm prologue supports K <= %d at batch %d", 2 * g.nw * 64 * 32 / g.mt,
                   M);
  bool ok = false;
  if (g.mt == 4) ok = launch_q4_u<4, 2, 4, EPI, NORM, XT, YT>(g, x, M, K, batch, na, lds, stream);
  else if (g.mt == 2) ok = launch_q4_u<4, 2, 2, EPI, NORM, XT, YT>(g, x, M, K, batch, na, lds, stream);
  else if (g.nw == 4 && g.r == 2) ok = launch_q4_u<4, 2, 1, EPI, NORM, XT, YT>(g, x, M, K, batch, na, lds, stream);
  else if constexpr (!kPair) {
    // (4 rows per wave, or 8 waves x 2 rows, spill registers at long rows and
    // never won a measurement: not built)
    if (g.nw == 4 && g.r == 1) ok = launch_q4_u<4, 1, 1, EPI, NORM, XT, YT>(g, x, M, K, batch, na, lds, stream);
    else if (g.nw == 8 && g.r == 1) ok = launch_q4_u<8, 1, 1, EPI, NORM, XT, YT>(g, x, M, K, batch, na, lds, stream);
  }
  if (!ok)
    return strata_set_error(STRATA_EINVAL, "q4 GEMV: no kernel for geometry nw=%d r=%d u=%d mt=%d",
                            g.nw, g.r, g.u, g.mt);
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}

// Concatenate several linears that share x into one launch's problem list.
inline Q4Batch make_batch(const strata_q4_weight* ws, int count, int epi) {
  Q4Batch batch{};
  batch.count = count;
  batch.epi = epi;
  int rows = 0;
  for (int i = 0; i < count; ++i) {
    batch.p[i].w = reinterpret_cast<const uint4*>(ws[i].w);
    batch.p[i].s = ws[i].scales;
    batch.p[i].b = ws[i].biases;
    batch.p[i].y = ws[i].y;
    batch.p[i].n = static_cast<int>(ws[i].N);
    batch.p[i].row0 = rows;
    rows += static_cast<int>(ws[i].N);
  }
  batch.total_rows = rows;
  return batch;
}

}  // namespace
