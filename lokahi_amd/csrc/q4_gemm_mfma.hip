// Prefill q4 GEMM for large M: Y[M, N] = X[M, K] @ dequant(W)[N, K]^T on
// bf16 MFMA, dequantizing in the kernel (no bf16 copy of the weight).
//
// Same maths as mx.quantized_matmul(transpose=True) on the prefill path
// (src/ollm/llama_mlx.py:53-74, 393-432): W[n, k] = s[n, k/64] * q + b[n, k/64],
// rounded once to bf16 (fp32 FMA, round-to-nearest-even), as MLX's qmm
// stages dequantized tiles in the activation dtype; fp32 accumulation.
//
// Workgroup tile 256 (M) x 256 (N), K step 64 = one quantization group.
// 4 waves, one per SIMD: wave w owns all 256 rows x columns 64w .. 64w+63,
// i.e. 16 x 4 blocks of v_mfma_f32_16x16x32_bf16 (256 fp32 accumulators per
// lane, in AGPRs).
//   * X tiles go through LDS: 256 x 64 bf16 (32 KB) per stage, 16-byte
//     chunks XOR-swizzled (chunk c of row r at c ^ ((r >> 1) & 7)) so the
//     MFMA operand reads of a 16-lane phase touch 64 distinct banks.
//   * Weights are dequantized in registers, straight into the B operand:
//     16x16x32 wants, per lane, 8 consecutive k of one weight row = one
//     packed uint32 word, so each wave handles exactly the words of its own
//     64 columns; each weight is dequantized once per workgroup (mask,
//     v_cvt_f32_ubyteN, FMA, v_cvt_pk_bf16_f32).
//   * Every global read is a direct global -> LDS buffer load (no VGPR
//     staging): the X tile, and each wave's own weight words, scales and
//     biases.  Three LDS stages; the loads of step g+2 are issued at the
//     top of step g, so they have ~1.5 steps to land.
//   * While the MFMAs of step g run, the wave dequantizes the fragments the
//     next MFMAs need (each k half is rewritten right after its last MFMA
//     of the step has issued), in fixed slots between the MFMAs.  One
//     barrier per K step.
//   * Workgroup order: tiles are dealt to the 8 XCDs in contiguous runs
//     (block b runs on XCD b % 8), grouped 4 M-tiles x N-tiles, so the
//     ~32 workgroups resident on one XCD share X and W tiles in its L2.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "strata_internal.h"

namespace {

constexpr int TN = 256, TK = 64;
constexpr int NTHR = 256;
constexpr int WN = 64;              // columns per wave
constexpr int NB = WN / 32;         // 32-column MFMA blocks per wave
constexpr int KB = TK / 16;         // 16-deep MFMA k blocks per K step
constexpr int kGroupM = 4;          // M tiles per group of the tile order

typedef float f32x16_t __attribute__((ext_vector_type(16)));

// 32x32x16 rather than 16x16x32: each instruction runs long enough for the
// VALU dequantization issued between MFMAs to overlap it (measured on
// MI355X: 2 VALU per 16x16x32 cost a third of the MFMA rate, 4 per
// 32x32x16 about 14%).
__device__ __forceinline__ f32x16_t mfma32(const uint4& a, const uint4& b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

template <int B>
__device__ __forceinline__ float ubyte(uint32_t v) {
  float r;
  if constexpr (B == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
  if constexpr (B == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
  if constexpr (B == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
  if constexpr (B == 3) asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
  return r;
}

// Tile index -> (m tile, n tile): groups of kGroupM M tiles sweeping the
// N tiles.
__device__ __forceinline__ void group_tile(int t, int mt, int nt, int* tm, int* tn) {
  const int per_group = kGroupM * nt;
  const int grp = t / per_group, rem = t - grp * per_group;
  const int gm = min(kGroupM, mt - grp * kGroupM);
  *tm = grp * kGroupM + rem % gm;
  *tn = rem / gm;
}

// LDS stage layout (bytes): X tile 256 x 128 (swizzled 16-byte chunks), then
// per wave its 64 weight rows x 32 bytes, then per wave 64 (s | b << 16)
// words.  Three stages: the loads of step g + 2 are issued at the top of
// step g.
constexpr int kWBytes = 4 * 64 * 32;             // 8 KB
constexpr int kSBBytes = 4 * 64 * 4;             // 1 KB
constexpr int kStages = 3;

// N % 256 == 0, K % 64 == 0, and every operand under 4 GiB (the launcher
// checks); any M.
// Per-M-tile constants: TM = 256 (one workgroup per CU) or 128 (two per
// CU, for problems with few 256-row tiles).
template <int TM>
struct Tile {
  static constexpr int MB = TM / 32;                    // 32-row MFMA blocks per wave
  static constexpr int XCH = TM * 8 / NTHR;             // X chunks (16 B) per thread per step
  static constexpr int kXBytes = TM * TK * 2;
  static constexpr int kStage = kXBytes + kWBytes + kSBBytes;
  static constexpr int kDmaPerStep = XCH + 2 + 1;       // per lane: X chunks, W halves, (s, b)
  static constexpr size_t kLds = (size_t)kStages * kStage;
};

// Outputs of the linears that share x, concatenated along N (each a
// multiple of 256 columns): problem p owns columns n0[p] .. n0[p + 1] of
// the re-laid-out weight and writes y[p] [M, n0[p + 1] - n0[p]].
struct GemmOut {
  void* y[kMaxGemmProblems];
  int n0[kMaxGemmProblems + 1];
  int count;
};

// The part of the problem space one launch covers: M tiles 0 .. mt - 1 (the
// last one may be partial: rows at or past M read as zero and are not
// stored), N tiles ntile0 .. ntile0 + nts - 1 of the re-laid-out weight, and
// S slices of the K groups.  With S > 1 each slice writes its fp32 partial
// sums to part [S][mt * TM][nts * 256] and q4_gemm_splitk_reduce adds them
// up in slice order.
struct GemmSplit {
  int mt, ntile0, nts, S;
  float* part;
};

// SPLIT: the launch's K slices write fp32 partial sums (sp.part) instead
// of the outputs; a separate instance, so the other one carries no partial
// pointer arithmetic (it spilled to scratch when it did).
template <int TM, typename YT, bool SPLIT>
__global__ __launch_bounds__(NTHR) __attribute__((amdgpu_waves_per_eu(TM == 256 ? 1 : 2, TM == 256 ? 1 : 2)))
void q4_gemm_mfma_kernel(const uint16_t* __restrict__ x, int M, int K,
                         const uint32_t* __restrict__ wt, const uint32_t* __restrict__ sbt,
                         int N, GemmOut out, GemmSplit sp) {
  constexpr int MB = Tile<TM>::MB, XCH = Tile<TM>::XCH, kXBytes = Tile<TM>::kXBytes;
  constexpr int kStage = Tile<TM>::kStage, kDmaPerStep = Tile<TM>::kDmaPerStep;
  constexpr int QPS = 8 / MB;  // dequant quarters per sub-step
  // Sub-step that reads step g + 1's code words and scales (after this
  // lane's loads of step g + 1 are waited for, which needs every load of
  // step g + 2 issued first).
  constexpr int kReadSt = 3 * MB - 4;
  static_assert(kReadSt - 1 >= kDmaPerStep - 1, "the load wait must follow step g + 2's issue");
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  // Workgroups are dealt to the 8 XCDs in contiguous runs of the (slice,
  // tile) order (block b runs on XCD b % 8), so a run shares its K slice.
  const int mt = sp.mt, nts = sp.nts, S = sp.S, tiles = mt * nts;
  int u = blockIdx.x;
  if ((tiles * S) % 8 == 0) u = (u % 8) * (tiles * S / 8) + u / 8;
  const int ks = u / tiles;
  int tmi, tnl;
  group_tile(u - ks * tiles, mt, nts, &tmi, &tnl);
  const int m0 = tmi * TM, n0 = (sp.ntile0 + tnl) * TN;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = K / TK;
  const int g0 = (int)((int64_t)ks * G / S), g1 = (int)((int64_t)(ks + 1) * G / S);
  const uint32_t kb = (uint32_t)K * 2;   // bytes per X row
  const uint32_t wgb = (uint32_t)N * 32;  // bytes per group of the re-laid-out codes
  const uint32_t sgb = (uint32_t)N * 4;   // bytes per group of (s, b) words
  const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) uint8_t*)lds);

  const v4i32_t rx = rsrc(x, (uint32_t)((size_t)M * kb));
  const v4i32_t rw = rsrc(wt, (uint32_t)((size_t)G * wgb));
  const v4i32_t rs = rsrc(sbt, (uint32_t)((size_t)G * sgb));

  // X DMA instruction i of wave w fills 16-byte slots S = (8w + i) * 64 + lane
  // of the stage: row r = S / 8, slot p = lane % 8 holds chunk
  // c = p ^ ((r >> 1) & 7) = (lane & 7) ^ (4 (i & 1) + (lane >> 4)).
  const uint32_t xl0 = (lane >> 3) * kb + (((lane & 7) ^ (lane >> 4)) << 4);
  const uint32_t xl1 = (lane >> 3) * kb + (((lane & 7) ^ (4 + (lane >> 4))) << 4);
  // W DMA j of this wave: 16-byte chunk q = 64 j + lane = row q/2, half q%2
  // of the group-major codes (rows of one group are 32 bytes apart).
  const uint32_t wl = lane * 16;
  const uint32_t sl = lane * 4;
  // DMA piece p (0 .. kDmaPerStep - 1) of step g into stage stg: X chunks
  // 0-7, the two weight halves, the scales, the biases.
  auto issue1 = [&](int g, int stg, int p) {
    const uint32_t base = lds0 + stg * kStage;
    if (p < XCH) {
      dma16(base + (wave * XCH + p) * 1024, (p & 1) ? xl1 : xl0, rx,
            (uint32_t)(m0 + (wave * XCH + p) * 8) * kb + g * TK * 2);
    } else if (p < XCH + 2) {
      const int j = p - XCH;
      dma16(base + kXBytes + wave * 2048 + j * 1024, wl, rw,
            g * wgb + (uint32_t)(n0 + wave * WN + j * 32) * 32);
    } else {
      dma4(base + kXBytes + kWBytes + wave * 256, sl, rs, g * sgb + (uint32_t)(n0 + wave * WN) * 4);
    }
  };
  auto issue = [&](int g, int stg) {
#pragma unroll
    for (int p = 0; p < kDmaPerStep; ++p) issue1(g, stg, p);
  };
  // Wait until at most N loads are outstanding (loads complete in order).
  auto vm_wait = [&](auto N) {
    asm volatile("s_waitcnt vmcnt(%0)" :: "n"(decltype(N)::value) : "memory");
  };
  auto vm_wait_step = [&]() { vm_wait(std::integral_constant<int, kDmaPerStep>{}); };

  // 32x32x16 operand layouts (wave64): A (32 x 16): lane l holds row l % 32,
  // k 8 (l / 32) .. +8; B (16 x 32): lane l holds column l % 32, the same k;
  // C (32 x 32): lane l holds column l % 32, rows 8 (i / 4) + 4 (l / 32) +
  // i % 4 for i < 16.
  const int c32 = lane & 31, kh = lane >> 5;
  // A fragment (mb, kblk): row mb*32 + c32, 16-byte chunk 2 kblk + kh of the
  // swizzled row ((r >> 1) & 7 == (c32 >> 1) & 7 for every mb).
  auto aoff = [&](int mb, int kblk) {
    return ((mb * 32 + c32) * TK + (((2 * kblk + kh) ^ ((c32 >> 1) & 7)) << 3)) * 2;
  };

  // B fragment (nb, kblk) = 8 codes of row nb*32 + c32, word 2 kblk + kh of
  // the group, found as word kblk of the row's 16-byte half kh (the re-layout
  // stores each row as its even words, then its odd words, the two halves
  // swapped on rows with bit 2 set so that the 8 lanes of one LDS read cycle
  // cover all banks).  bf[nb][kblk]: frag (nb, k) of step g is rewritten for
  // step g + 1 in the k block after its last use (k block 3 of step g + 1
  // during k block 0 of step g + 1).
  uint4 bf[NB][KB];
  // dw / dsf, dbf: code words, scales and biases of the step being
  // dequantized; dwn / dsbn: the next step's words and (s | b << 16), read
  // ahead of their first use.
  uint4 dw[NB], dwn[NB];
  float dsf[NB], dbf[NB];
  uint32_t dsbn[NB];
  auto read_sb = [&](int stg, uint32_t (&o)[NB]) {
    const uint8_t* ss = lds + stg * kStage + kXBytes + kWBytes + wave * 256;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) o[nb] = *reinterpret_cast<const uint32_t*>(ss + (nb * 32 + c32) * 4);
  };
  auto read_w = [&](int stg, uint4 (&o)[NB]) {
    const uint8_t* ws = lds + stg * kStage + kXBytes + wave * 2048;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      o[nb] = *reinterpret_cast<const uint4*>(ws + (nb * 32 + c32) * 32 +
                                              ((kh ^ ((c32 >> 2) & 1)) << 4));
  };
  // quarter q of the word of fragment nb: output register q (codes 2q, 2q+1)
  uint32_t dlo[NB], dhi[NB];
  auto dequant_q = [&](int nb, int kblk, int q) {
    if (q == 0) {
      const uint32_t v = kblk == 0 ? dw[nb].x : kblk == 1 ? dw[nb].y : kblk == 2 ? dw[nb].z : dw[nb].w;
      dlo[nb] = v & 0x0f0f0f0fu;
      dhi[nb] = (v >> 4) & 0x0f0f0f0fu;
    }
    uint32_t* o = reinterpret_cast<uint32_t*>(&bf[nb][kblk]);
    float a, c;
    if (q == 0) { a = ubyte<0>(dlo[nb]); c = ubyte<0>(dhi[nb]); }
    if (q == 1) { a = ubyte<1>(dlo[nb]); c = ubyte<1>(dhi[nb]); }
    if (q == 2) { a = ubyte<2>(dlo[nb]); c = ubyte<2>(dhi[nb]); }
    if (q == 3) { a = ubyte<3>(dlo[nb]); c = ubyte<3>(dhi[nb]); }
    o[q] = pk_bf16(fmaf(dsf[nb], a, dbf[nb]), fmaf(dsf[nb], c, dbf[nb]));
  };
  auto dequant_all = [&](int kblk) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int q = 0; q < 4; ++q) dequant_q(nb, kblk, q);
  };

  f32x16_t acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // prologue: steps 0 and 1 in flight; step 0 complete and its k block 0
  // dequantized (k blocks 1-3 follow during step 0).
  issue(g0, 0);
  issue(min(g0 + 1, g1 - 1), 1);
  vm_wait_step();
  __syncthreads();
  read_sb(0, dsbn);
  read_w(0, dw);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    dsf[nb] = __uint_as_float(dsbn[nb] << 16);
    dbf[nb] = __uint_as_float(dsbn[nb] & 0xffff0000u);
  }
  dequant_all(0);

  // One K step = 32 sub-steps (k block kblk = st / 8, row block mb = st % 8),
  // each: the A fragment of the next sub-step is read ahead, the 2 MFMAs
  // of (mb, kblk) issue, then a small piece of other work.  Fragments are
  // dequantized one k block ahead of their use, a quarter word per
  // sub-step: during k block j the fragments of k block j + 1 (of step g,
  // or of step g + 1 for j = 3), whose registers were last read in k block
  // j + 1 of the previous step.
  //   st < kDmaPerStep  one load each of step g + 2 (stage read in step g - 1)
  //   last sub-step of k block 2: wait for this lane's loads of step g + 1
  //             (the loads of step g + 2 may remain in flight)
  //   first sub-step of k block 3: read step g + 1's scales, biases and
  //             code words
  //   end       barrier: X(g + 1) of every wave complete
  // In the last step the loads repeat the last step's addresses and the
  // fragments dequantized for the step after it are never used.
  int stg = 0;
  for (int g = g0; g < g1; ++g) {
    const int stg1 = stg == kStages - 1 ? 0 : stg + 1;
    const int stg2 = stg1 == kStages - 1 ? 0 : stg1 + 1;
    const int gn = min(g + 2, g1 - 1);
    const uint8_t* xb = lds + stg * kStage;
    uint4 a = *reinterpret_cast<const uint4*>(xb + aoff(0, 0));
    uint4 an = *reinterpret_cast<const uint4*>(xb + aoff(1 % MB, 1 / MB));
#pragma unroll
    for (int st = 0; st < KB * MB; ++st) {
      const int kblk = st / MB, mb = st % MB;
      uint4 ann = an;
      if (st + 2 < KB * MB)
        ann = *reinterpret_cast<const uint4*>(xb + aoff((st + 2) % MB, (st + 2) / MB));
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = mfma32(a, bf[nb][kblk], acc[mb][nb]);
#ifndef GEMM_EXP_NO_DMA
      if (st < kDmaPerStep) issue1(gn, stg2, st);
#endif
#ifndef GEMM_EXP_NO_WAIT
      if (st == kReadSt - 1) vm_wait_step();
#endif
      if (st == kReadSt) {  // step g + 1's words, four sub-steps before their first use
        read_sb(stg1, dsbn);
        read_w(stg1, dwn);
      }
      if (st == 3 * MB) {  // step g's last dequant was one sub-step earlier
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          dw[nb] = dwn[nb];
          dsf[nb] = __uint_as_float(dsbn[nb] << 16);
          dbf[nb] = __uint_as_float(dsbn[nb] & 0xffff0000u);
        }
      }
#ifndef GEMM_EXP_NO_DEQ
#pragma unroll
      for (int t = 0; t < QPS; ++t) {
        const int j = mb * QPS + t;  // quarter j % 4 of fragment j / 4
        dequant_q(j / 4, (kblk + 1) % KB, j % 4);
      }
#endif
      __builtin_amdgcn_sched_barrier(0);
      a = an;
      an = ann;
    }
#ifndef GEMM_EXP_NO_BAR
    __syncthreads();
#endif
    stg = stg1;
  }
  // C layout: lane holds column c32, rows 8 (i / 4) + 4 kh + i % 4.
  if constexpr (SPLIT) {  // this K slice's fp32 partial sums, every row of the tile
    const int ld = nts * TN;
    float* pb = sp.part + ((int64_t)ks * (mt * TM) + m0 + 4 * kh) * ld + tnl * TN + wave * WN + c32;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          pb[(int64_t)(mb * 32 + 8 * (i / 4) + i % 4) * ld + nb * 32] = acc[mb][nb][i];
  } else {
  // The tile's problem (wave-uniform): the last one starting at or before n0.
  int p = 0;
#pragma unroll
  for (int t = 1; t < kMaxGemmProblems; ++t)
    if (t < out.count && n0 >= out.n0[t]) p = t;
  const int np = out.n0[p + 1] - out.n0[p];
  YT* yb = static_cast<YT*>(out.y[p]) + (int64_t)(m0 + 4 * kh) * np + (n0 - out.n0[p]) +
           wave * WN + c32;
  if (m0 + TM <= M) {  // a full tile (wave-uniform): stores without a row check
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          Elem<YT>::store(yb, (int64_t)(mb * 32 + 8 * (i / 4) + i % 4) * np + nb * 32,
                          acc[mb][nb][i]);
  } else {  // the partial last tile: rows at or past M are not stored
    const int rows_left = M - (m0 + 4 * kh);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int r = mb * 32 + 8 * (i / 4) + i % 4;
          if (r < rows_left) Elem<YT>::store(yb, (int64_t)r * np + nb * 32, acc[mb][nb][i]);
        }
  }
  }
}

// One launch's split linears, after its slices: y_p[m, c] = sum over
// slices s = 0 .. S - 1, in that order, of part[s][m][n0_p - c0 + c], where
// the launch covered columns c0 .. c0 + ld of the concatenated linears (each
// N a multiple of 256); four columns per thread.
template <typename YT>
__global__ __launch_bounds__(256) void q4_gemm_splitk_reduce(const float* __restrict__ part, int S,
                                                             int64_t slice, int ld, int c0, int M,
                                                             GemmOut out) {
  const int c4 = ld >> 2;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)M * c4) return;
  const int64_t m = i / c4;
  const int c = (int)(i - m * c4) * 4;  // column in the launch
  int p = 0;
#pragma unroll
  for (int t = 1; t < kMaxGemmProblems; ++t)
    if (t < out.count && c0 + c >= out.n0[t]) p = t;
  const int np = out.n0[p + 1] - out.n0[p], cp = c0 + c - out.n0[p];
  const float* pp = part + m * ld + c;
  float4 a = *reinterpret_cast<const float4*>(pp);
  for (int s = 1; s < S; ++s) {
    const float4 b = *reinterpret_cast<const float4*>(pp + s * slice);
    a.x += b.x;
    a.y += b.y;
    a.z += b.z;
    a.w += b.w;
  }
  YT* y = static_cast<YT*>(out.y[p]);
  const int64_t off = m * np + cp;
  Elem<YT>::store(y, off, a.x);
  Elem<YT>::store(y, off + 1, a.y);
  Elem<YT>::store(y, off + 2, a.z);
  Elem<YT>::store(y, off + 3, a.w);
}

// Re-layout of one q4 weight for the kernel above (a pass over the weight,
// ~1% of the GEMM at 8192 rows): codes group-major, wt[g][n][8 words], so a
// K step's rows are contiguous, each row's words in the order 0 2 4 6 | 1 3
// 5 7 (halves swapped when bit 2 of n is set); scale and bias of (n, g)
// packed in one word, sbt[g][n] = s | b << 16.
// Rows 0 .. Np - 1 of one weight go to rows n_off .. of a layout Ntot rows
// wide (the linears of one launch, concatenated).  A workgroup moves a tile
// of 32 rows x 8 groups: thread t takes row t / 8 and group t % 8, so the
// reads (8 groups of a row, 256 contiguous bytes) and the writes (8 rows of
// a group, 256 contiguous bytes) both run in 256-byte pieces.
__global__ __launch_bounds__(256) void q4_gemm_relayout_kernel(
    const uint4* __restrict__ w, const uint16_t* __restrict__ s, const uint16_t* __restrict__ b,
    int Np, int G, int Ntot, int n_off, uint4* __restrict__ wt, uint32_t* __restrict__ sbt) {
  const int gtiles = (G + 7) / 8;
  const int nt = blockIdx.x / gtiles, gt = blockIdx.x - nt * gtiles;
  const int nl = nt * 32 + (threadIdx.x >> 3), g = gt * 8 + (threadIdx.x & 7);
  if (nl >= Np || g >= G) return;
  const int64_t i = (int64_t)nl * G + g;  // (row, group) of the source
  const int n = n_off + nl;
  const uint4 lo = w[i * 2], hi = w[i * 2 + 1];
  const uint4 ev = make_uint4(lo.x, lo.z, hi.x, hi.z), od = make_uint4(lo.y, lo.w, hi.y, hi.w);
  const int sw = (n >> 2) & 1;
  wt[((int64_t)g * Ntot + n) * 2 + sw] = ev;
  wt[((int64_t)g * Ntot + n) * 2 + (sw ^ 1)] = od;
  sbt[(int64_t)g * Ntot + n] = (uint32_t)s[i] | ((uint32_t)b[i] << 16);
}

}  // namespace

size_t strata_q4_gemm_mfma_scratch(int64_t N, int K) {  // == strata_q4_gemm_pack's buffer
  return (size_t)N * K / 2 + (size_t)N * (K / TK) * 4;
}

namespace {
// Checks the linears of one launch and fills their output table; returns the
// concatenated N through *Ntot.
int gemm_problems(const strata_q4_weight* ws, int count, GemmOut* out, int* Ntot) {
  STRATA_REQUIRE(count >= 1 && count <= kMaxGemmProblems, "q4 GEMM: 1..%d linears per launch",
                 kMaxGemmProblems);
  *out = GemmOut{};
  out->count = count;
  int64_t N = 0;
  for (int p = 0; p < count; ++p) {
    STRATA_REQUIRE(ws[p].N > 0 && ws[p].N % TN == 0,
                   "q4 GEMM (256-tile kernel): N must be a positive multiple of 256");
    out->y[p] = ws[p].y;
    out->n0[p] = (int)N;
    N += ws[p].N;
  }
  STRATA_REQUIRE(N <= INT32_MAX, "q4 GEMM: too many output columns");
  out->n0[count] = (int)N;
  *Ntot = (int)N;
  return STRATA_OK;
}
}  // namespace

int strata_q4_gemm_pack(const strata_q4_weight* ws, int count, int K, void* packed, void* stream) {
  STRATA_REQUIRE(K % TK == 0 && K >= TK, "q4 GEMM: K must be a positive multiple of 64");
  GemmOut out;
  int N = 0;
  int rc = gemm_problems(ws, count, &out, &N);
  if (rc) return rc;
  STRATA_REQUIRE((uint64_t)N * K / 2 < (1ull << 32), "q4 GEMM (256-tile kernel): weight over 4 GiB");
  STRATA_REQUIRE(packed && (reinterpret_cast<uintptr_t>(packed) & 15) == 0,
                 "q4 GEMM: unaligned packed buffer");
  const int G = K / TK;
  uint32_t* wt = static_cast<uint32_t*>(packed);
  uint32_t* sbt = wt + (size_t)N * K / 8;
  for (int p = 0; p < count; ++p) {
    STRATA_REQUIRE((reinterpret_cast<uintptr_t>(ws[p].w) & 15) == 0, "q4 GEMM: unaligned weight");
    const int64_t tiles = (ws[p].N + 31) / 32 * ((G + 7) / 8);
    hipLaunchKernelGGL(q4_gemm_relayout_kernel, dim3((unsigned)tiles), dim3(256), 0,
                       as_stream(stream), reinterpret_cast<const uint4*>(ws[p].w), ws[p].scales,
                       ws[p].biases, (int)ws[p].N, G, N, out.n0[p], reinterpret_cast<uint4*>(wt),
                       sbt);
    STRATA_HIP_CHECK(hipGetLastError());
  }
  return STRATA_OK;
}

namespace {
int num_cus() {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  return cus;
}

// K slices for one linear of N columns at M rows.  The 128-row tiles times
// the slices aim at one workgroup per CU for long rows (K >= 8192) and half
// that otherwise (measured on the 8B shapes at 128-512 rows: more slices
// cost more in partial sums than they gain); a power of two, each slice at
// least 4 K groups, at most 16 (8 below K = 8192, so that q, k and v
// share a launch).  It depends on (M, K, N) only, so a linear
// gives the same bits in a fused launch and alone.  (At 2048 rows, two
// slices for the 8B launches under 2-3 workgroups per CU made the engine's
// prefill slower: 30.0 against 28.7 ms.)
int splitk_slices(int M, int K, int N, int cus) {
  const int G = K / TK;
  // A narrow linear (k, v) counts as 16 column tiles: it then gets the
  // slices of the 4096-column one (q) it is usually launched with.
  const int64_t tiles = (int64_t)((M + 127) / 128) * std::max(N / TN, 16);
  const int64_t target = G >= 128 ? cus : cus / 2;
  int S = tiles >= target ? 1 : (int)(target / tiles);
  int p2 = 1;
  while (p2 * 2 <= S) p2 *= 2;
  S = p2;
  S = std::min(S, std::min(G >= 128 ? 16 : 8, std::max(1, G / 4)));
  return std::max(S, 1);
}

size_t splitk_part_bytes(int M, int N, int S) {
  return S > 1 ? (size_t)S * ((M + 127) / 128 * 128) * N * 4 : 0;
}

// Slices of each linear, and runs of consecutive linears with the same
// slice count (one launch each): run r covers linears first[r] ..
// first[r + 1] - 1.
struct SplitPlan {
  int S[kMaxGemmProblems];
  int first[kMaxGemmProblems + 1];
  int runs;
};
SplitPlan split_plan(int M, int K, const strata_q4_weight* ws, int count, int cus, bool allow) {
  SplitPlan pl{};
  for (int p = 0; p < count; ++p) pl.S[p] = allow ? splitk_slices(M, K, (int)ws[p].N, cus) : 1;
  pl.runs = 0;
  for (int p = 0; p < count; ++p)
    if (p == 0 || pl.S[p] != pl.S[p - 1]) pl.first[pl.runs++] = p;
  pl.first[pl.runs] = count;
  return pl;
}
size_t plan_part_bytes(const SplitPlan& pl, int M, const strata_q4_weight* ws) {
  size_t need = 0;
  for (int r = 0; r < pl.runs; ++r) {
    int64_t n = 0;
    for (int p = pl.first[r]; p < pl.first[r + 1]; ++p) n += ws[p].N;
    need = std::max(need, splitk_part_bytes(M, (int)n, pl.S[pl.first[r]]));
  }
  return need;
}

template <int TM, typename YT, bool SPLIT>
void gemm_go(const void* x, int M, int K, const uint32_t* wt, const uint32_t* sbt, int N,
             const GemmOut& out, const GemmSplit& sp, hipStream_t st) {
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute((const void*)q4_gemm_mfma_kernel<TM, YT, SPLIT>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, Tile<TM>::kLds);
    attr = true;
  }
  hipLaunchKernelGGL((q4_gemm_mfma_kernel<TM, YT, SPLIT>), dim3(sp.mt * sp.nts * sp.S), dim3(NTHR),
                     Tile<TM>::kLds, st, (const uint16_t*)x, M, K, wt, sbt, N, out, sp);
}
}  // namespace

size_t strata_q4_gemm_mfma_part_bytes(int M, int K, const strata_q4_weight* ws, int count) {
  if (count < 1 || count > kMaxGemmProblems) return 0;
  return plan_part_bytes(split_plan(M, K, ws, count, num_cus(), true), M, ws);
}

int strata_q4_gemm_mfma_launch(const void* x, int M, int K, const strata_q4_weight* ws, int count,
                               int y_dtype, void* scratch, void* stream) {
  const int rc = strata_q4_gemm_pack(ws, count, K, scratch, stream);
  if (rc) return rc;
  return strata_q4_gemm_mfma_run(x, M, K, scratch, ws, count, y_dtype, stream);
}

int strata_q4_gemm_mfma_run(const void* x, int M, int K, const void* packed,
                            const strata_q4_weight* ws, int count, int y_dtype, void* stream,
                            float* part, size_t part_bytes) {
  STRATA_REQUIRE(K % TK == 0 && K >= TK, "q4 GEMM: K must be a positive multiple of 64");
  GemmOut out;
  int N = 0;
  int rc = gemm_problems(ws, count, &out, &N);
  if (rc) return rc;
  STRATA_REQUIRE(M > 0, "q4 GEMM (256-column kernel): M must be positive");
  STRATA_REQUIRE((uint64_t)M * K * 2 < (1ull << 32) && (uint64_t)N * K / 2 < (1ull << 32),
                 "q4 GEMM (256-column kernel): operands must be under 4 GiB");
  STRATA_REQUIRE(packed && (reinterpret_cast<uintptr_t>(packed) & 15) == 0,
                 "q4 GEMM: unaligned packed buffer");
  const uint32_t* wt = static_cast<const uint32_t*>(packed);
  const uint32_t* sbt = wt + (size_t)N * K / 8;
  hipStream_t st = as_stream(stream);
  const bool bf = y_dtype == STRATA_BF16;
  const int cus = num_cus();
  // A launch over columns [ntile0, ntile0 + nts) tiles with S slices: 256-row
  // tiles unless that leaves the GPU under two workgroups per CU.
  auto go = [&](int ntile0, int nts, int S) {
    bool big = S == 1 && (int64_t)((M + 255) / 256) * nts >= 2 * cus;
    const int TM = big ? 256 : 128;
    const GemmSplit sp{(M + TM - 1) / TM, ntile0, nts, S, S > 1 ? part : nullptr};
    if (S > 1)  // 128-row tiles; the partial sums are fp32 whatever y's dtype
      gemm_go<128, float, true>(x, M, K, wt, sbt, N, out, sp, st);
    else if (big) {
      if (bf) gemm_go<256, bf16_t, false>(x, M, K, wt, sbt, N, out, sp, st);
      else gemm_go<256, float, false>(x, M, K, wt, sbt, N, out, sp, st);
    } else {
      if (bf) gemm_go<128, bf16_t, false>(x, M, K, wt, sbt, N, out, sp, st);
      else gemm_go<128, float, false>(x, M, K, wt, sbt, N, out, sp, st);
    }
  };
  SplitPlan pl = split_plan(M, K, ws, count, cus, part != nullptr);
  if (plan_part_bytes(pl, M, ws) > part_bytes) pl = split_plan(M, K, ws, count, cus, false);
  // One launch per run of linears with the same slice count; a split run is
  // followed by one launch that sums its slices in order for all of its
  // linears (the partial buffer is reused run after run, in stream order).
  for (int r = 0; r < pl.runs; ++r) {
    const int pa = pl.first[r], pe = pl.first[r + 1], S = pl.S[pa];
    const int c0 = out.n0[pa], ncols = out.n0[pe] - c0;
    go(c0 / TN, ncols / TN, S);
    if (S == 1) continue;
    STRATA_HIP_CHECK(hipGetLastError());
    const int64_t slice = (int64_t)((M + 127) / 128 * 128) * ncols;
    const unsigned blocks = (unsigned)(((int64_t)M * (ncols / 4) + 255) / 256);
    if (bf)
      hipLaunchKernelGGL(q4_gemm_splitk_reduce<bf16_t>, dim3(blocks), dim3(256), 0, st, part, S,
                         slice, ncols, c0, M, out);
    else
      hipLaunchKernelGGL(q4_gemm_splitk_reduce<float>, dim3(blocks), dim3(256), 0, st, part, S,
                         slice, ncols, c0, M, out);
  }
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}
