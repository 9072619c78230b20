// q4 linear for a few rows (9 <= M < 40 on the default path, up to 64): Y[M, N] =
// X[M, K] @ dequant(W)[N, K]^T on bf16 16x16x32 MFMAs, every weight read once.
//
// Same maths as mx.quantized_matmul(transpose=True) (src/ollm/llama_mlx.py:
// 53-74, the prefill call at 393-432 with a short prompt): each weight is
// s * q + b in fp32, rounded once to bf16 (as the 256-tile GEMM does), and the
// products accumulate in fp32.
//
// Sizing for MI355X: the 128 x 128-tile kernel (q4_gemm.hip) covers a 6144 x
// 4096 projection at 16 rows with 48 workgroups and takes ~230 us; here every
// workgroup owns only NC x 16 output columns, so the same launch has 384-1536
// workgroups streaming their weight rows in parallel.
//   * Workgroup = 4 waves on the same NC x 16 columns; wave w reduces the K
//     quarter w, and the four partial sums meet in LDS at the end.
//   * Per 128-k chunk a lane loads, for each of its NC columns (row
//     n0 + 16 c + lane % 16), the 16-byte code run of k 32 (lane / 16) .. +32
//     with that group's scale and bias, and for each of its MB x row blocks
//     (row 16 mb + lane % 16) the 32 x values of the same k.  Word j of the
//     run is the B operand of MFMA k-step j: lane (c, g) supplies k slots
//     8 g .. 8 g + 7 of each 32-k step from k 32 g + 8 j .. +8, and its A
//     operand (x) uses the same k, so the dot products are unchanged.
//   * The next NB - 1 chunks' loads are issued before the current chunk's
//     math (NB register sets).
//   * Outputs: lane (c, g) of the 16x16 accumulator holds column c and rows
//     4 g .. 4 g + 3.
#include <type_traits>

#include "strata_internal.h"

#ifndef SKINNY_NB
#define SKINNY_NB 3
#endif

namespace {

struct SkinnyProblem {
  const uint4* w;      // [n, K/32] uint4
  const uint16_t* s;   // [n, K/64]
  const uint16_t* b;
  void* y;             // [M, n]
  int n;
  int col0;            // first column of this linear in the launch
};

struct SkinnyBatch {
  SkinnyProblem p[kMaxGemmProblems];
  int count;
};

__device__ __forceinline__ f32x4_t mfma16x32(const uint4& a, const uint4& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// 8 codes of one word (k order, nibble i = code i) -> 8 bf16 s*q + b
__device__ __forceinline__ uint4 dequant8(uint32_t w, float s, float b) {
  const uint32_t lo = w & 0x0f0f0f0fu;         // codes 0, 2, 4, 6
  const uint32_t hi = (w >> 4) & 0x0f0f0f0fu;  // codes 1, 3, 5, 7
  uint4 o;
  o.x = pk_bf16(fmaf(s, (float)(lo & 0xffu), b), fmaf(s, (float)(hi & 0xffu), b));
  o.y = pk_bf16(fmaf(s, (float)((lo >> 8) & 0xffu), b), fmaf(s, (float)((hi >> 8) & 0xffu), b));
  o.z = pk_bf16(fmaf(s, (float)((lo >> 16) & 0xffu), b), fmaf(s, (float)((hi >> 16) & 0xffu), b));
  o.w = pk_bf16(fmaf(s, (float)(lo >> 24), b), fmaf(s, (float)(hi >> 24), b));
  return o;
}

template <int MB, int NC, int NB, typename YT>
__global__ __launch_bounds__(256) void q4_gemm_skinny_kernel(const uint16_t* __restrict__ x, int M,
                                                             int K, SkinnyBatch bt) {
  __shared__ f32x4_t red[3][MB * NC][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, kq = lane >> 4;
  const int col0 = blockIdx.x * (16 * NC);
  int p = 0;
#pragma unroll
  for (int t = 1; t < kMaxGemmProblems; ++t)
    if (t < bt.count && col0 >= bt.p[t].col0) p = t;
  const SkinnyProblem& P = bt.p[p];
  const int n0 = col0 - P.col0;
  const int nv = K >> 5, ng = K >> 6;
  const int kw = K >> 2, kbeg = wave * kw, nch = kw >> 7;

  const uint4* wr[NC];
  const uint16_t* sr[NC];
  const uint16_t* br[NC];
#pragma unroll
  for (int cc = 0; cc < NC; ++cc) {
    const int row = n0 + 16 * cc + c;
    wr[cc] = P.w + (int64_t)row * nv;
    sr[cc] = P.s + (int64_t)row * ng;
    br[cc] = P.b + (int64_t)row * ng;
  }
  const uint16_t* xr[MB];
  bool live[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = 16 * mb + c;
    live[mb] = m < M;
    xr[mb] = x + (int64_t)min(m, M - 1) * K;
  }

  uint4 wv[NB][NC], xv[NB][MB][4];
  uint32_t sv[NB][NC], bv[NB][NC];
  // The register set is a compile-time constant (std::integral_constant), so
  // the sets stay in registers whatever the inliner decides.
  auto issue = [&](auto BC, int ch) {
    constexpr int buf = decltype(BC)::value;
    const int kb = kbeg + (ch << 7) + 32 * kq;  // this lane's first k of the chunk
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      wv[buf][cc] = load_nt(wr[cc] + (kb >> 5));
      sv[buf][cc] = sr[cc][kb >> 6];
      bv[buf][cc] = br[cc][kb >> 6];
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < 4; ++j) xv[buf][mb][j] = reinterpret_cast<const uint4*>(xr[mb] + kb)[j];
  };

  f32x4_t acc[MB][NC];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) acc[mb][cc] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](auto BC) {
    constexpr int buf = decltype(BC)::value;
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      const float s = __uint_as_float(sv[buf][cc] << 16), b = __uint_as_float(bv[buf][cc] << 16);
      const uint32_t ww[4] = {wv[buf][cc].x, wv[buf][cc].y, wv[buf][cc].z, wv[buf][cc].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 bw = dequant8(ww[j], s, b);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const uint4 a = live[mb] ? xv[buf][mb][j] : make_uint4(0, 0, 0, 0);
          acc[mb][cc] = mfma16x32(a, bw, acc[mb][cc]);
        }
      }
    }
  };

  // NB register sets: chunks ch + 1 .. ch + NB - 1 are in flight while
  // chunk ch is computed (set indices are compile-time constants)
  issue(std::integral_constant<int, 0>{}, 0);
  if constexpr (NB > 2)
    if (1 < nch) issue(std::integral_constant<int, 1>{}, 1);
  if constexpr (NB > 3)
    if (2 < nch) issue(std::integral_constant<int, 2>{}, 2);
  auto step = [&](int ch, auto BC) {
    constexpr int BUF = decltype(BC)::value;
    if (ch + NB - 1 < nch) issue(std::integral_constant<int, (BUF + NB - 1) % NB>{}, ch + NB - 1);
    compute(BC);
  };
  for (int ch = 0; ch < nch; ch += NB) {
    step(ch, std::integral_constant<int, 0>{});
    if (ch + 1 < nch) step(ch + 1, std::integral_constant<int, 1 % NB>{});
    if constexpr (NB > 2)
      if (ch + 2 < nch) step(ch + 2, std::integral_constant<int, 2 % NB>{});
    if constexpr (NB > 3)
      if (ch + 3 < nch) step(ch + 3, std::integral_constant<int, 3 % NB>{});
  }

  // the four K quarters meet in LDS; wave 0 adds them in wave order and stores
  if (wave > 0) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) red[wave - 1][mb * NC + cc][lane] = acc[mb][cc];
  }
  __syncthreads();
  if (wave != 0) return;
  YT* y = static_cast<YT*>(P.y);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      f32x4_t v = acc[mb][cc];
#pragma unroll
      for (int w = 0; w < 3; ++w) v += red[w][mb * NC + cc][lane];
      const int n = n0 + 16 * cc + c;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 16 * mb + 4 * kq + r;
        if (m < M) Elem<YT>::store(y, (int64_t)m * P.n + n, v[r]);
      }
    }
}

template <int MB, int NC>
void launch_skinny(const uint16_t* x, int M, int K, const SkinnyBatch& bt, int cols, int y_dtype,
                   hipStream_t stream) {
  constexpr int NB = SKINNY_NB;
  const dim3 grid(cols / (16 * NC));
  if (y_dtype == STRATA_BF16)
    hipLaunchKernelGGL((q4_gemm_skinny_kernel<MB, NC, NB, bf16_t>), grid, dim3(256), 0, stream, x,
                       M, K, bt);
  else
    hipLaunchKernelGGL((q4_gemm_skinny_kernel<MB, NC, NB, float>), grid, dim3(256), 0, stream, x,
                       M, K, bt);
}

}  // namespace

bool strata_q4_skinny_fits(int M, int K, const strata_q4_weight* ws, int count) {
  if (M < 1 || M > kSkinnyMaxRows || K % 512 != 0 || count < 1 || count > kMaxGemmProblems)
    return false;
  for (int i = 0; i < count; ++i)
    if (ws[i].N % 16 != 0 || !aligned16(ws[i].w)) return false;
  return true;
}

int strata_q4_gemm_skinny(const void* x, int M, int K, const strata_q4_weight* ws, int count,
                          int y_dtype, void* stream) {
  STRATA_REQUIRE(strata_q4_skinny_fits(M, K, ws, count),
                 "q4 skinny GEMM: needs 1 <= M <= %d, K %% 512 == 0, N %% 16 == 0", kSkinnyMaxRows);
  STRATA_REQUIRE(aligned16(x), "q4 skinny GEMM: x must be 16-byte aligned");
  SkinnyBatch bt{};
  bt.count = count;
  int cols = 0;
  bool n64 = true;  // every linear a multiple of 64 columns
  for (int i = 0; i < count; ++i) {
    bt.p[i] = SkinnyProblem{reinterpret_cast<const uint4*>(ws[i].w), ws[i].scales, ws[i].biases,
                            ws[i].y, static_cast<int>(ws[i].N), cols};
    cols += static_cast<int>(ws[i].N);
    n64 = n64 && ws[i].N % 64 == 0;
  }
  hipStream_t s = as_stream(stream);
  const uint16_t* xx = static_cast<const uint16_t*>(x);
  // 64-column workgroups (4 column blocks share each x fragment) when that
  // still gives >= 256 workgroups, else 16-column workgroups; x row blocks of
  // 16 per wave up to 2 (64 columns) or 4 (16 columns) within the registers.
  const bool wide = n64 && cols >= 16384 && M <= 32;
  if (wide) {
    if (M <= 16) launch_skinny<1, 4>(xx, M, K, bt, cols, y_dtype, s);
    else launch_skinny<2, 4>(xx, M, K, bt, cols, y_dtype, s);
  } else {
    if (M <= 16) launch_skinny<1, 1>(xx, M, K, bt, cols, y_dtype, s);
    else if (M <= 32) launch_skinny<2, 1>(xx, M, K, bt, cols, y_dtype, s);
    else launch_skinny<4, 1>(xx, M, K, bt, cols, y_dtype, s);
  }
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}
