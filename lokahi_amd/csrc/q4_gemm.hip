// Prefill-side q4 GEMM: Y[M, N] = X[M, K] @ dequant(W)[N, K]^T on bf16 MFMA.
//
// Same maths as mx.quantized_matmul(transpose=True) (src/ollm/llama_mlx.py:53-74)
// on the prefill path (M = tokens > 8).  Each K step is exactly one
// quantization group (64): the workgroup dequantizes its 128 x 64 weight tile
// once into LDS as bf16 (s*q + b, fp32 then round-to-nearest-even, as MLX's
// qmm dequantizes into threadgroup memory in the activation dtype), stages the
// 128 x 64 activation tile next to it, and 4 waves (2 x 2) each run a 64 x 64
// block of v_mfma_f32_16x16x32_bf16 with fp32 accumulators.  The next tile's
// global loads are issued before the current tile's MFMAs (register prefetch).
//
// Dequantization costs ~3 VALU per code: nibbles are masked into bytes once
// per word, each byte converts with one v_cvt_f32_ubyte*, one FMA applies
// s and b, and v_cvt_pk_bf16_f32 rounds two values at a time.  LDS rows are
// 64 bf16 (128 B) with no padding; the 16-byte chunk c of row r is stored at
// chunk c ^ ((r >> 1) & 7), so every 16-lane phase of the b128 stores and of
// the MFMA operand reads touches 64 distinct banks.
#include "strata_common.h"

namespace {

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDS_STRIDE = BK;  // bf16 elements per LDS row (128 B), chunks XOR-swizzled

// Element offset of 16-byte chunk `c` (0..7) of row `r` in a swizzled tile.
__device__ __forceinline__ int swz(int r, int c) { return r * LDS_STRIDE + ((c ^ ((r >> 1) & 7)) << 3); }

__device__ __forceinline__ f32x4_t mfma16(const uint4& a, const uint4& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Two floats -> packed bf16 pair, round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t bf16x2_from(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

template <typename YT>
__global__ __launch_bounds__(256) void q4_gemm_kernel(const uint16_t* __restrict__ x, int M, int K,
                                                      const uint32_t* __restrict__ w,
                                                      const uint16_t* __restrict__ sc,
                                                      const uint16_t* __restrict__ bi, int N,
                                                      YT* __restrict__ y) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[BM * LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) uint16_t ws[BN * LDS_STRIDE];

  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int col = lane & 15, grp = lane >> 4;
  const int groups = K / BK;

  // X staging: 128 rows x 8 uint4 per K step -> 4 uint4 per thread.
  // W staging: thread handles row tid/2, codes (tid%2)*32 .. +32 (one uint4).
  const int wrow = tid >> 1, whalf = tid & 1;
  const bool wrow_ok = n0 + wrow < N;
  const uint4* wsrc = reinterpret_cast<const uint4*>(w + (int64_t)(n0 + wrow) * (K / 8));

  // Register prefetch: tile g+1's global loads are in flight while tile g
  // computes.  (A second register stage costs occupancy and measured slower.)
  struct Stage {
    uint4 xr[4];
    uint4 wr;
    uint16_t sr, br;
  };
  Stage sa;
  auto load_tile = [&](Stage& st, int g) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + c * 256;
      const int r = idx >> 3, ch = idx & 7;
      st.xr[c] = (m0 + r < M)
                     ? *reinterpret_cast<const uint4*>(x + (int64_t)(m0 + r) * K + g * BK + ch * 8)
                     : make_uint4(0, 0, 0, 0);
    }
    if (wrow_ok) {
      st.wr = load_nt(wsrc + g * 2 + whalf);
      st.sr = sc[(int64_t)(n0 + wrow) * groups + g];
      st.br = bi[(int64_t)(n0 + wrow) * groups + g];
    } else {
      st.wr = make_uint4(0, 0, 0, 0);
      st.sr = 0;
      st.br = 0;
    }
  };
  auto store_tile = [&](const Stage& st) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + c * 256;
      const int r = idx >> 3, ch = idx & 7;
      *reinterpret_cast<uint4*>(&xs[swz(r, ch)]) = st.xr[c];
    }
    const float s = bf16_to_f32(st.sr), b = bf16_to_f32(st.br);
    const uint32_t words[4] = {st.wr.x, st.wr.y, st.wr.z, st.wr.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t u = words[j];
      const uint32_t lo = u & 0x0f0f0f0fu;          // codes 0, 2, 4, 6 (one per byte)
      const uint32_t hi = (u >> 4) & 0x0f0f0f0fu;   // codes 1, 3, 5, 7
      float q[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        q[2 * e] = static_cast<float>((lo >> (8 * e)) & 0xffu);
        q[2 * e + 1] = static_cast<float>((hi >> (8 * e)) & 0xffu);
      }
      uint4 o;
      o.x = bf16x2_from(fmaf(s, q[0], b), fmaf(s, q[1], b));
      o.y = bf16x2_from(fmaf(s, q[2], b), fmaf(s, q[3], b));
      o.z = bf16x2_from(fmaf(s, q[4], b), fmaf(s, q[5], b));
      o.w = bf16x2_from(fmaf(s, q[6], b), fmaf(s, q[7], b));
      *reinterpret_cast<uint4*>(&ws[swz(wrow, whalf * 4 + j)]) = o;
    }
  };

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&]() {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      uint4 a[4], bfr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a[i] = *reinterpret_cast<const uint4*>(&xs[swz(wm * 64 + i * 16 + col, kk * 4 + grp)]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bfr[j] = *reinterpret_cast<const uint4*>(&ws[swz(wn * 64 + j * 16 + col, kk * 4 + grp)]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16(a[i], bfr[j], acc[i][j]);
    }
  };

  load_tile(sa, 0);
  for (int g = 0; g < groups; ++g) {
    store_tile(sa);
    __syncthreads();
    if (g + 1 < groups) load_tile(sa, g + 1);
    compute();
    __syncthreads();
  }

  // C layout: lane holds column n = col, rows m = grp*4 + r of each 16x16 tile.
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + wn * 64 + j * 16 + col;
      if (n >= N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * 64 + i * 16 + grp * 4 + r;
        if (m < M) Elem<YT>::store(y, (int64_t)m * N + n, acc[i][j][r]);
      }
    }
}

}  // namespace

int strata_q4_gemm_launch(const void* x, int M, int K, const uint32_t* w, const uint16_t* s,
                          const uint16_t* b, int N, void* y, int y_dtype, void* stream) {
  dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
  if (y_dtype == STRATA_BF16)
    hipLaunchKernelGGL(q4_gemm_kernel<bf16_t>, grid, dim3(256), 0, as_stream(stream),
                       (const uint16_t*)x, M, K, w, s, b, N, (bf16_t*)y);
  else
    hipLaunchKernelGGL(q4_gemm_kernel<float>, grid, dim3(256), 0, as_stream(stream),
                       (const uint16_t*)x, M, K, w, s, b, N, (float*)y);
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}
