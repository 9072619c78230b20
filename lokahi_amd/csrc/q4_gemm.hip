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
#include "strata_common.h"

namespace {

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDS_STRIDE = BK + 8;  // bf16 elements per LDS row (144 B, conflict-free 16 B reads)

__device__ __forceinline__ f32x4_t mfma16(const uint4& a, const uint4& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t bf16x2_from(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
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

  uint4 xr[4];
  uint4 wr;
  uint16_t sr, br;
  auto load_tile = [&](int g) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + c * 256;
      const int r = idx >> 3, ch = idx & 7;
      xr[c] = (m0 + r < M)
                  ? *reinterpret_cast<const uint4*>(x + (int64_t)(m0 + r) * K + g * BK + ch * 8)
                  : make_uint4(0, 0, 0, 0);
    }
    if (wrow_ok) {
      wr = load_nt(wsrc + g * 2 + whalf);
      sr = sc[(int64_t)(n0 + wrow) * groups + g];
      br = bi[(int64_t)(n0 + wrow) * groups + g];
    } else {
      wr = make_uint4(0, 0, 0, 0);
      sr = 0;
      br = 0;
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + c * 256;
      const int r = idx >> 3, ch = idx & 7;
      *reinterpret_cast<uint4*>(&xs[r * LDS_STRIDE + ch * 8]) = xr[c];
    }
    const float s = bf16_to_f32(sr), b = bf16_to_f32(br);
    const uint32_t words[4] = {wr.x, wr.y, wr.z, wr.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t u = words[j];
      uint4 o;
      o.x = bf16x2_from(fmaf(s, (float)(u & 15u), b), fmaf(s, (float)((u >> 4) & 15u), b));
      o.y = bf16x2_from(fmaf(s, (float)((u >> 8) & 15u), b), fmaf(s, (float)((u >> 12) & 15u), b));
      o.z = bf16x2_from(fmaf(s, (float)((u >> 16) & 15u), b), fmaf(s, (float)((u >> 20) & 15u), b));
      o.w = bf16x2_from(fmaf(s, (float)((u >> 24) & 15u), b), fmaf(s, (float)(u >> 28), b));
      *reinterpret_cast<uint4*>(&ws[wrow * LDS_STRIDE + whalf * 32 + j * 8]) = o;
    }
  };

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  load_tile(0);
  for (int g = 0; g < groups; ++g) {
    store_tile();
    __syncthreads();
    if (g + 1 < groups) load_tile(g + 1);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      uint4 a[4], bfr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a[i] = *reinterpret_cast<const uint4*>(
            &xs[(wm * 64 + i * 16 + col) * LDS_STRIDE + kk * 32 + grp * 8]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bfr[j] = *reinterpret_cast<const uint4*>(
            &ws[(wn * 64 + j * 16 + col) * LDS_STRIDE + kk * 32 + grp * 8]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16(a[i], bfr[j], acc[i][j]);
    }
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
