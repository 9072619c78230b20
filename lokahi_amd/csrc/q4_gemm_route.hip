// Prefill q4 linears (M > 8 rows): routing to the hand-written kernels, and
// the q4 -> bf16 expansion behind strata_dequantize_q4.
//
// Same maths as mx.quantized_matmul(transpose=True) (src/ollm/llama_mlx.py:53-74)
// on the prefill path: the fused-dequant MFMA GEMM for 40 rows and more
// (q4_gemm_mfma.hip), the skinny MFMA kernel below (q4_gemm_skinny.hip),
// the 128 x 128 tile kernel for shapes neither takes (q4_gemm.hip).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>

#include "strata_common.h"
#include "strata_internal.h"

namespace {

// One thread expands 32 codes (one uint4 of packed words) into 64 bytes of bf16.
__global__ __launch_bounds__(256) void q4_dequant_bf16_kernel(const uint4* __restrict__ w,
                                                              const uint16_t* __restrict__ sc,
                                                              const uint16_t* __restrict__ bi,
                                                              int64_t n_chunks, int chunks_per_row,
                                                              uint4* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n_chunks) return;
  const int64_t row = i / chunks_per_row;
  const int c = (int)(i - row * chunks_per_row);
  const int groups = chunks_per_row >> 1;  // two chunks per group of 64
  const uint4 u4 = load_nt(w + i);
  const float s = bf16_to_f32(sc[row * groups + (c >> 1)]);
  const float b = bf16_to_f32(bi[row * groups + (c >> 1)]);
  const uint32_t words[4] = {u4.x, u4.y, u4.z, u4.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t lo = words[j] & 0x0f0f0f0fu;          // codes 0, 2, 4, 6
    const uint32_t hi = (words[j] >> 4) & 0x0f0f0f0fu;   // codes 1, 3, 5, 7
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = fmaf(s, static_cast<float>((lo >> (8 * e)) & 0xffu), b);
      const float d = fmaf(s, static_cast<float>((hi >> (8 * e)) & 0xffu), b);
      const bf16x2_t v = {static_cast<__bf16>(a), static_cast<__bf16>(d)};
      o[e] = __builtin_bit_cast(uint32_t, v);
    }
    out[i * 4 + j] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

}  // namespace

int strata_q4_dequant_launch(const uint32_t* w, const uint16_t* s, const uint16_t* b, int64_t N,
                             int K, uint16_t* out, void* stream) {
  const int chunks_per_row = K / 32;
  const int64_t n_chunks = N * chunks_per_row;
  if (n_chunks == 0) return STRATA_OK;
  hipLaunchKernelGGL(q4_dequant_bf16_kernel, dim3((unsigned)((n_chunks + 255) / 256)), dim3(256),
                     0, as_stream(stream), reinterpret_cast<const uint4*>(w), s, b, n_chunks,
                     chunks_per_row, reinterpret_cast<uint4*>(out));
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}

int strata_q4_gemm_multi(strata_ctx* ctx, const void* x, int M, int K, const strata_q4_weight* ws,
                         int count, int y_dtype, void* stream, const GemmPacked* packed) {
  const size_t ye = y_dtype == STRATA_BF16 ? 2 : 4;
  // Each linear goes its own way, so that it gives the same bits in a
  // fused call as alone:
  //   * from kMfmaMidRows rows, N a multiple of 256: the 256-column MFMA
  //     kernel over all rows (a partial last row tile; K split over several
  //     workgroups for linears with few tiles), the linears of one call in
  //     as few launches as their splits allow;
  //   * below that, shapes the skinny kernel takes (K % 512 == 0, N % 16 ==
  //     0): the skinny kernel, rows in slices of 64, one launch per slice;
  //   * anything else: the 128 x 128 kernel, one launch per linear.
  const int mid_min = kMfmaMidRows;
  const bool x_ok = aligned16(x) && K % 64 == 0 && (uint64_t)M * K * 2 < (1ull << 32);
  strata_q4_weight fast[kMaxGemmProblems];
  int nfast = 0;
  int64_t Nfast = 0;
  for (int i = 0; i < count; ++i) {
    bool f = false;
    if (M >= mid_min)
      f = x_ok && ws[i].N % 256 == 0 && aligned16(ws[i].w) &&
          (uint64_t)(Nfast + ws[i].N) * K / 2 < (1ull << 32);
    else
      f = aligned16(x) && strata_q4_skinny_fits(1, K, &ws[i], 1);
    if (f && nfast < kMaxGemmProblems) {
      fast[nfast++] = ws[i];
      Nfast += ws[i].N;
    } else {
      const int rc = strata_q4_gemm_launch(x, M, K, ws[i].w, ws[i].scales, ws[i].biases,
                                           (int)ws[i].N, ws[i].y, y_dtype, stream);
      if (rc) return rc;
    }
  }
  if (nfast == 0) return STRATA_OK;
  if (M < mid_min) {
    for (int r0 = 0; r0 < M; r0 += kSkinnyMaxRows) {
      const int mr = std::min(kSkinnyMaxRows, M - r0);
      strata_q4_weight sl[kMaxGemmProblems];
      for (int i = 0; i < nfast; ++i) {
        sl[i] = fast[i];
        sl[i].y = static_cast<char*>(fast[i].y) + (size_t)r0 * fast[i].N * ye;
      }
      const int rc = strata_q4_gemm_skinny(static_cast<const uint16_t*>(x) + (size_t)r0 * K, mr,
                                           K, sl, nfast, y_dtype, stream);
      if (rc) return rc;
    }
    return STRATA_OK;
  }
  // The decoder's load-time re-layout is used when it was built for exactly
  // these linears (all of them on this path, the same total N and K);
  // otherwise this call re-lays the weights out into the scratch arena,
  // ahead of the fp32 partial sums of split linears.
  const void* pk_in = packed && packed->buf && nfast == count && packed->N == Nfast &&
                              packed->K == K && packed->count == count
                          ? packed->buf
                          : nullptr;
  const size_t pb = strata_q4_gemm_mfma_part_bytes(M, K, fast, nfast);
  const size_t pk = pk_in ? 0 : (strata_q4_gemm_mfma_scratch(Nfast, K) + 255) / 256 * 256;
  void* scr = nullptr;
  if (pk + pb > 0) {
    const int rc = strata_ctx_scratch(ctx, pk + pb, &scr, stream);
    if (rc) return rc;
  }
  if (!pk_in) {
    const int rc = strata_q4_gemm_pack(fast, nfast, K, scr, stream);
    if (rc) return rc;
    pk_in = scr;
  }
  float* part = pb ? reinterpret_cast<float*>(static_cast<char*>(scr) + pk) : nullptr;
  return strata_q4_gemm_mfma_run(x, M, K, pk_in, fast, nfast, y_dtype, stream, part, pb);
}

int strata_q4_gemm(strata_ctx* ctx, const void* x, int M, int K, const uint32_t* w,
                   const uint16_t* s, const uint16_t* b, int N, void* y, int y_dtype,
                   void* stream) {
  const strata_q4_weight wt{w, s, b, N, y};
  return strata_q4_gemm_multi(ctx, x, M, K, &wt, 1, y_dtype, stream);
}
