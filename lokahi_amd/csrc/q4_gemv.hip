// Entry points of the decode-side q4 GEMV and the bf16 GEMV (lm_head); the
// kernels and their design notes are in q4_gemv_impl.h.
#include "q4_gemv_impl.h"

int strata_q4_gemv(strata_ctx* ctx, const void* x, int x_dtype, int M, int K,
                   const strata_q4_weight* ws, int count, int y_dtype, void* stream) {
  Q4Batch batch = make_batch(ws, count, EPI_STORE);
  hipStream_t s = as_stream(stream);
  const NormArgs na{nullptr, 0.f};
  if (x_dtype == STRATA_BF16 && y_dtype == STRATA_BF16)
    return dispatch_q4<EPI_STORE, false, bf16_t, bf16_t>(ctx, x, M, K, batch, na, s);
  if (x_dtype == STRATA_BF16 && y_dtype == STRATA_F32)
    return dispatch_q4<EPI_STORE, false, bf16_t, float>(ctx, x, M, K, batch, na, s);
  if (x_dtype == STRATA_F32 && y_dtype == STRATA_F32)
    return dispatch_q4<EPI_STORE, false, float, float>(ctx, x, M, K, batch, na, s);
  if (x_dtype == STRATA_F32 && y_dtype == STRATA_BF16)
    return dispatch_q4<EPI_STORE, false, float, bf16_t>(ctx, x, M, K, batch, na, s);
  return strata_set_error(STRATA_EINVAL, "q4 GEMV: unsupported dtype pair (%d, %d)", x_dtype,
                          y_dtype);
}

int strata_bf16_gemv(strata_ctx* ctx, const void* x, int M, int K, const uint16_t* w, int N,
                     void* y, int y_dtype, void* stream) {
  const int MT = M >= 4 ? 4 : (M >= 2 ? 2 : 1);
  const size_t lds = (size_t)MT * K * 2;
  STRATA_REQUIRE((int64_t)lds <= ctx->max_lds_per_block, "bf16 GEMV: K=%d too large", K);
  // 8 uint4 (64 weights) per lane per chunk, one row per wave, 8 waves per WG.
  constexpr int NW = 8, R = 1, U = 8;
  dim3 grid((N + NW * R - 1) / (NW * R), (M + MT - 1) / MT);
  hipStream_t s = as_stream(stream);
  const uint16_t* xx = reinterpret_cast<const uint16_t*>(x);
  const uint4* ww = reinterpret_cast<const uint4*>(w);
  if (MT == 1 && K >= 4096) {
    // batch 1, K >= 4096: 16 waves per workgroup, x staged after the first
    // weight loads (8B lm_head, 1.05 GB: 159 -> 152-153 us against 8 waves
    // with x first; the 3B head, K = 3072, stays on 8 waves: 112 against 114 us)
    constexpr int NW1 = 16;
    const dim3 g1((N + NW1 - 1) / NW1);
    if (y_dtype == STRATA_F32)
      hipLaunchKernelGGL((bf16_gemv_kernel<NW1, 1, U, 1, float, 0>), g1, dim3(NW1 * 64), lds, s, xx,
                         M, K, ww, N, reinterpret_cast<float*>(y));
    else
      hipLaunchKernelGGL((bf16_gemv_kernel<NW1, 1, U, 1, bf16_t, 0>), g1, dim3(NW1 * 64), lds, s, xx,
                         M, K, ww, N, reinterpret_cast<bf16_t*>(y));
    STRATA_HIP_CHECK(hipGetLastError());
    return STRATA_OK;
  }
  // x ahead of the weights when each batch row is one uint4 per thread
  // (K = 4096: the lm_head of the Llama-3-8B shape)
  const int xi = K / 8 == NW * 64 ? MT : 0;
#define STRATA_BF16_LAUNCH(MTV, XIV)                                                           \
  if (MT == MTV && xi == XIV) {                                                                \
    if (y_dtype == STRATA_F32)                                                                 \
      hipLaunchKernelGGL((bf16_gemv_kernel<NW, R, U, MTV, float, XIV>), grid, dim3(NW * 64),   \
                         lds, s, xx, M, K, ww, N, reinterpret_cast<float*>(y));                \
    else                                                                                       \
      hipLaunchKernelGGL((bf16_gemv_kernel<NW, R, U, MTV, bf16_t, XIV>), grid, dim3(NW * 64),  \
                         lds, s, xx, M, K, ww, N, reinterpret_cast<bf16_t*>(y));               \
    STRATA_HIP_CHECK(hipGetLastError());                                                       \
    return STRATA_OK;                                                                          \
  }
  STRATA_BF16_LAUNCH(1, 1)
  STRATA_BF16_LAUNCH(1, 0)
  STRATA_BF16_LAUNCH(2, 2)
  STRATA_BF16_LAUNCH(2, 0)
  STRATA_BF16_LAUNCH(4, 4)
  STRATA_BF16_LAUNCH(4, 0)
#undef STRATA_BF16_LAUNCH
  return strata_set_error(STRATA_EINVAL, "bf16 GEMV: no kernel for batch tile %d", MT);
}
