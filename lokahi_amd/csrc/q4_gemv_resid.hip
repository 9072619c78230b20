// q4 GEMV whose epilogue adds into the residual stream in place
// (its own translation unit, so the library's kernels build in parallel).
#include "q4_gemv_impl.h"

int strata_q4_gemv_resid(strata_ctx* ctx, const void* x, int M, int K, const strata_q4_weight* ws,
                         int count, void* stream) {
  STRATA_REQUIRE(count == 1, "residual epilogue takes one linear");
  const Q4Batch batch = make_batch(ws, count, EPI_RESID);
  const NormArgs na{nullptr, 0.f};
  return dispatch_q4<EPI_RESID, false, bf16_t, bf16_t>(ctx, x, M, K, batch, na, as_stream(stream));
}
