// q4 GEMV with the decode engine's prologue/epilogues (RMSNorm, SiLU pair,
// RoPE + KV append, residual add); see q4_gemv_impl.h.
#include "q4_gemv_impl.h"

int strata_q4_gemv_epi(strata_ctx* ctx, const void* x, int M, int K, const strata_q4_weight* ws,
                       int count, const GemvEpilogue& e, void* stream) {
  STRATA_REQUIRE(e.mode == EPI_STORE || e.mode == EPI_SILU_PAIR || e.mode == EPI_ROPE_KV ||
                     e.mode == EPI_RESID,
                 "unknown GEMV epilogue");
  STRATA_REQUIRE(M >= 1 && M <= 8 && K % 64 == 0, "GEMV epilogue: unsupported shape M=%d K=%d",
                 M, K);
  Q4Batch batch = make_batch(ws, count, e.mode);
  if (e.mode == EPI_SILU_PAIR)
    STRATA_REQUIRE(count == 2 && ws[0].N == ws[1].N, "SiLU pair epilogue needs gate/up of one size");
  if (e.mode == EPI_ROPE_KV) {
    STRATA_REQUIRE(count == 3 && e.head_dim % 2 == 0 &&
                       ws[0].N == (int64_t)e.n_heads * e.head_dim &&
                       ws[1].N == (int64_t)e.n_kv_heads * e.head_dim && ws[2].N == ws[1].N,
                   "RoPE/KV epilogue needs q/k/v of [Hq*D, Hkv*D, Hkv*D] rows");
    batch.head_dim = e.head_dim;
    batch.n_heads = e.n_heads;
    batch.n_kv_heads = e.n_kv_heads;
    batch.lmax = e.lmax;
    batch.pos0 = e.pos0;
    batch.dpos = e.dpos;
    batch.theta = e.theta;
    STRATA_REQUIRE(e.rope_table != nullptr, "RoPE/KV epilogue needs the (cos, sin) table");
    batch.rope_table = e.rope_table;
    STRATA_REQUIRE(e.dpos == nullptr || e.rope_cur != nullptr,
                   "RoPE/KV epilogue with a device position needs the staged (cos, sin) row");
    batch.rope_cur = e.rope_cur;
    batch.q_out = e.q_out;
    batch.kc = e.kc;
    batch.vc = e.vc;
  }
  const NormArgs na{e.norm_w, e.eps};
  hipStream_t s = as_stream(stream);
  const bool norm = e.norm_w != nullptr;
  switch (e.mode) {
    case EPI_STORE:
      return norm ? dispatch_q4<EPI_STORE, true, bf16_t, bf16_t>(ctx, x, M, K, batch, na, s)
                  : dispatch_q4<EPI_STORE, false, bf16_t, bf16_t>(ctx, x, M, K, batch, na, s);
    case EPI_SILU_PAIR:
      return norm ? dispatch_q4<EPI_SILU_PAIR, true, bf16_t, bf16_t>(ctx, x, M, K, batch, na, s)
                  : dispatch_q4<EPI_SILU_PAIR, false, bf16_t, bf16_t>(ctx, x, M, K, batch, na, s);
    case EPI_ROPE_KV:
      if (e.dpos)
        return norm ? dispatch_q4<EPI_ROPE_KV_DEV, true, bf16_t, bf16_t>(ctx, x, M, K, batch, na, s)
                    : dispatch_q4<EPI_ROPE_KV_DEV, false, bf16_t, bf16_t>(ctx, x, M, K, batch, na, s);
      return norm ? dispatch_q4<EPI_ROPE_KV, true, bf16_t, bf16_t>(ctx, x, M, K, batch, na, s)
                  : dispatch_q4<EPI_ROPE_KV, false, bf16_t, bf16_t>(ctx, x, M, K, batch, na, s);
    default:
      STRATA_REQUIRE(count == 1 && !norm, "residual epilogue takes one linear and no RMSNorm");
      return strata_q4_gemv_resid(ctx, x, M, K, ws, count, stream);
  }
}

