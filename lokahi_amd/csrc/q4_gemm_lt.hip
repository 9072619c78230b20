// Prefill q4 linear for long prompts: dequantize, then a library bf16 GEMM.
//
// Same maths as mx.quantized_matmul(transpose=True) (src/ollm/llama_mlx.py:53-74)
// on the prefill path.  At prefill sizes the GEMM is compute-bound and the
// weight is tiny next to it (gate projection of an 8B model at 8192 tokens:
// 29 MB of codes against 0.96 TFLOP), so the weight is expanded ONCE per call
// into a bf16 [N, K] tile (s*q + b in fp32, round-to-nearest-even: the values
// the fused kernel stages in LDS, bit for bit) and the product runs on
// hipBLASLt's tuned gfx950 MFMA kernels with fp32 accumulation.  The expansion
// is one HBM pass (K/2 bytes read, 2K written per row) and costs ~1-3% of the
// GEMM at 8k tokens.
//
// Layout: row-major Y[M, N] = X[M, K] W[N, K]^T is column-major
// Y^T (N x M, ld N) = op_T(W as K x N, ld K) * op_N(X^T as K x M, ld K).
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <cstdlib>
#include <map>
#include <tuple>

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

constexpr size_t kLtWorkspace = 64u << 20;

struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  bool ok = false;
};

}  // namespace

struct GemmLt {
  hipblasLtHandle_t handle = nullptr;
  void* workspace = nullptr;
  void* wdq = nullptr;  // bf16 weight tile [N, K]
  size_t wdq_bytes = 0;
  std::map<std::tuple<int, int, int, int>, Plan> plans;
};

namespace {

#define LT_CHECK(expr)                                                              \
  do {                                                                              \
    hipblasStatus_t _s = (expr);                                                    \
    if (_s != HIPBLAS_STATUS_SUCCESS)                                               \
      return strata_set_error(STRATA_EHIP, "%s failed: status %d", #expr, (int)_s); \
  } while (0)

int lt_init(strata_ctx* ctx) {
  if (ctx->lt) return STRATA_OK;
  auto* lt = new GemmLt();
  if (hipblasLtCreate(&lt->handle) != HIPBLAS_STATUS_SUCCESS) {
    delete lt;
    return strata_set_error(STRATA_EHIP, "hipblasLtCreate failed");
  }
  if (hipMalloc(&lt->workspace, kLtWorkspace) != hipSuccess) {
    hipblasLtDestroy(lt->handle);
    delete lt;
    return strata_set_error(STRATA_ENOMEM, "GEMM workspace allocation failed");
  }
  ctx->lt = lt;
  return STRATA_OK;
}

void plan_release(Plan& p) {
  if (p.a) hipblasLtMatrixLayoutDestroy(p.a);
  if (p.b) hipblasLtMatrixLayoutDestroy(p.b);
  if (p.c) hipblasLtMatrixLayoutDestroy(p.c);
  if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
}

// Plans are cached per (M, N, K, output dtype).  Prefill M is the prompt
// length, so the cache is bounded: past kMaxPlans entries it is emptied
// (the caller's stream is synchronized first: queued GEMMs may still use a
// plan's descriptors).
constexpr size_t kMaxPlans = 256;

int lt_plan(GemmLt* lt, int M, int N, int K, int y_dtype, void* stream, Plan** out) {
  auto key = std::make_tuple(M, N, K, y_dtype);
  auto it = lt->plans.find(key);
  if (it != lt->plans.end()) {
    *out = &it->second;
    return STRATA_OK;
  }
  if (lt->plans.size() >= kMaxPlans) {
    STRATA_HIP_CHECK(hipStreamSynchronize(as_stream(stream)));
    for (auto& kv : lt->plans) plan_release(kv.second);
    lt->plans.clear();
  }
  Plan p;
  const hipDataType yt = y_dtype == STRATA_F32 ? HIP_R_32F : HIP_R_16BF;
  const int32_t opT = HIPBLAS_OP_T, opN = HIPBLAS_OP_N;
  const uint64_t ws = kLtWorkspace;
  hipblasLtMatmulPreference_t pref = nullptr;
  hipblasLtMatmulHeuristicResult_t heur[1];
  int found = 0;
  // any failure releases what was created and leaves the shape unplanned
  bool built =
      hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opT, sizeof(opT)) ==
          HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opN, sizeof(opN)) ==
          HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16BF, K, N, K) == HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16BF, K, M, K) == HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatrixLayoutCreate(&p.c, yt, N, M, N) == HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                            sizeof(ws)) == HIPBLAS_STATUS_SUCCESS;
  built = built && hipblasLtMatmulAlgoGetHeuristic(lt->handle, p.desc, p.a, p.b, p.c, p.c, pref,
                                                   1, heur, &found) == HIPBLAS_STATUS_SUCCESS;
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  p.ok = built && found > 0 && heur[0].workspaceSize <= kLtWorkspace;
  if (p.ok) {
    p.algo = heur[0].algo;
  } else {
    plan_release(p);  // the shape falls back to the fused kernel
    p = Plan{};
  }
  auto ins = lt->plans.emplace(key, p);
  *out = &ins.first->second;
  return STRATA_OK;
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

void strata_gemm_lt_destroy(strata_ctx* ctx) {
  GemmLt* lt = ctx->lt;
  if (!lt) return;
  for (auto& kv : lt->plans) plan_release(kv.second);
  if (lt->wdq) (void)hipFree(lt->wdq);
  if (lt->workspace) (void)hipFree(lt->workspace);
  if (lt->handle) hipblasLtDestroy(lt->handle);
  delete lt;
  ctx->lt = nullptr;
}

int strata_q4_gemm_multi(strata_ctx* ctx, const void* x, int M, int K, const strata_q4_weight* ws,
                         int count, int y_dtype, void* stream, const void* packed) {
  // Default: the hand-written kernels only (fused dequant, bf16 MFMA).
  // STRATA_GEMM_LT_MIN_M > 0 opts into the dequantize + hipBLASLt path from
  // that many rows (comparison runs only).
  const char* e = getenv("STRATA_GEMM_LT_MIN_M");
  const int min_rows = e ? atoi(e) : 0;
  const size_t ye = y_dtype == STRATA_BF16 ? 2 : 4;
  if (min_rows > 0 && M >= min_rows) {
    for (int i = 0; i < count; ++i) {
      const int rc = strata_q4_gemm(ctx, x, M, K, ws[i].w, ws[i].scales, ws[i].biases,
                                    (int)ws[i].N, ws[i].y, y_dtype, stream);
      if (rc) return rc;
    }
    return STRATA_OK;
  }
  // Each linear goes its own way, so that it gives the same bits in a
  // fused call as alone:
  //   * from kMfmaMidRows rows, N a multiple of 256: the 256-column MFMA
  //     kernel over all rows (a partial last row tile; K split over several
  //     workgroups for linears with few tiles), the linears of one call in
  //     as few launches as their splits allow;
  //   * below that, shapes the skinny kernel takes (K % 512 == 0, N % 16 ==
  //     0): the skinny kernel, rows in slices of 64, one launch per slice;
  //   * anything else: the 128 x 128 kernel, one launch per linear.
  int mid_min = kMfmaMidRows;
  if (const char* em = getenv("STRATA_GEMM_MFMA_MIN_M")) mid_min = atoi(em);
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
  // The decoder's load-time re-layout covers all of the call's linears in
  // order; otherwise this call re-lays the weights out into the scratch
  // arena, ahead of the fp32 partial sums of split linears.
  const void* pk_in = nfast == count ? packed : nullptr;
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
  const char* e = getenv("STRATA_GEMM_LT_MIN_M");
  const int min_rows = e ? atoi(e) : 0;
  if (min_rows <= 0 || M < min_rows || !aligned16(y)) {
    const strata_q4_weight wt{w, s, b, N, y};
    return strata_q4_gemm_multi(ctx, x, M, K, &wt, 1, y_dtype, stream);
  }
  int rc = lt_init(ctx);
  if (rc) return rc;
  GemmLt* lt = ctx->lt;
  Plan* p = nullptr;
  rc = lt_plan(lt, M, N, K, y_dtype, stream, &p);
  if (rc) return rc;
  if (!p->ok)  // no library kernel for this shape: the fused-dequant kernel covers it
    return strata_q4_gemm_launch(x, M, K, w, s, b, N, y, y_dtype, stream);

  const size_t need = (size_t)N * K * 2;
  if (need > lt->wdq_bytes) {
    if (lt->wdq) {
      // The tile may still be read by queued work.
      STRATA_HIP_CHECK(hipDeviceSynchronize());
      STRATA_HIP_CHECK(hipFree(lt->wdq));
      lt->wdq = nullptr;
      lt->wdq_bytes = 0;
    }
    if (hipMalloc(&lt->wdq, need) != hipSuccess) {  // no room for the tile: fused kernel
      lt->wdq = nullptr;
      (void)hipGetLastError();
      return strata_q4_gemm_launch(x, M, K, w, s, b, N, y, y_dtype, stream);
    }
    lt->wdq_bytes = need;
  }
  rc = strata_q4_dequant_launch(w, s, b, N, K, static_cast<uint16_t*>(lt->wdq), stream);
  if (rc) return rc;
  const float alpha = 1.f, beta = 0.f;
  LT_CHECK(hipblasLtMatmul(lt->handle, p->desc, &alpha, lt->wdq, p->a, x, p->b, &beta, y, p->c, y,
                           p->c, &p->algo, lt->workspace, kLtWorkspace, as_stream(stream)));
  return STRATA_OK;
}
