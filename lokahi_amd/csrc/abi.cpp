// C ABI entry points of libstrata_hip.so: argument validation (messages mirror
// the reference's ValueErrors), the context and its scratch arena, the KV-cache
// object and the self-test gate.  Kernels live in the *.hip files.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "strata_common.h"

#include "strata_internal.h"

namespace {
thread_local std::string g_error;
}  // namespace

// Scratch of strata_attn_gqa_noalloc: a file-scope device array, so that
// entry point never allocates.  Each device holds its own copy until the
// process ends; host code reaches it only through the address
// hipGetSymbolAddress returns for the current device (kept in the ctx).
constexpr size_t kFixedScratchBytes = 16u << 20;
static __device__ __align__(256) float scratch[kFixedScratchBytes / sizeof(float)];

int strata_set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int strata_ctx_scratch(strata_ctx* ctx, size_t bytes, void** out, void* stream) {
  if (bytes > ctx->scratch_bytes) {
    // Growing synchronizes the device and frees the old arena: neither is
    // legal while a stream is being captured, and a graph captured earlier
    // would keep the freed address.  Capturing callers size the arena first.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(as_stream(stream), &cs) == hipSuccess &&
        cs != hipStreamCaptureStatusNone)
      return strata_set_error(STRATA_EINVAL,
                              "scratch arena must grow to %zu bytes during stream capture; "
                              "run the call once uncaptured first", bytes);
    if (ctx->scratch) {
      // The arena may still be read by queued work on any stream.
      STRATA_HIP_CHECK(hipDeviceSynchronize());
      STRATA_HIP_CHECK(hipFree(ctx->scratch));
      ctx->scratch = nullptr;
      ctx->scratch_bytes = 0;
    }
    size_t sz = bytes < (1u << 20) ? (1u << 20) : bytes;
    if (hipMalloc(&ctx->scratch, sz) != hipSuccess) {
      ctx->scratch = nullptr;
      return strata_set_error(STRATA_ENOMEM, "scratch allocation of %zu bytes failed", sz);
    }
    ctx->scratch_bytes = sz;
  }
  *out = ctx->scratch;
  return STRATA_OK;
}

extern "C" {

int strata_abi_version(void) { return STRATA_ABI_VERSION; }

const char* strata_last_error(void) { return g_error.c_str(); }

int strata_ctx_create(int device, strata_ctx** out) {
  STRATA_REQUIRE(out != nullptr, "ctx_create: out is NULL");
  *out = nullptr;
  int dev = device;
  if (dev < 0) STRATA_HIP_CHECK(hipGetDevice(&dev));
  STRATA_HIP_CHECK(hipSetDevice(dev));
  hipDeviceProp_t prop;
  STRATA_HIP_CHECK(hipGetDeviceProperties(&prop, dev));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return strata_set_error(STRATA_ENOTSUP, "device %d is %s; this library is built for gfx950",
                            dev, prop.gcnArchName);
  auto* c = new strata_ctx{};
  c->device = dev;
  c->num_cus = prop.multiProcessorCount;
  c->max_lds_per_block = 65536;  // portable launch limit for dynamic LDS
  c->scratch = nullptr;
  c->scratch_bytes = 0;
  c->fixed_scratch = nullptr;
  // With `dev` current: this device's address of the static scratch array.
  void* fixed = nullptr;
  const hipError_t se = hipGetSymbolAddress(&fixed, HIP_SYMBOL(scratch));
  if (se != hipSuccess || fixed == nullptr) {
    delete c;
    return strata_set_error(STRATA_EHIP, "hipGetSymbolAddress(scratch) failed: %s",
                            hipGetErrorString(se));
  }
  c->fixed_scratch = static_cast<float*>(fixed);
  *out = c;
  return STRATA_OK;
}

int strata_ctx_destroy(strata_ctx* ctx) {
  if (!ctx) return STRATA_OK;
  (void)hipDeviceSynchronize();
  if (ctx->scratch) (void)hipFree(ctx->scratch);
  delete ctx;
  return STRATA_OK;
}

// ------------------------------------------------------------------ linear
static int check_q4_common(strata_ctx* ctx, const void* x, int x_dtype, int64_t M, int64_t K,
                           int group_size, int bits, int y_dtype) {
  STRATA_REQUIRE(ctx != nullptr, "ctx is NULL");
  STRATA_REQUIRE(bits == 4, "only 4-bit quantization is supported (got bits=%d)", bits);
  STRATA_REQUIRE(group_size == 64, "only group_size 64 is supported (got %d)", group_size);
  STRATA_REQUIRE(dtype_ok(x_dtype) && dtype_ok(y_dtype), "unknown dtype code");
  STRATA_REQUIRE(M >= 0 && K > 0, "invalid shape M=%lld K=%lld", (long long)M, (long long)K);
  STRATA_REQUIRE(K % group_size == 0, "K=%lld must be divisible by group_size=%d", (long long)K,
                 group_size);
  STRATA_REQUIRE(M <= INT32_MAX && K <= INT32_MAX, "shape too large");
  STRATA_REQUIRE(M == 0 || (x != nullptr && aligned16(x)), "x must be a 16-byte aligned device pointer");
  return STRATA_OK;
}

int strata_linear_q4_multi(strata_ctx* ctx, const void* x, int x_dtype, int64_t M, int64_t K,
                           const strata_q4_weight* weights, int count, int group_size, int bits,
                           int y_dtype, void* stream) {
  int rc = check_q4_common(ctx, x, x_dtype, M, K, group_size, bits, y_dtype);
  if (rc) return rc;
  STRATA_REQUIRE(count >= 1 && count <= 8, "count must be in 1..8 (got %d)", count);
  int64_t rows = 0;
  for (int i = 0; i < count; ++i) {
    const strata_q4_weight& wt = weights[i];
    STRATA_REQUIRE(wt.N > 0 && wt.w && wt.scales && wt.biases && wt.y,
                   "weight %d: null pointer or N <= 0", i);
    STRATA_REQUIRE(aligned16(wt.w), "weight %d: packed weights must be 16-byte aligned", i);
    rows += wt.N;
  }
  STRATA_REQUIRE(rows <= INT32_MAX, "too many output rows");
  if (M == 0) return STRATA_OK;
  if (M > 8 && x_dtype == STRATA_BF16)
    return strata_q4_gemm_multi(ctx, x, (int)M, (int)K, weights, count, y_dtype, stream);
  return strata_q4_gemv(ctx, x, x_dtype, (int)M, (int)K, weights, count, y_dtype, stream);
}

int strata_linear_q4(strata_ctx* ctx, const void* x, int x_dtype, int64_t M, int64_t K,
                     const uint32_t* w, const uint16_t* scales, const uint16_t* biases, int64_t N,
                     int group_size, int bits, void* y, int y_dtype, void* stream) {
  strata_q4_weight wt{w, scales, biases, N, y};
  return strata_linear_q4_multi(ctx, x, x_dtype, M, K, &wt, 1, group_size, bits, y_dtype, stream);
}

struct strata_q4_layout {
  GemvLayout L;
};

int strata_q4_layout_create(strata_ctx* ctx, const strata_q4_weight* weights, int count, int64_t K,
                            strata_q4_layout** out) {
  STRATA_REQUIRE(ctx != nullptr && weights != nullptr && out != nullptr, "null argument");
  STRATA_REQUIRE(count >= 1 && count <= 8, "count must be in 1..8 (got %d)", count);
  STRATA_REQUIRE(K > 0 && K % 64 == 0 && K <= 16384,
                 "K=%lld must be a positive multiple of 64, at most 16384", (long long)K);
  for (int i = 0; i < count; ++i) {
    const strata_q4_weight& wt = weights[i];
    STRATA_REQUIRE(wt.N > 0 && wt.N <= (1 << 24) && wt.w && wt.scales && wt.biases,
                   "weight %d: null pointer or N outside 1..2^24", i);
  }
  auto* h = new strata_q4_layout{};
  const int rc = strata_gemv_layout_build(weights, count, (int)K, 0, 0, &h->L, nullptr);
  if (rc) {
    delete h;
    return rc;
  }
  if (hipStreamSynchronize(nullptr) != hipSuccess) {
    strata_gemv_layout_free(&h->L);
    delete h;
    return strata_set_error(STRATA_EHIP, "layout: re-layout kernels failed");
  }
  *out = h;
  return STRATA_OK;
}

int strata_q4_layout_destroy(strata_q4_layout* layout) {
  if (!layout) return STRATA_OK;
  strata_gemv_layout_free(&layout->L);
  delete layout;
  return STRATA_OK;
}

int strata_linear_q4_layout(strata_ctx* ctx, const void* x, int x_dtype, int64_t M,
                            const strata_q4_layout* layout, void* const* ys, int y_dtype,
                            void* stream) {
  STRATA_REQUIRE(ctx != nullptr && layout != nullptr && x != nullptr && ys != nullptr,
                 "null argument");
  STRATA_REQUIRE(x_dtype == STRATA_BF16, "the layout GEMV takes bf16 activations");
  STRATA_REQUIRE(dtype_ok(y_dtype), "unknown dtype code");
  STRATA_REQUIRE(M >= 0 && M <= kGvMaxRows, "M=%lld outside 0..%d", (long long)M, kGvMaxRows);
  STRATA_REQUIRE(aligned16(x), "x must be 16-byte aligned");
  for (int i = 0; i < layout->L.count; ++i) STRATA_REQUIRE(ys[i] != nullptr, "output %d is NULL", i);
  if (M == 0) return STRATA_OK;
  return strata_gemv_layout_run(layout->L, x, (int)M, ys, y_dtype, nullptr, stream);
}

int strata_linear_bf16(strata_ctx* ctx, const void* x, int x_dtype, int64_t M, int64_t K,
                       const uint16_t* w, int64_t N, void* y, int y_dtype, void* stream) {
  STRATA_REQUIRE(ctx != nullptr, "ctx is NULL");
  STRATA_REQUIRE(x_dtype == STRATA_BF16, "bf16 linear requires bf16 activations");
  STRATA_REQUIRE(dtype_ok(y_dtype), "unknown dtype code");
  STRATA_REQUIRE(M >= 0 && K > 0 && N > 0 && K % 8 == 0, "invalid shape (K must be a multiple of 8)");
  STRATA_REQUIRE(M <= INT32_MAX && K <= INT32_MAX && N <= INT32_MAX, "shape too large");
  STRATA_REQUIRE(aligned16(x) && aligned16(w), "x and w must be 16-byte aligned");
  if (M == 0) return STRATA_OK;
  // Each pass covers up to 4 x rows; more rows are processed in passes.
  return strata_bf16_gemv(ctx, x, (int)M, (int)K, w, (int)N, y, y_dtype, stream);
}

// -------------------------------------------------------------------- rope
int strata_rope(strata_ctx* ctx, void* q, void* k, const int32_t* pos, int B, int Hq, int Hkv,
                int L, int D, float theta, int dtype, void* stream) {
  STRATA_REQUIRE(ctx != nullptr, "ctx is NULL");
  STRATA_REQUIRE(dtype_ok(dtype), "unknown dtype code");
  STRATA_REQUIRE(B > 0 && L >= 0 && D > 0 && D % 2 == 0, "invalid shape (D must be even)");
  STRATA_REQUIRE(pos != nullptr || L == 0, "pos is NULL");
  STRATA_REQUIRE(theta > 0.f, "theta must be positive");
  if (L == 0) return STRATA_OK;
  return strata_rope_launch(q, k, pos, B, Hq, Hkv, L, D, theta, dtype, stream);
}

// ---------------------------------------------------------------- attention
int strata_attn_gqa(strata_ctx* ctx, const void* q, int q_dtype, const void* k, int k_dtype,
                    const void* v, int v_dtype, int64_t kv_batch_stride, int64_t kv_head_stride,
                    const int32_t* qpos, int B, int Hq, int Hkv, int Lq, int Lk, int D, int causal,
                    int q_blk, int k_blk, float eps, void* out, void* stream) {
  STRATA_REQUIRE(ctx != nullptr, "ctx is NULL");
  // Order and wording follow mlx_ops.py:48-67.
  STRATA_REQUIRE(q_blk > 0 && k_blk > 0, "attention block sizes must be positive");
  STRATA_REQUIRE(dtype_ok(q_dtype) && dtype_ok(k_dtype) && dtype_ok(v_dtype), "unknown dtype code");
  STRATA_REQUIRE(B > 0 && Lq >= 0 && Lk >= 0 && D > 0, "invalid shape");
  STRATA_REQUIRE(D <= 256, "head_dim %d > 256 is not supported", D);
  STRATA_REQUIRE(Hkv > 0 && Hq % Hkv == 0, "query heads must be divisible by key/value heads");
  STRATA_REQUIRE(!causal || Lk >= Lq, "causal attention requires key length >= query length");
  STRATA_REQUIRE(kv_head_stride >= (int64_t)Lk * D && kv_batch_stride >= kv_head_stride * Hkv,
                 "key/value strides are smaller than the key/value extent");
  if (Lq == 0) return STRATA_OK;
  STRATA_REQUIRE(q && out, "null tensor pointer");
  if (Lk == 0) {  // no keys: wv = 0 and s = 0, so out = 0 / eps = 0 (mlx_ops.py:146-147)
    return strata_zero_fill_launch(out, (int64_t)B * Hq * Lq * D * dtype_size(q_dtype), stream);
  }
  STRATA_REQUIRE(k && v, "null tensor pointer");
  return strata_attention_dispatch(ctx, q, q_dtype, k, k_dtype, v, v_dtype, kv_batch_stride,
                                   kv_head_stride, qpos, B, Hq, Hkv, Lq, Lk, D, causal, eps, out,
                                   AttnExtra{}, stream);
}

int strata_attn_gqa_noalloc(strata_ctx* ctx, const void* q, int q_dtype, const void* k,
                            int k_dtype, const void* v, int v_dtype, int64_t kv_batch_stride,
                            int64_t kv_head_stride, const int32_t* qpos, int B, int Hq, int Hkv,
                            int Lq, int Lk, int D, int causal, int q_blk, int k_blk, float eps,
                            void* out, void* stream) {
  STRATA_REQUIRE(ctx != nullptr, "ctx is NULL");
  STRATA_REQUIRE(ctx->fixed_scratch != nullptr, "ctx has no static scratch address");
  STRATA_REQUIRE(q_blk > 0 && k_blk > 0, "attention block sizes must be positive");
  STRATA_REQUIRE(dtype_ok(q_dtype) && dtype_ok(k_dtype) && dtype_ok(v_dtype), "unknown dtype code");
  STRATA_REQUIRE(B > 0 && Lq >= 0 && Lk >= 0 && D > 0, "invalid shape");
  STRATA_REQUIRE(D <= 256, "head_dim %d > 256 is not supported", D);
  STRATA_REQUIRE(Hkv > 0 && Hq % Hkv == 0, "query heads must be divisible by key/value heads");
  STRATA_REQUIRE(!causal || Lk >= Lq, "causal attention requires key length >= query length");
  STRATA_REQUIRE(kv_head_stride >= (int64_t)Lk * D && kv_batch_stride >= kv_head_stride * Hkv,
                 "key/value strides are smaller than the key/value extent");
  if (Lq == 0) return STRATA_OK;
  STRATA_REQUIRE(q && out, "null tensor pointer");
  if (Lk == 0)
    return strata_zero_fill_launch(out, (int64_t)B * Hq * Lq * D * dtype_size(q_dtype), stream);
  STRATA_REQUIRE(k && v, "null tensor pointer");
  // Only the split-K decode uses scratch (its partials, each written before
  // it is read, so nothing needs clearing).
  AttnExtra ex{};
  if (Lq == 1) {
    const int splits = strata_attn_decode_splits(ctx, B, Hkv, Lk);
    const size_t need = splits > 1 ? (size_t)B * Hq * part_stride(splits, D) * sizeof(float) : 0;
    STRATA_REQUIRE(need <= kFixedScratchBytes,
                   "attn_gqa_noalloc: %d x %d query heads over %d keys need %zu bytes of split-K "
                   "scratch; the static scratch holds %zu",
                   B, Hq, Lk, need, kFixedScratchBytes);
    ex.part = ctx->fixed_scratch;
    ex.part_splits = splits;
  }
  return strata_attention_dispatch(ctx, q, q_dtype, k, k_dtype, v, v_dtype, kv_batch_stride,
                                   kv_head_stride, qpos, B, Hq, Hkv, Lq, Lk, D, causal, eps, out,
                                   ex, stream);
}

// ---------------------------------------------------------------- KV cache
int strata_kv_create(strata_ctx* ctx, int layers, int B, int Hkv, int Lmax, int D, int dtype,
                     void* k_storage, void* v_storage, strata_kv** out) {
  STRATA_REQUIRE(ctx != nullptr && out != nullptr, "ctx/out is NULL");
  STRATA_REQUIRE(layers > 0 && B > 0 && Hkv > 0 && Lmax > 0 && D > 0, "invalid KV-cache geometry");
  STRATA_REQUIRE(dtype_ok(dtype), "unknown dtype code");
  STRATA_REQUIRE((k_storage == nullptr) == (v_storage == nullptr),
                 "k_storage and v_storage must both be given or both be NULL");
  auto* kv = new strata_kv{};
  kv->ctx = ctx;
  kv->layers = layers; kv->B = B; kv->Hkv = Hkv; kv->Lmax = Lmax; kv->D = D; kv->dtype = dtype;
  kv->len.assign(layers, 0);
  const size_t bytes = kv->layer_elems() * layers * dtype_size(dtype);
  if (k_storage) {
    kv->k = k_storage;
    kv->v = v_storage;
    kv->owned = false;
  } else {
    if (hipMalloc(&kv->k, bytes) != hipSuccess) {
      delete kv;
      return strata_set_error(STRATA_ENOMEM, "KV cache allocation of %zu bytes failed", bytes);
    }
    if (hipMalloc(&kv->v, bytes) != hipSuccess) {
      (void)hipFree(kv->k);
      delete kv;
      return strata_set_error(STRATA_ENOMEM, "KV cache allocation of %zu bytes failed", bytes);
    }
    kv->owned = true;
  }
  *out = kv;
  return STRATA_OK;
}

int strata_kv_destroy(strata_kv* kv) {
  if (!kv) return STRATA_OK;
  if (kv->owned) {
    (void)hipDeviceSynchronize();
    (void)hipFree(kv->k);
    (void)hipFree(kv->v);
  }
  delete kv;
  return STRATA_OK;
}

static int check_append(strata_kv* kv, int layer, int Lnew, int pos0) {
  STRATA_REQUIRE(kv != nullptr, "kv is NULL");
  STRATA_REQUIRE(layer >= 0, "layer_idx must be a non-negative integer");
  STRATA_REQUIRE(layer < kv->layers, "layer_idx %d is outside configured layer count %d", layer,
                 kv->layers);
  STRATA_REQUIRE(Lnew >= 0, "invalid append length %d", Lnew);
  const int prev = kv->len[layer];
  if (pos0 != prev)
    return strata_set_error(STRATA_EINVAL,
                            "cache_position must append exactly after the cached sequence; "
                            "expected start %d, got %d",
                            prev, pos0);
  STRATA_REQUIRE((int64_t)prev + Lnew <= kv->Lmax,
                 "KV cache capacity exceeded: %d + %d > Lmax %d", prev, Lnew, kv->Lmax);
  return STRATA_OK;
}

int strata_kv_append(strata_kv* kv, int layer, const void* k_new, const void* v_new, int src_dtype,
                     int Lnew, int pos0, void* stream) {
  int rc = check_append(kv, layer, Lnew, pos0);
  if (rc) return rc;
  STRATA_REQUIRE(dtype_ok(src_dtype), "unknown dtype code");
  if (Lnew == 0) return STRATA_OK;
  rc = strata_kv_copy_launch(k_new, src_dtype, kv->kl(layer), kv->dtype, kv->B, kv->Hkv, Lnew,
                             kv->Lmax, kv->D, pos0, stream);
  if (rc) return rc;
  rc = strata_kv_copy_launch(v_new, src_dtype, kv->vl(layer), kv->dtype, kv->B, kv->Hkv, Lnew,
                             kv->Lmax, kv->D, pos0, stream);
  if (rc) return rc;
  kv->len[layer] = pos0 + Lnew;
  return STRATA_OK;
}

int strata_kv_restore(strata_kv* kv, int layer, const void* k_src, const void* v_src,
                      int src_dtype, int L, void* stream) {
  STRATA_REQUIRE(kv != nullptr, "kv is NULL");
  STRATA_REQUIRE(layer >= 0 && layer < kv->layers,
                 "layer_idx %d is outside configured layer count %d", layer, kv->layers);
  STRATA_REQUIRE(L >= 0 && L <= kv->Lmax, "restored length %d exceeds the cache capacity %d", L,
                 kv->Lmax);
  STRATA_REQUIRE(L == 0 || (k_src != nullptr && v_src != nullptr), "null key/value snapshot");
  STRATA_REQUIRE(dtype_ok(src_dtype), "unknown dtype code");
  if (L > 0) {
    int rc = strata_kv_copy_launch(k_src, src_dtype, kv->kl(layer), kv->dtype, kv->B, kv->Hkv, L,
                                   kv->Lmax, kv->D, 0, stream);
    if (rc) return rc;
    rc = strata_kv_copy_launch(v_src, src_dtype, kv->vl(layer), kv->dtype, kv->B, kv->Hkv, L,
                               kv->Lmax, kv->D, 0, stream);
    if (rc) return rc;
  }
  kv->len[layer] = L;
  return STRATA_OK;
}

int strata_rope_kv_append(strata_kv* kv, int layer, const void* q_src, const void* k_src,
                          const void* v_src, int src_dtype, int Hq, int L, int pos0, float theta,
                          void* q_out, void* stream) {
  int rc = check_append(kv, layer, L, pos0);
  if (rc) return rc;
  STRATA_REQUIRE(dtype_ok(src_dtype), "unknown dtype code");
  STRATA_REQUIRE(Hq > 0 && Hq % kv->Hkv == 0, "query heads must be divisible by key/value heads");
  STRATA_REQUIRE(kv->D % 2 == 0, "head_dim must be even for RoPE");
  STRATA_REQUIRE(theta > 0.f, "theta must be positive");
  if (L == 0) return STRATA_OK;
  rc = strata_rope_kv_fused_launch(q_src, k_src, v_src, src_dtype, kv->B, Hq, kv->Hkv, L, kv->D,
                                   kv->Lmax, pos0, nullptr, theta, q_out, kv->kl(layer), kv->vl(layer),
                                   kv->dtype, stream);
  if (rc) return rc;
  kv->len[layer] = pos0 + L;
  return STRATA_OK;
}

int strata_kv_view(strata_kv* kv, int layer, void** k, void** v, int64_t* batch_stride,
                   int64_t* head_stride, int* length) {
  STRATA_REQUIRE(kv != nullptr, "kv is NULL");
  STRATA_REQUIRE(layer >= 0 && layer < kv->layers, "layer_idx %d is outside configured layer count %d",
                 layer, kv->layers);
  if (k) *k = kv->kl(layer);
  if (v) *v = kv->vl(layer);
  if (batch_stride) *batch_stride = (int64_t)kv->Hkv * kv->Lmax * kv->D;
  if (head_stride) *head_stride = (int64_t)kv->Lmax * kv->D;
  if (length) *length = kv->len[layer];
  return STRATA_OK;
}

int strata_kv_len(strata_kv* kv, int layer, int* length) {
  STRATA_REQUIRE(kv != nullptr && length != nullptr, "kv/length is NULL");
  if (layer < 0) {  // max over layers (get_seq_length(None), mlx_kvcache.py:169-171)
    int m = 0;
    for (int l : kv->len) m = l > m ? l : m;
    *length = m;
    return STRATA_OK;
  }
  STRATA_REQUIRE(layer < kv->layers, "layer_idx %d is outside configured layer count %d", layer,
                 kv->layers);
  *length = kv->len[layer];
  return STRATA_OK;
}

int strata_kv_clear(strata_kv* kv) {
  STRATA_REQUIRE(kv != nullptr, "kv is NULL");
  for (int& l : kv->len) l = 0;
  return STRATA_OK;
}

// ------------------------------------------------------------------- glue
int strata_rmsnorm(strata_ctx* ctx, void* x, const void* residual, const uint16_t* w, int64_t rows,
                   int64_t H, float eps, void* y, void* stream) {
  STRATA_REQUIRE(ctx && x && w && y, "null pointer");
  STRATA_REQUIRE(rows >= 0 && H > 0, "invalid shape");
  if (rows == 0) return STRATA_OK;
  return strata_rmsnorm_launch(x, residual, w, rows, H, eps, y, stream);
}

int strata_silu_mul(strata_ctx* ctx, const void* g, const void* u, int64_t n, void* a,
                    void* stream) {
  STRATA_REQUIRE(ctx && g && u && a && n >= 0, "invalid arguments");
  if (n == 0) return STRATA_OK;
  return strata_silu_mul_launch(g, u, n, a, stream);
}

int strata_add(strata_ctx* ctx, const void* x, const void* r, int64_t n, void* y, void* stream) {
  STRATA_REQUIRE(ctx && x && r && y && n >= 0, "invalid arguments");
  if (n == 0) return STRATA_OK;
  return strata_add_launch(x, r, n, y, stream);
}

int strata_embed(strata_ctx* ctx, const uint16_t* table, int64_t V, int64_t H, const int32_t* ids,
                 int64_t n, void* y, void* stream) {
  STRATA_REQUIRE(ctx && table && ids && y && V > 0 && H > 0 && n >= 0, "invalid arguments");
  if (n == 0) return STRATA_OK;
  return strata_embed_launch(table, V, H, ids, n, y, stream);
}

int strata_argmax(strata_ctx* ctx, const float* logits, int64_t rows, int64_t V, int32_t* out,
                  void* stream) {
  STRATA_REQUIRE(ctx && logits && out && rows >= 0 && V > 0 && V <= INT32_MAX, "invalid arguments");
  if (rows == 0) return STRATA_OK;
  void* part = nullptr;
  const int rc = strata_ctx_scratch(ctx, (size_t)rows * kArgmaxBlocks * 8, &part, stream);
  if (rc) return rc;
  return strata_argmax_launch(logits, rows, V, 1.0f, out, part, stream);
}

int strata_dequantize_q4(strata_ctx* ctx, const uint32_t* w, const uint16_t* scales,
                         const uint16_t* biases, int64_t N, int64_t K, int group_size, int bits,
                         uint16_t* out, void* stream) {
  STRATA_REQUIRE(ctx && w && scales && biases && out, "null pointer");
  STRATA_REQUIRE(bits == 4, "only 4-bit quantization is supported (got bits=%d)", bits);
  STRATA_REQUIRE(group_size == 64, "only group_size 64 is supported (got %d)", group_size);
  STRATA_REQUIRE(N >= 0 && K > 0 && K % group_size == 0, "K must be divisible by group_size");
  STRATA_REQUIRE(K <= INT32_MAX && N * (K / 32) <= (int64_t)UINT32_MAX * 256, "shape too large");
  STRATA_REQUIRE(aligned16(w) && aligned16(out), "w and out must be 16-byte aligned");
  return strata_q4_dequant_launch(w, scales, biases, N, (int)K, out, stream);
}

int strata_quantize_q4(strata_ctx* ctx, const void* wsrc, int w_dtype, int64_t N, int64_t K,
                       int group_size, uint32_t* w, uint16_t* scales, uint16_t* biases,
                       void* stream) {
  STRATA_REQUIRE(ctx && wsrc && w && scales && biases, "null pointer");
  STRATA_REQUIRE(dtype_ok(w_dtype), "unknown dtype code");
  STRATA_REQUIRE(group_size == 64, "only group_size 64 is supported (got %d)", group_size);
  STRATA_REQUIRE(N > 0 && K > 0 && K % group_size == 0, "K must be divisible by group_size");
  return strata_quantize_launch(wsrc, w_dtype, N, K, group_size, w, scales, biases, stream);
}

// ---------------------------------------------------------------- selftest
int strata_selftest(strata_ctx* ctx, char* json, size_t cap) {
  STRATA_REQUIRE(ctx != nullptr && json != nullptr && cap > 0, "invalid arguments");
  // q4 GEMV: N=64 rows, K=128; codes (n + k) % 16, scale 1/16, bias -0.5, x = (k%7 - 3)/4.
  const int N = 64, K = 128, G = 64;
  std::vector<uint32_t> w(N * K / 8, 0);
  std::vector<uint16_t> s(N * K / G), b(N * K / G);
  std::vector<uint16_t> x(K);
  auto to_bf = [](float f) { uint32_t u; std::memcpy(&u, &f, 4); return (uint16_t)((u + 0x7fff + ((u >> 16) & 1)) >> 16); };
  auto from_bf = [](uint16_t h) { uint32_t u = (uint32_t)h << 16; float f; std::memcpy(&f, &u, 4); return f; };
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < K; ++k) w[(n * K + k) / 8] |= (uint32_t)((n + k) % 16) << (4 * (k % 8));
  for (size_t i = 0; i < s.size(); ++i) { s[i] = to_bf(1.0f / 16); b[i] = to_bf(-0.5f); }
  for (int k = 0; k < K; ++k) x[k] = to_bf((k % 7 - 3) / 4.0f);
  std::vector<float> ref(N);
  for (int n = 0; n < N; ++n) {
    double acc = 0;
    for (int k = 0; k < K; ++k) {
      const int q = (n + k) % 16;
      acc += (double)from_bf(x[k]) * (from_bf(s[n * 2 + k / G]) * q + from_bf(b[n * 2 + k / G]));
    }
    ref[n] = (float)acc;
  }
  void *dw = nullptr, *ds = nullptr, *db = nullptr, *dx = nullptr, *dy = nullptr;
  int rc = STRATA_OK;
  float max_err = INFINITY;
  bool ok = false;
  std::vector<float> y(N);
  if (hipMalloc(&dw, w.size() * 4) == hipSuccess && hipMalloc(&ds, s.size() * 2) == hipSuccess &&
      hipMalloc(&db, b.size() * 2) == hipSuccess && hipMalloc(&dx, x.size() * 2) == hipSuccess &&
      hipMalloc(&dy, N * 4) == hipSuccess) {
    const bool copied =
        hipMemcpy(dw, w.data(), w.size() * 4, hipMemcpyHostToDevice) == hipSuccess &&
        hipMemcpy(ds, s.data(), s.size() * 2, hipMemcpyHostToDevice) == hipSuccess &&
        hipMemcpy(db, b.data(), b.size() * 2, hipMemcpyHostToDevice) == hipSuccess &&
        hipMemcpy(dx, x.data(), x.size() * 2, hipMemcpyHostToDevice) == hipSuccess;
    rc = copied ? strata_linear_q4(ctx, dx, STRATA_BF16, 1, K, (const uint32_t*)dw,
                                   (const uint16_t*)ds, (const uint16_t*)db, N, G, 4, dy,
                                   STRATA_F32, nullptr)
                : strata_set_error(STRATA_EHIP, "selftest: host-to-device copy failed");
    if (rc == STRATA_OK && hipDeviceSynchronize() == hipSuccess &&
        hipMemcpy(y.data(), dy, N * 4, hipMemcpyDeviceToHost) == hipSuccess) {
      max_err = 0.f;
      for (int n = 0; n < N; ++n) max_err = fmaxf(max_err, fabsf(y[n] - ref[n]) / (1.f + fabsf(ref[n])));
      ok = max_err <= 1e-4f;
    }
  }
  for (void* p : {dw, ds, db, dx, dy})
    if (p) (void)hipFree(p);
  snprintf(json, cap,
           "{\"schema_version\":1,\"backend\":\"hip\",\"operation\":\"linear_q4_gemv\","
           "\"device\":%d,\"compute_units\":%d,\"dispatch_success\":%s,"
           "\"numerical_max_error\":%.9g,\"threshold\":1e-4}",
           ctx->device, ctx->num_cus, ok ? "true" : "false", (double)max_err);
  if (rc) return rc;
  return ok ? STRATA_OK : strata_set_error(STRATA_EHIP, "selftest failed (max error %g)", (double)max_err);
}

}  // extern "C"
