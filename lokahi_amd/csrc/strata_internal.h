// Host-side declarations shared by the library's translation units: kernel
// launchers (defined in the .hip files) and the KV-cache object.
#pragma once

#include <vector>

#include "strata_common.h"

inline bool dtype_ok(int d) { return d == STRATA_F32 || d == STRATA_BF16; }
inline size_t dtype_size(int d) { return d == STRATA_F32 ? 4 : 2; }
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// GEMV prologue/epilogues used by the decode engine (bf16 x, M <= 8).
// mode 0: plain store; 1: SiLU pair of gate/up; 2: RoPE + KV append of
// q/k/v; 3: residual add in place (y is the residual stream).  norm_w != null
// applies RMSNorm (weight norm_w, eps) to x first.
struct GemvEpilogue {
  int mode;
  int head_dim, n_heads, n_kv_heads, lmax, pos0;
  const int* dpos;
  float theta;
  uint16_t* q_out;
  uint16_t* kc;
  uint16_t* vc;
  const uint16_t* norm_w;
  float eps;
  const float2* rope_table;  // (cos, sin) table [lmax][head_dim/2], required by mode 2
  const float2* rope_cur;    // with dpos: (cos, sin) [head_dim/2] of position *dpos
};
// Decode GEMV over the load-time "GEMV layout" (q4_gemv_mfma.hip): the
// linears of one launch re-laid out once into 16-row blocks for the 16x16x32
// bf16 matrix-core kernel.  perm: 0 rows in order (store / residual
// epilogues), 1 gate/up pairs (SiLU epilogue; ws = {gate, up}), 2 rotate-half
// pairs inside heads of head_dim rows (RoPE + KV append; ws = {q, k, v}).
constexpr int kGvMaxProblems = 8;
struct GemvLayout {
  void* buf = nullptr;  // codes, then the packed (scale, bias) words
  size_t code_bytes = 0, sb_bytes = 0;
  int K = 0, nt = 0, nrb = 0, perm = 0, head_dim = 0;
  int count = 0;                      // output problems (1 for perm 1)
  int rb0[kGvMaxProblems + 1] = {};  // first row block of each problem
  int64_t N[kGvMaxProblems] = {};     // output rows of each problem
};
// Batch rows of one layout launch: up to kGvMaxRows (5-8 rows run as two
// 4-row workgroups per row block in one grid).
constexpr int kGvMaxRows = 8;
// K % 64 == 0, K <= 16384 and 1 <= M <= 8.
bool strata_gemv_layout_fits(int K, int M);
int strata_gemv_layout_build(const strata_q4_weight* ws, int count, int K, int perm, int head_dim,
                             GemvLayout* out, void* stream);
void strata_gemv_layout_free(GemvLayout* L);
// bf16 x [M, K]; ys[i] is problem i's output (perm 1: act [M, N]); e (may be
// null) selects the prologue/epilogue as for strata_q4_gemv_epi.
int strata_gemv_layout_run(const GemvLayout& L, const void* x, int M, void* const* ys, int y_dtype,
                           const GemvEpilogue* e, void* stream);
int strata_q4_gemv_epi(strata_ctx* ctx, const void* x, int M, int K, const strata_q4_weight* ws,
                       int count, const GemvEpilogue& e, void* stream);
int strata_q4_gemv_resid(strata_ctx* ctx, const void* x, int M, int K, const strata_q4_weight* ws,
                         int count, void* stream);
int strata_q4_gemv(strata_ctx* ctx, const void* x, int x_dtype, int M, int K,
                   const strata_q4_weight* ws, int count, int y_dtype, void* stream);
int strata_bf16_gemv(strata_ctx* ctx, const void* x, int M, int K, const uint16_t* w, int N,
                     void* y, int y_dtype, void* stream);
int strata_q4_gemm_launch(const void* x, int M, int K, const uint32_t* w, const uint16_t* s,
                          const uint16_t* b, int N, void* y, int y_dtype, void* stream);
// Prefill q4 linear (bf16 x, M > 8): the hand-written fused-dequant MFMA
// kernels.
int strata_q4_gemm(strata_ctx* ctx, const void* x, int M, int K, const uint32_t* w,
                   const uint16_t* s, const uint16_t* b, int N, void* y, int y_dtype,
                   void* stream);
// 256-column-tile fused-dequant MFMA GEMM (M >= kMfmaMidRows on the default
// path).
// scratch: strata_q4_gemm_mfma_scratch(N, K) bytes, 16-byte aligned (the
// weight's per-call re-layout).
size_t strata_q4_gemm_mfma_scratch(int64_t N, int K);
// The linears of `ws` (same x; N of each a multiple of 256) in one launch of
// the 256-column-tile kernel, without a K split.
constexpr int kMaxGemmProblems = 8;
int strata_q4_gemm_mfma_launch(const void* x, int M, int K, const strata_q4_weight* ws, int count,
                               int y_dtype, void* scratch, void* stream);
// The same in two parts: the weights' re-layout into `packed`
// (strata_q4_gemm_mfma_scratch(sum of N, K) bytes, 16-byte aligned; done
// once at load time by the decoder), then GEMMs on it (the ws' w, scales and
// biases are not read, only N and y).
int strata_q4_gemm_pack(const strata_q4_weight* ws, int count, int K, void* packed, void* stream);
// Any M.  With `part` (fp32 scratch of part_bytes), linears whose tiles
// leave CUs idle split K over several workgroups and add the slices up in
// order (strata_q4_gemm_mfma_part_bytes sizes it); without it, no split.
int strata_q4_gemm_mfma_run(const void* x, int M, int K, const void* packed,
                            const strata_q4_weight* ws, int count, int y_dtype, void* stream,
                            float* part = nullptr, size_t part_bytes = 0);
size_t strata_q4_gemm_mfma_part_bytes(int M, int K, const strata_q4_weight* ws, int count);
// From this many rows the linears sharing x go to the 256-column MFMA kernel
// when every N is a multiple of 256 (STRATA_GEMM_MFMA_MIN_M overrides).
// (Measured on the 8B shapes: the skinny kernel is faster up to ~32 rows,
// this one from ~48.)
constexpr int kMfmaMidRows = 40;
// Prefill linears sharing x (M > 8 rows, bf16 x): one launch where the
// shapes allow, else one per linear.
// A load-time re-layout (strata_q4_gemm_pack) of `count` linears with N
// rows in all and width K; a call uses it only when it matches.
struct GemmPacked {
  const void* buf = nullptr;
  int64_t N = 0;
  int K = 0;
  int count = 0;
};
int strata_q4_gemm_multi(strata_ctx* ctx, const void* x, int M, int K, const strata_q4_weight* ws,
                         int count, int y_dtype, void* stream, const GemmPacked* packed = nullptr);
// Linears sharing x for a few rows (M <= kSkinnyMaxRows, K % 512 == 0, every
// N % 16 == 0, 16-byte aligned weights and x): one launch, each weight read once.
constexpr int kSkinnyMaxRows = 64;
bool strata_q4_skinny_fits(int M, int K, const strata_q4_weight* ws, int count);
int strata_q4_gemm_skinny(const void* x, int M, int K, const strata_q4_weight* ws, int count,
                          int y_dtype, void* stream);
// bf16 [N, K] = s*q + b (fp32, one RNE rounding) of a q4 triple; K % 64 == 0,
// w and out 16-byte aligned.
int strata_q4_dequant_launch(const uint32_t* w, const uint16_t* s, const uint16_t* b, int64_t N,
                             int K, uint16_t* out, void* stream);
int strata_attention_dispatch(strata_ctx* ctx, const void* q, int qd, const void* k, int kd,
                              const void* v, int vd, int64_t kv_bs, int64_t kv_hs,
                              const int32_t* qpos, int B, int Hq, int Hkv, int Lq, int Lk, int D,
                              int causal, float eps, void* out, const AttnExtra& ex,
                              void* stream);
int strata_attn_decode_splits(strata_ctx* ctx, int B, int Hkv, int Lcap);
int strata_rope_launch(void* q, void* k, const int32_t* pos, int B, int Hq, int Hkv, int L, int D,
                       float theta, int dtype, void* stream);
int strata_kv_copy_launch(const void* src, int src_dtype, void* dst, int dst_dtype, int B, int H,
                          int Lnew, int Lmax, int D, int pos0, void* stream);
int strata_rope_kv_fused_launch(const void* qs, const void* ks, const void* vs, int src_dtype,
                                int B, int Hq, int Hkv, int L, int D, int Lmax, int pos0,
                                const int* dpos, float theta, void* q_out, void* kc, void* vc,
                                int cache_dtype, void* stream, const void* rope_table = nullptr);
int strata_rmsnorm_launch(void* x, const void* res, const uint16_t* w, int64_t rows, int64_t H,
                          float eps, void* y, void* stream);
int strata_silu_mul_launch(const void* g, const void* u, int64_t n, void* a, void* stream);
int strata_add_launch(const void* x, const void* r, int64_t n, void* y, void* stream);
// Clears `bytes` bytes at p (16-byte aligned) with a kernel.
int strata_zero_fill_launch(void* p, int64_t bytes, void* stream);
int strata_embed_launch(const uint16_t* table, int64_t V, int64_t H, const int32_t* ids,
                        int64_t n, void* y, void* stream);
constexpr int kArgmaxBlocks = 128;  // workgroups per row of the first argmax stage
int strata_argmax_launch(const float* logits, int64_t rows, int64_t V, float temperature,
                         int32_t* out, void* partial, void* stream);
int strata_quantize_launch(const void* src, int dtype, int64_t N, int64_t K, int G, uint32_t* w,
                           uint16_t* s, uint16_t* b, void* stream);
// (cos, sin) of RoPE for positions 0..lmax-1 and pairs 0..D/2-1, evaluated
// exactly as the in-kernel RoPE evaluates them (bit-identical).
int strata_rope_table_launch(float2* table, int lmax, int D, float theta, void* stream);
// Records the step's tokens, advances {step, position, key count} and, when
// rope_cur is given, stages rope_table's row of the new position into it.
// Greedy argmax of B logit rows (two kernels: partials, then one workgroup
// that also records the tokens, gathers their embeddings into h and
// advances the counters like strata_decode_advance_launch).
int strata_decode_tail_launch(const float* logits, int B, int64_t V, float temperature,
                              void* partial, int32_t* ids, int32_t* out_tokens, int out_stride,
                              int* counters, const float2* rope_table, int lmax, int half,
                              float2* rope_cur, const uint16_t* table, int64_t H, void* h,
                              void* stream);
int strata_decode_advance_launch(const int32_t* ids, int B, int32_t* out_tokens, int out_stride,
                                 int* counters, const float2* rope_table, int lmax, int half,
                                 float2* rope_cur, void* stream);

struct strata_kv {
  strata_ctx* ctx;
  int layers, B, Hkv, Lmax, D, dtype;
  void* k;
  void* v;
  bool owned;
  std::vector<int> len;
  size_t layer_elems() const { return (size_t)B * Hkv * Lmax * D; }
  char* kl(int layer) const { return static_cast<char*>(k) + layer * layer_elems() * dtype_size(dtype); }
  char* vl(int layer) const { return static_cast<char*>(v) + layer * layer_elems() * dtype_size(dtype); }
};
