/*
 * strata_hip.h — C ABI of the MI355X (gfx950) Strata hot-path library.
 *
 * This is the drop-in boundary for the reference's per-token inference path
 * (Ikaikaalika/lokahi, Python package `ollm`).  Each entry point names the
 * reference interface it replaces (paths relative to the reference root).
 * The reference binds its compute through Python; the binding for this
 * library is ctypes (lokahi_amd/_abi.py), registered as the "hip" backend in
 * the same registry as `MLXBackend` (src/ollm/backends/base.py:50-80,
 * src/ollm/backends/__init__.py:22-24).
 *
 * Conventions
 *   - All tensor pointers are DEVICE pointers owned by the caller, except the
 *     KV-cache storage a strata_kv allocates itself when given none.
 *   - bf16 tensors are uint16_t bit patterns; dtype codes are STRATA_F32 /
 *     STRATA_BF16.
 *   - `stream` is a hipStream_t passed as void* (NULL = default stream).  All
 *     compute is asynchronous on that stream; the caller synchronizes.
 *   - Every function returns STRATA_OK (0) or a negative status; the reason
 *     is in strata_last_error() (thread-local).
 *   - A strata_ctx is not thread-safe: use one per thread or serialize.
 */
#ifndef STRATA_HIP_H
#define STRATA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define STRATA_ABI_VERSION 2

enum strata_status {
  STRATA_OK = 0,
  STRATA_EHIP = -5,      /* a HIP runtime call failed */
  STRATA_ENOMEM = -12,   /* device allocation failed */
  STRATA_EINVAL = -22,   /* invalid argument / shape / contract violation */
  STRATA_ENOTSUP = -95   /* valid request this build does not implement */
};

enum strata_dtype { STRATA_F32 = 0, STRATA_BF16 = 1 };

typedef struct strata_ctx strata_ctx;
typedef struct strata_kv strata_kv;

/* ---------------------------------------------------------------- library */
int strata_abi_version(void);
const char* strata_last_error(void);

/* Create a context bound to HIP device `device` (the current device if < 0). */
int strata_ctx_create(int device, strata_ctx** out);
int strata_ctx_destroy(strata_ctx* ctx);

/* Self-test gate: runs one tiny q4 GEMV on the device, checks it against
 * host arithmetic and writes a JSON envelope
 * {"schema_version":1,"backend":"hip","operation":...,"dispatch_success":...,
 *  "numerical_max_error":...} into `json` (capacity `cap`).  Mirrors the
 * fail-closed probe contract of src/ollm/backends/metal_backend.py:74-163. */
int strata_selftest(strata_ctx* ctx, char* json, size_t cap);

/* ---------------------------------------------------------- quantized linear
 * Replaces `_linear` -> `mx.quantized_matmul(x, w, scales, biases,
 * transpose=True, group_size, bits, mode="affine")`
 * (src/ollm/llama_mlx.py:53-74; callers 257-268, 313-316, 393-408, 902-910).
 *   x       [M, K]   x_dtype (f32 or bf16)
 *   w       [N, K/8] uint32, element k = nibble k%8 of word k/8 (LSB first)
 *   scales  [N, K/group] bf16, biases [N, K/group] bf16
 *   y       [M, N]   y_dtype;  y = x @ (scales*q + biases).T, fp32 accumulate
 * Rejects bits != 4, group_size != 64, K % group_size != 0 with STRATA_EINVAL
 * (mode is always "affine"). M <= 8 runs the streaming GEMV; larger M
 * (bf16 x only) runs the fused-dequant bf16 MFMA GEMMs, which re-lay the
 * weight out into the context's scratch arena for the call: issue large-M
 * calls of one ctx on one stream (or order the streams). */
int strata_linear_q4(strata_ctx* ctx, const void* x, int x_dtype, int64_t M, int64_t K,
                     const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                     int64_t N, int group_size, int bits, void* y, int y_dtype,
                     void* stream);

/* Several q4 linears sharing one input x (q/k/v of llama_mlx.py:257-268, or
 * gate/up of llama_mlx.py:395-407) in one launch.  count <= 8. */
typedef struct strata_q4_weight {
  const uint32_t* w;
  const uint16_t* scales;
  const uint16_t* biases;
  int64_t N;
  void* y;
} strata_q4_weight;

int strata_linear_q4_multi(strata_ctx* ctx, const void* x, int x_dtype, int64_t M,
                           int64_t K, const strata_q4_weight* weights, int count,
                           int group_size, int bits, int y_dtype, void* stream);

/* Decode linears over a load-time weight layout.  The reference places each
 * layer's quantized tensors on the device once when it loads the layer
 * (`_load_layer_weights` / `_assign_layer_weight`,
 * src/ollm/llama_mlx.py:498-580) and every step then runs `_linear` on them
 * (53-74).  strata_q4_layout_create is that load step for linears sharing x
 * (q/k/v, or gate/up): it copies the MLX-layout triples into the layout the
 * matrix-core decode GEMV streams (16-row blocks, scale and bias packed next
 * to the codes, K padded to a multiple of 1024); the MLX tensors may be
 * freed afterwards.  strata_linear_q4_layout then computes
 * y_i = x @ (scales_i*q_i + biases_i).T for 1 <= M <= 8 bf16 rows, fp32
 * accumulate, y_dtype f32 or bf16 (ys[i] is [M, N_i]).
 * Requirements: K % 64 == 0, K <= 16384, count 1..8, group_size 64, 4 bits.
 * The layout is read-only after creation: calls may share it. */
typedef struct strata_q4_layout strata_q4_layout;
int strata_q4_layout_create(strata_ctx* ctx, const strata_q4_weight* weights, int count,
                            int64_t K, strata_q4_layout** out);
int strata_q4_layout_destroy(strata_q4_layout* layout);
int strata_linear_q4_layout(strata_ctx* ctx, const void* x, int x_dtype, int64_t M,
                            const strata_q4_layout* layout, void* const* ys, int y_dtype,
                            void* stream);

/* Dense bf16-weight linear y = x @ W.T, W [N, K] bf16, fp32 accumulate.
 * Replaces the unquantized `_linear` branch `mx.matmul(x, weight.T)`
 * (src/ollm/llama_mlx.py:64-65) used for the bf16 lm_head (886-910). */
int strata_linear_bf16(strata_ctx* ctx, const void* x, int x_dtype, int64_t M, int64_t K,
                       const uint16_t* w, int64_t N, void* y, int y_dtype, void* stream);

/* ------------------------------------------------------------------- RoPE
 * Replaces MLXRotaryEmbedding + apply_rotary_pos_emb_mlx / rotate_half
 * (src/ollm/llama_mlx.py:95-182): non-interleaved rotate-half RoPE,
 * inv_freq[i] = 1/theta^(2i/D).  In place on q [B,Hq,L,D] and k [B,Hkv,L,D]
 * (either may be NULL); pos int32 [B,L] device pointer. */
int strata_rope(strata_ctx* ctx, void* q, void* k, const int32_t* pos, int B, int Hq,
                int Hkv, int L, int D, float theta, int dtype, void* stream);

/* --------------------------------------------------------------- attention
 * Replaces online_chunked_grouped_attention_mx (src/ollm/backends/mlx_ops.py:32-152)
 * and, with causal = 0, online_chunked_grouped_attention_rope_no_mask_mx
 * (mlx_ops.py:155-178).
 *   q [B,Hq,Lq,D] (q_dtype); k, v: element (b,h,t,d) at
 *   base + b*kv_batch_stride + h*kv_head_stride + t*D + d (elements), so both
 *   plain [B,Hkv,Lk,D] tensors and KV-cache buffers [B,Hkv,Lmax,D] work;
 *   qpos int32 [B,Lq] or NULL (bottom-right default arange(Lk-Lq, Lk));
 *   out [B,Hq,Lq,D] in q_dtype.
 * Errors mirror the reference's ValueErrors (block sizes > 0, Hq % Hkv == 0,
 * causal requires Lk >= Lq).  q_blk/k_blk are accepted for interface parity;
 * results are independent of them up to fp32 rounding. */
int strata_attn_gqa(strata_ctx* ctx, const void* q, int q_dtype, const void* k, int k_dtype,
                    const void* v, int v_dtype, int64_t kv_batch_stride,
                    int64_t kv_head_stride, const int32_t* qpos, int B, int Hq, int Hkv,
                    int Lq, int Lk, int D, int causal, int q_blk, int k_blk, float eps,
                    void* out, void* stream);

/* No counterpart in the reference.  strata_attn_gqa for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): same arguments, results and errors, but
 * the split-K partials live in a static 16 MiB device array instead of the
 * ctx arena, and nothing is allocated.  Decode shapes needing more partials
 * (B * Hq * splits * (D + 4) * 4 bytes) fail with STRATA_EINVAL.  Every call
 * on one GPU shares that array: calls that overlap on one GPU (concurrent
 * streams or threads) race. */
int strata_attn_gqa_noalloc(strata_ctx* ctx, const void* q, int q_dtype, const void* k,
                            int k_dtype, const void* v, int v_dtype, int64_t kv_batch_stride,
                            int64_t kv_head_stride, const int32_t* qpos, int B, int Hq, int Hkv,
                            int Lq, int Lk, int D, int causal, int q_blk, int k_blk, float eps,
                            void* out, void* stream);

/* ---------------------------------------------------------------- KV cache
 * Replaces MLXKVCache's append/read contract (src/ollm/mlx_kvcache.py:65-172):
 * per-layer K/V [B,Hkv,Lmax,D] buffers, per-layer lengths, and rejection of
 * appends whose start position is not the current length ("append exactly").
 * If k_storage / v_storage are non-NULL they must hold layers*B*Hkv*Lmax*D
 * elements each and stay owned by the caller; otherwise the cache allocates. */
int strata_kv_create(strata_ctx* ctx, int layers, int B, int Hkv, int Lmax, int D,
                     int dtype, void* k_storage, void* v_storage, strata_kv** out);
int strata_kv_destroy(strata_kv* kv);

/* Append k_new/v_new [B,Hkv,Lnew,D] (dtype of `src_dtype`, converted to the
 * cache dtype) to `layer` at position pos0; pos0 must equal the layer length. */
int strata_kv_append(strata_kv* kv, int layer, const void* k_new, const void* v_new,
                     int src_dtype, int Lnew, int pos0, void* stream);

/* Replace layer's contents with a snapshot k_src/v_src [B,Hkv,L,D]
 * (src_dtype, converted to the cache dtype) and set its length to L: the
 * device side of reloading an offloaded layer (MLXKVCache._load_layer_from_disk,
 * src/ollm/mlx_kvcache.py:222-250). */
int strata_kv_restore(strata_kv* kv, int layer, const void* k_src, const void* v_src,
                      int src_dtype, int L, void* stream);

/* Fused decode/prefill step: take the token-major projection outputs
 * q_src [B, L, Hq*D], k_src / v_src [B, L, Hkv*D] (src_dtype, equal to the
 * cache dtype), apply RoPE at positions pos0..pos0+L-1 to q and k, write
 * q_out [B,Hq,L,D] and append rotated k and v to `layer`.
 * Replaces llama_mlx.py:271-297 (reshape/transpose, RoPE, cache.update). */
int strata_rope_kv_append(strata_kv* kv, int layer, const void* q_src, const void* k_src,
                          const void* v_src, int src_dtype, int Hq, int L, int pos0,
                          float theta, void* q_out, void* stream);

/* Read side: device base pointers of layer's K and V buffers, the element
 * strides to pass to strata_attn_gqa, and the current length. */
int strata_kv_view(strata_kv* kv, int layer, void** k, void** v, int64_t* batch_stride,
                   int64_t* head_stride, int* length);
int strata_kv_len(strata_kv* kv, int layer, int* length);
/* Reset all lengths to 0 (MLXKVCache.clear, mlx_kvcache.py:271-284). */
int strata_kv_clear(strata_kv* kv);

/* ----------------------------------------------------------- decoder glue
 * RMSNorm (src/ollm/llama_mlx.py:77-92): y = bf16(w * (x * rsqrt(mean(x^2)+eps)))
 * over rows of length H; x,y bf16 [rows,H], w bf16 [H].  If `residual` is
 * non-NULL, x is first replaced by bf16(x + residual) and that sum is written
 * back to `x` (the residual stream, llama_mlx.py:647,653). */
int strata_rmsnorm(strata_ctx* ctx, void* x, const void* residual, const uint16_t* w,
                   int64_t rows, int64_t H, float eps, void* y, void* stream);

/* a = bf16(silu(g) * u) for gate/up outputs (llama_mlx.py:399-407). */
int strata_silu_mul(strata_ctx* ctx, const void* g, const void* u, int64_t n, void* a,
                    void* stream);

/* y = bf16(x + r) elementwise (residual add, llama_mlx.py:647,653). */
int strata_add(strata_ctx* ctx, const void* x, const void* r, int64_t n, void* y,
               void* stream);

/* Embedding gather rows of a bf16 table [V,H] by int32 ids [n] (llama_mlx.py:724-738). */
int strata_embed(strata_ctx* ctx, const uint16_t* table, int64_t V, int64_t H,
                 const int32_t* ids, int64_t n, void* y, void* stream);

/* Greedy argmax over rows of fp32 logits [rows, V] / temperature; ties pick
 * the lowest index (generation.py:42-43). out int32 [rows]. */
int strata_argmax(strata_ctx* ctx, const float* logits, int64_t rows, int64_t V,
                  int32_t* out, void* stream);

/* Dequantize a q4 triple [N, K] to bf16: out = bf16(s*q + b), computed in
 * fp32 with one round-to-nearest-even.  mx.dequantize of an MLX 4-bit
 * checkpoint's quantized embedding (src/ollm/llama_mlx.py:722-738); a loader
 * expands the table once and gathers bf16 rows (same values as gathering
 * then dequantizing).  bits must be 4, group_size 64; w and out 16-byte
 * aligned. */
int strata_dequantize_q4(strata_ctx* ctx, const uint32_t* w, const uint16_t* scales,
                         const uint16_t* biases, int64_t N, int64_t K, int group_size, int bits,
                         uint16_t* out, void* stream);

/* Quantize fp32/bf16 weights [N,K] to the q4 affine triple with group 64:
 * per group scale = bf16((max-min)/15), bias = bf16(min),
 * q = clip(rint((w - bias)/scale), 0, 15).  The reference consumes
 * pre-quantized checkpoints (mx.quantize appears only in
 * tests/test_mlx_generation.py:180); this is the loader-side quantizer. */
int strata_quantize_q4(strata_ctx* ctx, const void* wsrc, int w_dtype, int64_t N, int64_t K,
                       int group_size, uint32_t* w, uint16_t* scales, uint16_t* biases,
                       void* stream);


/* ------------------------------------------------------------ decoder engine
 * Native Llama forward + greedy generation over the kernels above.  Replaces
 * MLXLlamaForCausalLM.__call__ (src/ollm/llama_mlx.py:863-912) with its
 * decoder layers (608-658, 220-342, 345-432) and greedy_generate_mx
 * (src/ollm/generation.py:7-50): prefill once, then one-token decodes with
 * the position and token kept on the device, launched from the host or
 * replayed as a captured HIP graph.  Weights and the KV cache stay
 * caller-owned. */
typedef struct strata_llama_config {
  int vocab_size, hidden_size, intermediate_size, num_layers, num_heads, num_kv_heads, head_dim;
  int group_size;
  float rms_norm_eps, rope_theta;
} strata_llama_config;

typedef struct strata_llama_layer {
  const uint16_t* input_norm;      /* bf16 [hidden] */
  const uint16_t* post_norm;       /* bf16 [hidden] */
  strata_q4_weight q, k, v, o, gate, up, down;  /* q4 triples; .y is ignored */
} strata_llama_layer;

typedef struct strata_decoder strata_decoder;

/* embed / lm_head bf16 [vocab, hidden]; final_norm bf16 [hidden].  The KV
 * cache must be bf16 with geometry (num_layers, B <= its batch, num_kv_heads,
 * Lmax, head_dim).  max_tokens bounds B * L of one forward call.  lm_head may
 * be NULL when a q4 head is set with strata_decoder_set_lm_head_q4 before the
 * first forward. */
int strata_decoder_create(strata_ctx* ctx, const strata_llama_config* cfg,
                          const uint16_t* embed, const uint16_t* final_norm,
                          const uint16_t* lm_head, const strata_llama_layer* layers,
                          strata_kv* kv, int max_batch, int max_tokens, strata_decoder** out);
int strata_decoder_destroy(strata_decoder* dec);

/* Use a q4 triple [vocab, hidden] (group_size of the config) as the final
 * projection, with fp32 logits: an MLX 4-bit checkpoint's quantized lm_head,
 * or its quantized embedding when the head is tied to it
 * (src/ollm/llama_mlx.py:886-910 projects through _linear on the triple).
 * Replaces any bf16 head; .y is ignored.  Discards captured decode graphs. */
int strata_decoder_set_lm_head_q4(strata_decoder* dec, const strata_q4_weight* head);

/* One forward over ids int32 [B, L] (device) appended to the KV cache at its
 * current length; writes fp32 logits of the last position, [B, vocab]. */
int strata_decoder_forward(strata_decoder* dec, const int32_t* ids, int B, int L, float* logits,
                           void* stream);

/* Greedy generation: prefill `prompt` [B, L] (device), then max_new - 1
 * decode steps; out_tokens int32 [B, max_new] (device) gets
 * argmax(logits / temperature) of every step (ties -> lowest id).
 * use_graph = 0 launches the decode steps from the host (7-11% faster on
 * ROCm 7 / MI355X); use_graph = 1 replays one captured HIP graph per step.
 * Synchronous: returns when all tokens are written. */
int strata_decoder_generate(strata_decoder* dec, const int32_t* prompt, int B, int L, int max_new,
                            float temperature, int use_graph, int32_t* out_tokens, void* stream);

/* ------------------------------------------------------ measurement helper
 * No counterpart in the reference: the plain-read floor the decode GEMV is
 * measured against.  Streams `bytes` (a multiple of 16) from the device
 * buffer p with 16-byte loads, `unroll` (4, 8 or 16) loads in flight per
 * lane, num_cus * wg_per_cu (1..16) workgroups of 256 threads striding over
 * the buffer; the loaded words are folded and written to sink (16 bytes,
 * device) only if they fold to a constant, so in practice nothing is
 * written.  No other work: its duration is what reading the bytes costs. */
int strata_bench_read(strata_ctx* ctx, const void* p, int64_t bytes, int wg_per_cu, int unroll,
                      void* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* STRATA_HIP_H */
