// Native Llama decoder engine: forward passes and greedy generation launched
// from C++ over the library's kernels.  Decode steps are launched from the
// host per token, or captured once per context bucket as a HIP graph and
// replayed (use_graph).
//
// Follows MLXLlamaForCausalLM.__call__ (src/ollm/llama_mlx.py:863-912),
// MLXLlamaModel.__call__ (740-833), MLXLlamaDecoderLayer.__call__ (608-658),
// MLXLlamaAttention.__call__ (220-342), MLXLlamaMLP (345-432) and
// greedy_generate_mx (src/ollm/generation.py:7-50).  Per layer of a
// prefill (the decode step fuses further, see forward_layers):
//   h <- h + delta;  xn = RMSNorm(h)               (fused residual + norm)
//   q, k, v = q4(xn)                               (one launch)
//   RoPE(q, k) at the cache position; append k, v   (one launch)
//   a = GQA attention(q, K[:len], V[:len])          (split-K decode / MFMA prefill)
//   h <- h + q4_o(a);  xn = RMSNorm(h)
//   delta = q4_down(silu(q4_gate(xn)) * q4_up(xn))  (gate/up in one launch)
// then logits = lm_head(RMSNorm(h + delta)) for the last position, argmax.
// Device counters {step, position, key count} let one captured step serve
// every token: RoPE/append read the position, attention reads the key count,
// and a final one-thread kernel records the token and advances the counters.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <map>
#include <vector>

#include "strata_internal.h"

struct strata_decoder {
  strata_ctx* ctx;
  strata_llama_config cfg;
  const uint16_t* embed;
  const uint16_t* final_norm;
  const uint16_t* lm_head;   // bf16 [vocab, hidden], or null with head_q4 set
  strata_q4_weight head_q4;  // q4 lm_head (head_q4.w != null selects it)
  std::vector<strata_llama_layer> layers;
  strata_kv* kv;
  int max_batch, max_tokens;
  // activations (bf16 unless noted)
  void *h, *xn, *q, *k, *v, *qr, *attn, *o, *gate, *up, *act, *delta, *hn;
  float* logits;          // fp32 [max_batch, vocab]
  int32_t* ids;           // [max_batch] current input ids of a decode step
  int32_t* tokens;        // [max_batch][Lmax] generated ids, copied out per call
  int* counters;          // {step, position, key count}
  float* part;            // split-K partials for graph-mode decode attention
  int part_splits;
  float2* rope_table;     // (cos, sin) [Lmax][head_dim/2], built once at creation
  float2* rope_cur;       // (cos, sin) [head_dim/2] of the position counters[1]
  void* amax;             // argmax partials [max_batch * kArgmaxBlocks * 8 B]
  hipStream_t stream;     // the decoder's own stream (graph capture / replay)
  // Captured decode steps, one per key-capacity bucket: a step at key count
  // n replays the graph captured for capacity roundup(n, kKeyBucket), so the
  // split-K attention launch is sized to the context actually in use.
  // The captured steps write into `tokens` (stride Lmax), so they stay valid
  // for every call with the same batch and temperature.
  std::map<int, hipGraphExec_t> graphs;
  int graph_batch;
  float graph_temp;
  // Prefill GEMM layout of each layer's launches (q/k/v, o, gate/up, down),
  // re-laid out once at creation (null: re-laid out per call).
  std::vector<GemmPacked> packed;
  // Decode GEMV layout of the same launches (4 per layer, q4_gemv_mfma.hip),
  // built once at creation; empty when the model's shapes do not fit it
  // (the decode step then runs the MLX-layout GEMV).
  std::vector<GemvLayout> dlay;
  GemvLayout head_lay;  // q4 lm_head in the GEMV layout (head_q4 set)
};

namespace {

// logits fp32 [M, vocab] = x bf16 [M, hidden] . lm_head^T: the bf16 head on
// the dense GEMV, a q4 head (MLX 4-bit checkpoints, possibly tied to the
// quantized embedding) on the q4 GEMV (llama_mlx.py:886-910).
int lm_head_launch(strata_decoder* d, const void* x, int M, float* logits, void* stream) {
  const strata_llama_config& c = d->cfg;
  if (d->head_q4.w) {
    if (d->head_lay.buf && M <= kGvMaxRows) {
      void* ys[1] = {logits};
      return strata_gemv_layout_run(d->head_lay, x, M, ys, STRATA_F32, nullptr, stream);
    }
    strata_q4_weight w = d->head_q4;
    w.y = logits;
    return strata_q4_gemv(d->ctx, x, STRATA_BF16, M, c.hidden_size, &w, 1, STRATA_F32, stream);
  }
  return strata_bf16_gemv(d->ctx, x, M, c.hidden_size, d->lm_head, c.vocab_size, logits,
                          STRATA_F32, stream);
}

int alloc(void** p, size_t bytes) {
  if (hipMalloc(p, bytes) != hipSuccess) {
    *p = nullptr;
    return strata_set_error(STRATA_ENOMEM, "decoder: allocation of %zu bytes failed", bytes);
  }
  return STRATA_OK;
}

#define RC(expr)                \
  do {                          \
    const int _rc = (expr);     \
    if (_rc) return _rc;        \
  } while (0)

constexpr int kKeyBucket = 256;

// One decoder forward over T = B*L tokens at positions pos0..pos0+L-1
// (pos0 < 0: read from counters[1], decode graph mode, L == 1, with at most
// `key_cap` keys per layer).
int forward_layers(strata_decoder* d, int B, int L, int pos0, void* stream, int key_cap = 0) {
  const strata_llama_config& c = d->cfg;
  const int T = B * L;
  const int H = c.hidden_size, F = c.intermediate_size, D = c.head_dim;
  const int Hq = c.num_heads, Hkv = c.num_kv_heads;
  strata_kv* kv = d->kv;
  const int64_t kv_bs = (int64_t)Hkv * kv->Lmax * D, kv_hs = (int64_t)kv->Lmax * D;
  const bool graph_mode = pos0 < 0;
  // One-token steps (T <= 8 rows) fuse RoPE/append and SiLU into GEMV epilogues.
  const bool decode = L == 1 && T <= 8;
  if (decode) {
    const bool use_lay = !d->dlay.empty();
    // Five launches per layer; the residual stream h is updated in place by
    // the o/down epilogues, and RMSNorm runs in the q/k/v and gate/up
    // prologues:
    //   q, k, v = q4(RMSNorm(h)); RoPE(q, k); append k, v     (one launch)
    //   a = GQA attention(q, K[:len], V[:len])                 (split-K)
    //   h = h + q4_o(a)                                        (one launch)
    //   act = silu(q4_gate(RMSNorm(h))) * q4_up(RMSNorm(h))    (one launch)
    //   h = h + q4_down(act)                                   (one launch)
    for (int li = 0; li < c.num_layers; ++li) {
      const strata_llama_layer& Lw = d->layers[li];
      void* kc = kv->kl(li);
      void* vc = kv->vl(li);
      const GemvLayout* lay = use_lay ? &d->dlay[(size_t)li * 4] : nullptr;
      strata_q4_weight qkv[3] = {Lw.q, Lw.k, Lw.v};
      GemvEpilogue eq{2, D, Hq, Hkv, kv->Lmax, graph_mode ? 0 : pos0,
                      graph_mode ? d->counters + 1 : nullptr, c.rope_theta,
                      (uint16_t*)d->qr, (uint16_t*)kc, (uint16_t*)vc, Lw.input_norm,
                      c.rms_norm_eps, d->rope_table, graph_mode ? d->rope_cur : nullptr};
      void* no_y[3] = {nullptr, nullptr, nullptr};
      if (lay) RC(strata_gemv_layout_run(lay[0], d->h, T, no_y, STRATA_BF16, &eq, stream));
      else RC(strata_q4_gemv_epi(d->ctx, d->h, T, H, qkv, 3, eq, stream));
      AttnExtra ex;
      ex.part = d->part;
      ex.part_splits = d->part_splits;
      if (graph_mode) ex.dlen = d->counters + 2;
      RC(strata_attention_dispatch(d->ctx, d->qr, STRATA_BF16, kc, STRATA_BF16, vc, STRATA_BF16,
                                   kv_bs, kv_hs, nullptr, B, Hq, Hkv, 1,
                                   graph_mode ? key_cap : pos0 + 1, D, 1, 1e-12f, d->attn, ex,
                                   stream));
      GemvEpilogue er{};
      er.mode = 3;
      strata_q4_weight o = Lw.o;
      o.y = d->h;
      void* yh[1] = {d->h};
      if (lay) RC(strata_gemv_layout_run(lay[1], d->attn, T, yh, STRATA_BF16, &er, stream));
      else RC(strata_q4_gemv_epi(d->ctx, d->attn, T, Hq * D, &o, 1, er, stream));
      strata_q4_weight gu[2] = {Lw.gate, Lw.up};
      gu[0].y = d->act;
      GemvEpilogue es{};
      es.mode = 1;
      es.norm_w = Lw.post_norm;
      es.eps = c.rms_norm_eps;
      void* ya[1] = {d->act};
      if (lay) RC(strata_gemv_layout_run(lay[2], d->h, T, ya, STRATA_BF16, &es, stream));
      else RC(strata_q4_gemv_epi(d->ctx, d->h, T, H, gu, 2, es, stream));
      strata_q4_weight dn = Lw.down;
      dn.y = d->h;
      if (lay) RC(strata_gemv_layout_run(lay[3], d->act, T, yh, STRATA_BF16, &er, stream));
      else RC(strata_q4_gemv_epi(d->ctx, d->act, T, F, &dn, 1, er, stream));
    }
    RC(strata_rmsnorm_launch(d->h, nullptr, d->final_norm, T, H, c.rms_norm_eps, d->hn, stream));
    return lm_head_launch(d, d->hn, B, d->logits, stream);
  }
  for (int li = 0; li < c.num_layers; ++li) {
    const strata_llama_layer& Lw = d->layers[li];
    RC(strata_rmsnorm_launch(d->h, li == 0 ? nullptr : d->delta, Lw.input_norm, T, H,
                             c.rms_norm_eps, d->xn, stream));
    strata_q4_weight qkv[3] = {Lw.q, Lw.k, Lw.v};
    qkv[0].y = d->q;
    qkv[1].y = d->k;
    qkv[2].y = d->v;
    void* kc = kv->kl(li);
    void* vc = kv->vl(li);
    const GemmPacked* pk = d->packed.empty() ? nullptr : &d->packed[(size_t)li * 4];
    RC(strata_q4_gemm_multi(d->ctx, d->xn, T, H, qkv, 3, STRATA_BF16, stream, pk ? &pk[0] : nullptr));
    RC(strata_rope_kv_fused_launch(d->q, d->k, d->v, STRATA_BF16, B, Hq, Hkv, L, D, kv->Lmax,
                                   pos0, nullptr, c.rope_theta, d->qr, kc, vc, STRATA_BF16,
                                   stream, d->rope_table));
    AttnExtra ex;
    ex.out_tm = 1;  // prefill writes [B, L, Hq, D], the o_proj input layout
    RC(strata_attention_dispatch(d->ctx, d->qr, STRATA_BF16, kc, STRATA_BF16, vc, STRATA_BF16,
                                 kv_bs, kv_hs, nullptr, B, Hq, Hkv, L, pos0 + L, D, 1, 1e-12f,
                                 d->attn, ex, stream));
    strata_q4_weight o = Lw.o;
    o.y = d->o;
    RC(strata_q4_gemm_multi(d->ctx, d->attn, T, Hq * D, &o, 1, STRATA_BF16, stream,
                            pk ? &pk[1] : nullptr));
    RC(strata_rmsnorm_launch(d->h, d->o, Lw.post_norm, T, H, c.rms_norm_eps, d->xn, stream));
    strata_q4_weight gu[2] = {Lw.gate, Lw.up};
    gu[0].y = d->gate;
    gu[1].y = d->up;
    RC(strata_q4_gemm_multi(d->ctx, d->xn, T, H, gu, 2, STRATA_BF16, stream, pk ? &pk[2] : nullptr));
    RC(strata_silu_mul_launch(d->gate, d->up, (int64_t)T * F, d->act, stream));
    strata_q4_weight dn = Lw.down;
    dn.y = d->delta;
    RC(strata_q4_gemm_multi(d->ctx, d->act, T, F, &dn, 1, STRATA_BF16, stream,
                            pk ? &pk[3] : nullptr));
  }
  // final norm of h + delta, then lm_head on the last position of each row
  RC(strata_rmsnorm_launch(d->h, d->delta, d->final_norm, T, H, c.rms_norm_eps, d->hn, stream));
  if (L == 1) {
    RC(lm_head_launch(d, d->hn, B, d->logits, stream));
  } else {
    for (int b = 0; b < B; ++b)
      RC(lm_head_launch(d, static_cast<char*>(d->hn) + ((int64_t)b * L + L - 1) * H * 2, 1,
                        d->logits + (int64_t)b * c.vocab_size, stream));
  }
  return STRATA_OK;
}

int check_forward(strata_decoder* d, int B, int L) {
  STRATA_REQUIRE(d != nullptr, "decoder is NULL");
  STRATA_REQUIRE(d->lm_head != nullptr || d->head_q4.w != nullptr,
                 "decoder has no lm_head (a bf16 head at creation or a q4 head via "
                 "strata_decoder_set_lm_head_q4)");
  STRATA_REQUIRE(B >= 1 && B <= d->max_batch && B <= d->kv->B,
                 "batch %d exceeds the decoder/KV-cache batch", B);
  STRATA_REQUIRE(L >= 1 && (int64_t)B * L <= d->max_tokens,
                 "B*L = %lld exceeds max_tokens %d", (long long)B * L, d->max_tokens);
  STRATA_REQUIRE(d->kv->B == B, "KV cache batch %d differs from input batch %d", d->kv->B, B);
  const int pos0 = d->kv->len[0];
  for (int li = 0; li < d->cfg.num_layers; ++li)
    STRATA_REQUIRE(d->kv->len[li] == pos0,
                   "cache_position must append exactly after the cached sequence; layer %d has "
                   "length %d, layer 0 has %d",
                   li, d->kv->len[li], pos0);
  STRATA_REQUIRE(pos0 + L <= d->kv->Lmax, "KV cache capacity exceeded: %d + %d > Lmax %d", pos0,
                 L, d->kv->Lmax);
  return STRATA_OK;
}

void set_lengths(strata_decoder* d, int len) {
  for (int& l : d->kv->len) l = len;
}

// Load-time re-layout of the prefill weights (the MLX layout stays the
// interchange and decode format): for each layer the four GEMM launches of a
// prefill, in the layout of q4_gemm_relayout_kernel, when prefills can reach
// the 256-column MFMA kernel and every linear qualifies.  Costs one more copy of the
// q4 linears; on an allocation failure the prefill re-lays out per call.
// STRATA_DECODER_NO_PREFILL_PACK (read per decoder creation) skips it:
// prefills then re-lay out per call and the copy's memory is not held.
int pack_prefill_weights(strata_decoder* d) {
  const strata_llama_config& c = d->cfg;
  if (getenv("STRATA_DECODER_NO_PREFILL_PACK") != nullptr || d->max_tokens < kMfmaMidRows)
    return STRATA_OK;
  const int H = c.hidden_size, F = c.intermediate_size, QW = c.num_heads * c.head_dim;
  std::vector<GemmPacked> packed;
  auto drop = [&]() {
    for (GemmPacked& q : packed) (void)hipFree(const_cast<void*>(q.buf));
  };
  for (const strata_llama_layer& L : d->layers) {
    const strata_q4_weight groups[4][3] = {{L.q, L.k, L.v}, {L.o}, {L.gate, L.up}, {L.down}};
    const int counts[4] = {3, 1, 2, 1}, Ks[4] = {H, QW, H, F};
    for (int gi = 0; gi < 4; ++gi) {
      int64_t N = 0;
      for (int i = 0; i < counts[gi]; ++i) {
        const strata_q4_weight& w = groups[gi][i];
        if (w.N % 256 != 0 || !aligned16(w.w)) {
          drop();
          return STRATA_OK;  // this model's prefill re-lays out per call
        }
        N += w.N;
      }
      void* p = nullptr;
      if (hipMalloc(&p, strata_q4_gemm_mfma_scratch(N, Ks[gi])) != hipSuccess) {
        (void)hipGetLastError();
        drop();
        return STRATA_OK;
      }
      GemmPacked g;
      g.buf = p;
      g.N = N;
      g.K = Ks[gi];
      g.count = counts[gi];
      packed.push_back(g);
      const int rc = strata_q4_gemm_pack(groups[gi], counts[gi], Ks[gi], p, nullptr);
      if (rc) {
        drop();
        return rc;
      }
    }
  }
  d->packed.swap(packed);
  return STRATA_OK;
}

// Load-time GEMV layout of every layer's decode launches: q/k/v (rows in
// rotate-half pairs for the RoPE epilogue), o, gate/up (SiLU pairs), down.
// Skipped (decode then reads the MLX layout) when a width is beyond the
// layout kernel (K > 16384) or the head size is not a multiple of 16.
// STRATA_DECODER_NO_GEMV_LAYOUT (read per decoder creation) keeps the MLX
// layout for decode.
int build_decode_layouts(strata_decoder* d) {
  const strata_llama_config& c = d->cfg;
  if (getenv("STRATA_DECODER_NO_GEMV_LAYOUT") != nullptr) return STRATA_OK;
  const int H = c.hidden_size, F = c.intermediate_size, QW = c.num_heads * c.head_dim;
  if (!strata_gemv_layout_fits(H, 1) || !strata_gemv_layout_fits(F, 1) ||
      !strata_gemv_layout_fits(QW, 1) || c.head_dim % 16 != 0)
    return STRATA_OK;
  std::vector<GemvLayout> lays;
  auto fail = [&](int rc) {
    for (GemvLayout& L : lays) strata_gemv_layout_free(&L);
    return rc;
  };
  for (const strata_llama_layer& L : d->layers) {
    const strata_q4_weight qkv[3] = {L.q, L.k, L.v}, gu[2] = {L.gate, L.up};
    GemvLayout g[4];
    int rc = strata_gemv_layout_build(qkv, 3, H, 2, c.head_dim, &g[0], nullptr);
    if (!rc) rc = strata_gemv_layout_build(&L.o, 1, QW, 0, 0, &g[1], nullptr);
    if (!rc) rc = strata_gemv_layout_build(gu, 2, H, 1, 0, &g[2], nullptr);
    if (!rc) rc = strata_gemv_layout_build(&L.down, 1, F, 0, 0, &g[3], nullptr);
    for (GemvLayout& x : g)
      if (x.buf) lays.push_back(x);
    if (rc) return fail(rc);
  }
  if (hipDeviceSynchronize() != hipSuccess)
    return fail(strata_set_error(STRATA_EHIP, "decoder: GEMV re-layout failed"));
  d->dlay.swap(lays);
  return STRATA_OK;
}

}  // namespace

extern "C" {

int strata_decoder_create(strata_ctx* ctx, const strata_llama_config* cfg,
                          const uint16_t* embed, const uint16_t* final_norm,
                          const uint16_t* lm_head, const strata_llama_layer* layers,
                          strata_kv* kv, int max_batch, int max_tokens, strata_decoder** out) {
  STRATA_REQUIRE(ctx && cfg && embed && final_norm && layers && kv && out,
                 "decoder_create: null argument");
  const strata_llama_config& c = *cfg;
  STRATA_REQUIRE(c.num_layers > 0 && c.hidden_size > 0 && c.num_heads > 0 && c.num_kv_heads > 0 &&
                     c.head_dim > 0 && c.vocab_size > 0 && c.intermediate_size > 0,
                 "decoder_create: invalid config");
  STRATA_REQUIRE(c.num_heads % c.num_kv_heads == 0,
                 "query heads must be divisible by key/value heads");
  STRATA_REQUIRE(c.group_size == 64, "only group_size 64 is supported");
  STRATA_REQUIRE(c.hidden_size % 64 == 0 && c.intermediate_size % 64 == 0 &&
                     (c.num_heads * c.head_dim) % 64 == 0,
                 "hidden, intermediate and head widths must be multiples of 64");
  STRATA_REQUIRE(c.head_dim == 64 || c.head_dim == 128, "head_dim must be 64 or 128");
  STRATA_REQUIRE(kv->layers == c.num_layers && kv->Hkv == c.num_kv_heads && kv->D == c.head_dim &&
                     kv->dtype == STRATA_BF16,
                 "KV cache geometry/dtype does not match the model (bf16 cache required)");
  STRATA_REQUIRE(max_batch >= 1 && max_batch <= 8 && max_tokens >= max_batch,
                 "max_batch must be in 1..8 and max_tokens >= max_batch");
  auto* d = new strata_decoder{};
  d->ctx = ctx;
  d->cfg = c;
  d->embed = embed;
  d->final_norm = final_norm;
  d->lm_head = lm_head;
  d->layers.assign(layers, layers + c.num_layers);
  d->kv = kv;
  d->max_batch = max_batch;
  d->max_tokens = max_tokens;
  const size_t T = max_tokens;
  const size_t H = c.hidden_size, F = c.intermediate_size, QW = (size_t)c.num_heads * c.head_dim,
               KW = (size_t)c.num_kv_heads * c.head_dim;
  int rc = STRATA_OK;
  struct { void** p; size_t bytes; } bufs[] = {
      {&d->h, T * H * 2},      {&d->xn, T * H * 2},     {&d->q, T * QW * 2},
      {&d->k, T * KW * 2},     {&d->v, T * KW * 2},     {&d->qr, T * QW * 2},
      {&d->attn, T * QW * 2},  {&d->o, T * H * 2},      {&d->gate, T * F * 2},
      {&d->up, T * F * 2},     {&d->act, T * F * 2},    {&d->delta, T * H * 2},
      {&d->hn, T * H * 2},
      {reinterpret_cast<void**>(&d->logits), (size_t)max_batch * c.vocab_size * 4},
      {reinterpret_cast<void**>(&d->ids), (size_t)max_batch * 4},
      {reinterpret_cast<void**>(&d->tokens), (size_t)max_batch * kv->Lmax * 4},
      {reinterpret_cast<void**>(&d->counters), 16},
      {&d->amax, (size_t)max_batch * kArgmaxBlocks * 8},
      {reinterpret_cast<void**>(&d->rope_table), (size_t)kv->Lmax * (c.head_dim / 2) * 8},
      {reinterpret_cast<void**>(&d->rope_cur), (size_t)(c.head_dim / 2) * 8},
  };
  for (auto& b : bufs)
    if (!rc) rc = alloc(b.p, b.bytes);
  d->part_splits = strata_attn_decode_splits(ctx, kv->B, c.num_kv_heads, kv->Lmax);
  if (!rc)
    rc = alloc(reinterpret_cast<void**>(&d->part),
               (size_t)kv->B * c.num_heads * part_stride(d->part_splits, c.head_dim) * 4);
  if (!rc) rc = pack_prefill_weights(d);
  if (!rc) rc = build_decode_layouts(d);
  if (!rc) rc = strata_rope_table_launch(d->rope_table, kv->Lmax, c.head_dim, c.rope_theta, nullptr);
  if (!rc && hipDeviceSynchronize() != hipSuccess)
    rc = strata_set_error(STRATA_EHIP, "decoder: RoPE table initialisation failed");
  if (!rc && hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking) != hipSuccess)
    rc = strata_set_error(STRATA_EHIP, "decoder: stream creation failed");
  if (rc) {
    strata_decoder_destroy(d);
    return rc;
  }
  *out = d;
  return STRATA_OK;
}

int strata_decoder_destroy(strata_decoder* d) {
  if (!d) return STRATA_OK;
  (void)hipDeviceSynchronize();
  for (auto& kvp : d->graphs) (void)hipGraphExecDestroy(kvp.second);
  for (GemmPacked& p : d->packed) (void)hipFree(const_cast<void*>(p.buf));
  for (GemvLayout& L : d->dlay) strata_gemv_layout_free(&L);
  strata_gemv_layout_free(&d->head_lay);
  void* ptrs[] = {d->h, d->xn, d->q, d->k, d->v, d->qr, d->attn, d->o, d->gate, d->up, d->act,
                  d->delta, d->hn, d->logits, d->ids, d->tokens, d->counters, d->part, d->amax,
                  d->rope_table, d->rope_cur};
  for (void* p : ptrs)
    if (p) (void)hipFree(p);
  if (d->stream) (void)hipStreamDestroy(d->stream);
  delete d;
  return STRATA_OK;
}

int strata_decoder_set_lm_head_q4(strata_decoder* d, const strata_q4_weight* head) {
  STRATA_REQUIRE(d != nullptr && head != nullptr, "set_lm_head_q4: null argument");
  STRATA_REQUIRE(head->w && head->scales && head->biases, "set_lm_head_q4: null weight pointer");
  STRATA_REQUIRE(head->N == d->cfg.vocab_size, "set_lm_head_q4: head has %lld rows, vocab is %d",
                 (long long)head->N, d->cfg.vocab_size);
  STRATA_REQUIRE(aligned16(head->w), "set_lm_head_q4: packed weights must be 16-byte aligned");
  // captured decode steps hold the previous head
  STRATA_HIP_CHECK(hipStreamSynchronize(d->stream));
  for (auto& kvp : d->graphs) (void)hipGraphExecDestroy(kvp.second);
  d->graphs.clear();
  strata_gemv_layout_free(&d->head_lay);
  d->head_q4 = *head;
  d->head_q4.y = nullptr;
  // the decode head in the GEMV layout (the MLX layout serves the rest)
  if (!d->dlay.empty() && strata_gemv_layout_fits(d->cfg.hidden_size, 1)) {
    RC(strata_gemv_layout_build(&d->head_q4, 1, d->cfg.hidden_size, 0, 0, &d->head_lay, nullptr));
    STRATA_HIP_CHECK(hipDeviceSynchronize());
  }
  return STRATA_OK;
}

int strata_decoder_forward(strata_decoder* d, const int32_t* ids, int B, int L, float* logits,
                           void* stream) {
  RC(check_forward(d, B, L));
  STRATA_REQUIRE(ids != nullptr && logits != nullptr, "null ids/logits");
  const int pos0 = d->kv->len[0];
  const strata_llama_config& c = d->cfg;
  RC(strata_embed_launch(d->embed, c.vocab_size, c.hidden_size, ids, (int64_t)B * L, d->h, stream));
  RC(forward_layers(d, B, L, pos0, stream));
  set_lengths(d, pos0 + L);
  STRATA_HIP_CHECK(hipMemcpyAsync(logits, d->logits, (size_t)B * c.vocab_size * 4,
                                  hipMemcpyDeviceToDevice, as_stream(stream)));
  return STRATA_OK;
}

int strata_decoder_generate(strata_decoder* d, const int32_t* prompt, int B, int L, int max_new,
                            float temperature, int use_graph, int32_t* out_tokens, void* stream) {
  RC(check_forward(d, B, L));
  STRATA_REQUIRE(prompt != nullptr && out_tokens != nullptr, "null prompt/out_tokens");
  STRATA_REQUIRE(max_new >= 1, "max_new_tokens must be positive");
  STRATA_REQUIRE(temperature > 0.f, "temperature must be positive");
  const int pos0 = d->kv->len[0];
  STRATA_REQUIRE(pos0 + L + max_new - 1 <= d->kv->Lmax,
                 "KV cache capacity exceeded: %d + %d + %d - 1 > Lmax %d", pos0, L, max_new,
                 d->kv->Lmax);
  const strata_llama_config& c = d->cfg;
  hipStream_t s = d->stream;
  // order the decoder stream after the caller's work
  hipEvent_t ev;
  STRATA_HIP_CHECK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  if (hipEventRecord(ev, as_stream(stream)) != hipSuccess || hipStreamWaitEvent(s, ev, 0) != hipSuccess) {
    (void)hipEventDestroy(ev);
    return strata_set_error(STRATA_EHIP, "generate: ordering after the caller's stream failed");
  }
  // Positions whose K/V the launched work appends; on any error the cache
  // length is set to what was launched, so host length and device contents
  // agree.
  int appended = pos0;
  auto run = [&]() -> int {
    // prefill
    RC(strata_embed_launch(d->embed, c.vocab_size, c.hidden_size, prompt, (int64_t)B * L, d->h, s));
    RC(forward_layers(d, B, L, pos0, s));
    appended = pos0 + L;
    // counters {step, position, key count}: the tail below records token 0
    // and leaves {1, pos0+L, pos0+L+1}, i.e. the next step processes the token
    // at position pos0+L against pos0+L+1 keys.
    const int init[4] = {0, pos0 + L - 1, pos0 + L, 0};
    STRATA_HIP_CHECK(hipMemcpyAsync(d->counters, init, sizeof(init), hipMemcpyHostToDevice, s));
    // Each step ends with the greedy token, its embedding in h (the next
    // step's input) and the advanced counters.
    auto tail = [&](hipStream_t st) -> int {
      return strata_decode_tail_launch(d->logits, B, c.vocab_size, temperature, d->amax, d->ids,
                                       d->tokens, d->kv->Lmax, d->counters, d->rope_table,
                                       d->kv->Lmax, c.head_dim / 2, d->rope_cur, d->embed,
                                       c.hidden_size, d->h, st);
    };
    RC(tail(s));

    auto decode_step = [&](hipStream_t st, int key_cap) -> int {
      RC(forward_layers(d, B, 1, -1, st, key_cap));
      return tail(st);
    };
    const bool reuse = d->graph_batch == B && d->graph_temp == temperature;
    if (max_new > 1 && !reuse) {
      for (auto& kvp : d->graphs) STRATA_HIP_CHECK(hipGraphExecDestroy(kvp.second));
      d->graphs.clear();
      d->graph_batch = B;
      d->graph_temp = temperature;
    }
    for (int i = 1; i < max_new; ++i) {
      // step i feeds the token at position pos0 + L + i - 1: that many keys + 1
      const int keys = pos0 + L + i;
      const int cap = std::min(d->kv->Lmax, (keys + kKeyBucket - 1) / kKeyBucket * kKeyBucket);
      if (!use_graph) {
        RC(decode_step(s, cap));
        appended = keys;
        continue;
      }
      auto it = d->graphs.find(cap);
      if (it == d->graphs.end()) {
        hipGraph_t g = nullptr;
        hipGraphExec_t ge = nullptr;
        STRATA_HIP_CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
        const int crc = decode_step(s, cap);
        const hipError_t ce = hipStreamEndCapture(s, &g);
        if (crc || ce != hipSuccess) {
          if (ce == hipSuccess && g) (void)hipGraphDestroy(g);
          if (crc) return crc;
          return strata_set_error(STRATA_EHIP, "decode graph capture failed: %s",
                                  hipGetErrorString(ce));
        }
        const hipError_t ie = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (ie != hipSuccess)
          return strata_set_error(STRATA_EHIP, "decode graph instantiation failed: %s",
                                  hipGetErrorString(ie));
        it = d->graphs.emplace(cap, ge).first;
      }
      STRATA_HIP_CHECK(hipGraphLaunch(it->second, s));
      appended = keys;
    }
    STRATA_HIP_CHECK(hipMemcpy2DAsync(out_tokens, (size_t)max_new * 4, d->tokens,
                                      (size_t)d->kv->Lmax * 4, (size_t)max_new * 4, B,
                                      hipMemcpyDeviceToDevice, s));
    return STRATA_OK;
  };
  const int rc = run();
  // The caller's stream waits for everything launched, success or not.
  const hipError_t e1 = hipEventRecord(ev, s);
  const hipError_t e2 = e1 == hipSuccess ? hipStreamWaitEvent(as_stream(stream), ev, 0) : e1;
  const hipError_t e3 = hipStreamSynchronize(s);
  (void)hipEventDestroy(ev);
  set_lengths(d, appended);
  if (rc) return rc;
  if (e2 != hipSuccess || e3 != hipSuccess)
    return strata_set_error(STRATA_EHIP, "generate: stream synchronization failed: %s",
                            hipGetErrorString(e3 != hipSuccess ? e3 : e2));
  return STRATA_OK;
}

}  // extern "C"
