/*
 * strata_oracle_llama.c — plain-C Llama decoder + greedy loop
 * (TEST INFRASTRUCTURE ONLY; never part of the product).
 *
 * Restates the same dtype flow as the NumPy oracle (oracle/llama.py), which
 * follows the reference's model adapter:
 *   RMSNorm            src/ollm/llama_mlx.py:77-92 (x * rsqrt(var + eps), then weight * x)
 *   q/k/v/o _linear    llama_mlx.py:53-74, 257-268, 313-316 (y = x @ (s*q + b).T)
 *   RoPE               llama_mlx.py:95-182 (rotate-half, inv_freq = 1/theta^(2i/D))
 *   KV append          llama_mlx.py:289-297 (cache_position = past .. past+L-1)
 *   attention          llama_mlx.py:300-308 -> backends/mlx_ops.py:32-152 with
 *                      k_block = 1e6 for L <= 128: one key block per query row,
 *                      so the online merge reduces to max / exp / sum / PV / divide
 *   MLP                llama_mlx.py:345-432 (down(silu(gate) * up))
 *   decoder layer      llama_mlx.py:608-658 (pre-norm residual blocks)
 *   model + head       llama_mlx.py:740-833, 863-912 (embedding, final norm, lm_head)
 *   greedy loop        src/ollm/generation.py:7-50 (prefill once, then 1-token steps,
 *                      argmax = first maximal logit)
 *
 * Rounding contract (identical to oracle/llama.py): every tensor crossing an
 * op boundary is rounded to bf16 (RNE); linears and the head accumulate in
 * double over the exactly dequantized weights and round once to fp32;
 * RMSNorm's variance is a double mean; attention, RoPE and SiLU are fp32
 * (SiLU through double, like the NumPy oracle).  Build with
 * -ffp-contract=off so no product/sum pair is fused.
 *
 * Parallelised with OpenMP over output rows and heads.  Prompt rows are
 * processed together (one pass over each weight row per layer), which is
 * the reference's single prefill forward.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline float bf(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t to_bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline float rbf(float f) { return bf(to_bf(f)); }

/* Linear order inside one layer: q, k, v, o, gate, up, down. */
enum { LQ = 0, LK, LV, LO, LG, LU, LD, NLIN };

typedef struct {
  int vocab, hidden, ffn, layers, heads, kv_heads, group;
  float eps, theta;
  const uint16_t* embed;   /* [vocab, hidden] bf16 */
  const uint16_t* norm;    /* [hidden] bf16 */
  const uint16_t* lm_head; /* [vocab, hidden] bf16, or NULL: tied to embed */
  const uint16_t* const* ln1; /* [layers] -> [hidden] bf16 */
  const uint16_t* const* ln2;
  const uint32_t* const* w;   /* [layers * 7] -> u32 [N, K/8] */
  const uint16_t* const* s;   /* [layers * 7] -> bf16 [N, K/group] */
  const uint16_t* const* b;
} OracleLlama;

/* Accumulation-order probe: when set, the linears accumulate in fp32 (group
 * sums, then a running fp32 total) instead of double.  The greedy ids of a
 * test model that change under this switch depend on accumulation order, so
 * they cannot be compared bit-exactly against any fp32 implementation. */
static int g_f32_accum = 0;
void oracle_llama_set_f32_accum(int on) { g_f32_accum = on != 0; }

/* y[m, n] = fp32(sum_k x[m, k] * (s*q + b)[n, k]) in double; x holds bf16 values. */
static void linear(const float* x, int M, int K, const uint32_t* w, const uint16_t* s,
                   const uint16_t* b, int N, int G, float* y) {
  double* xd = (double*)malloc(sizeof(double) * (size_t)M * K);
  for (int64_t i = 0; i < (int64_t)M * K; ++i) xd[i] = x[i];
  const int ng = K / G;
#pragma omp parallel
  {
    double* wr = (double*)malloc(sizeof(double) * (size_t)K);
#pragma omp for schedule(static)
    for (int n = 0; n < N; ++n) {
      for (int g = 0; g < ng; ++g) {
        const double sc = bf(s[(int64_t)n * ng + g]), bi = bf(b[(int64_t)n * ng + g]);
        for (int k = g * G; k < (g + 1) * G; ++k) {
          const uint32_t q = (w[(int64_t)n * (K / 8) + k / 8] >> (4 * (k % 8))) & 15u;
          wr[k] = sc * (double)q + bi;
        }
      }
      for (int m = 0; m < M; ++m) {
        const double* xr = xd + (int64_t)m * K;
        if (g_f32_accum) { /* perturbed variant: fp32 group sums, fp32 total */
          float acc = 0.f;
          for (int g = 0; g < ng; ++g) {
            float p = 0.f;
            for (int k = g * G; k < (g + 1) * G; ++k) p += (float)xr[k] * (float)wr[k];
            acc += p;
          }
          y[(int64_t)m * N + n] = acc;
          continue;
        }
        double a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int k = 0; k < K; k += 8)
          for (int j = 0; j < 8; ++j) a[j] += xr[k + j] * wr[k + j];
        y[(int64_t)m * N + n] = (float)(((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7])));
      }
    }
    free(wr);
  }
  free(xd);
}

static void rms_norm(const float* x, const uint16_t* wt, int H, float eps, float* out) {
  double ss = 0.0;
  for (int i = 0; i < H; ++i) ss += (double)x[i] * (double)x[i];
  const float r = (float)(1.0 / sqrt(ss / H + (double)eps));
  for (int i = 0; i < H; ++i) {
    const float t = x[i] * r;
    out[i] = rbf(t * bf(wt[i]));
  }
}

/* Rotate-half RoPE of one [D] head vector at position pos, result rounded to bf16. */
static void rope(float* v, int D, int pos, float theta) {
  float tmp[512];
  const int h = D / 2;
  for (int i = 0; i < h; ++i) {
    const float inv = (float)(1.0 / pow((double)theta, (double)(2 * i) / (double)D));
    const float ang = (float)pos * inv;
    const float c = (float)cos((double)ang), s = (float)sin((double)ang);
    const float x1 = v[i], x2 = v[i + h];
    const float a1 = x1 * c, b1 = (-x2) * s;
    const float a2 = x2 * c, b2 = x1 * s;
    tmp[i] = a1 + b1;
    tmp[i + h] = a2 + b2;
  }
  for (int i = 0; i < D; ++i) v[i] = rbf(tmp[i]);
}

typedef struct {
  const OracleLlama* m;
  int cap, len;
  uint16_t* k; /* [layers, kv_heads, cap, D] bf16 */
  uint16_t* v;
} Cache;

/* One forward over L rows at positions len .. len+L-1; logits of the last row -> out [vocab]. */
static void forward(Cache* c, const int64_t* ids, int L, float* logits) {
  const OracleLlama* m = c->m;
  const int H = m->hidden, F = m->ffn, hq = m->heads, hkv = m->kv_heads, D = H / hq;
  const int grp = hq / hkv, G = m->group, past = c->len;
  float* h = (float*)malloc(sizeof(float) * (size_t)L * H);
  float* xn = (float*)malloc(sizeof(float) * (size_t)L * H);
  float* q = (float*)malloc(sizeof(float) * (size_t)L * hq * D);
  float* kk = (float*)malloc(sizeof(float) * (size_t)L * hkv * D);
  float* vv = (float*)malloc(sizeof(float) * (size_t)L * hkv * D);
  float* o = (float*)malloc(sizeof(float) * (size_t)L * hq * D);
  float* t = (float*)malloc(sizeof(float) * (size_t)L * (F > H ? F : H));
  float* gg = (float*)malloc(sizeof(float) * (size_t)L * F);
  float* uu = (float*)malloc(sizeof(float) * (size_t)L * F);
  for (int r = 0; r < L; ++r)
    for (int i = 0; i < H; ++i) h[(int64_t)r * H + i] = bf(m->embed[ids[r] * H + i]);
  const float scale = (float)(1.0 / sqrt((double)D));
  for (int li = 0; li < m->layers; ++li) {
    const int64_t wi = (int64_t)li * NLIN;
    for (int r = 0; r < L; ++r) rms_norm(h + (int64_t)r * H, m->ln1[li], H, m->eps, xn + (int64_t)r * H);
    linear(xn, L, H, m->w[wi + LQ], m->s[wi + LQ], m->b[wi + LQ], hq * D, G, q);
    linear(xn, L, H, m->w[wi + LK], m->s[wi + LK], m->b[wi + LK], hkv * D, G, kk);
    linear(xn, L, H, m->w[wi + LV], m->s[wi + LV], m->b[wi + LV], hkv * D, G, vv);
    for (int r = 0; r < L; ++r) {
      for (int hh = 0; hh < hq; ++hh) {
        float* qv = q + ((int64_t)r * hq + hh) * D;
        for (int i = 0; i < D; ++i) qv[i] = rbf(qv[i]);
        rope(qv, D, past + r, m->theta);
      }
      for (int hh = 0; hh < hkv; ++hh) {
        float* kv = kk + ((int64_t)r * hkv + hh) * D;
        const float* vr = vv + ((int64_t)r * hkv + hh) * D;
        for (int i = 0; i < D; ++i) kv[i] = rbf(kv[i]);
        rope(kv, D, past + r, m->theta);
        const int64_t base = (((int64_t)li * hkv + hh) * c->cap + past + r) * D;
        for (int i = 0; i < D; ++i) {
          c->k[base + i] = to_bf(kv[i]);
          c->v[base + i] = to_bf(vr[i]);
        }
      }
    }
    /* one key block per query row: scores, masked max, exp, sum, PV, divide */
#pragma omp parallel for collapse(2) schedule(static)
    for (int r = 0; r < L; ++r) {
      for (int hh = 0; hh < hq; ++hh) {
        const int kvh = hh / grp, n = past + r + 1;
        const float* qv = q + ((int64_t)r * hq + hh) * D;
        const uint16_t* kb = c->k + ((int64_t)li * hkv + kvh) * c->cap * D;
        const uint16_t* vb = c->v + ((int64_t)li * hkv + kvh) * c->cap * D;
        float* sc = (float*)malloc(sizeof(float) * (size_t)n);
        float mx = -INFINITY;
        for (int j = 0; j < n; ++j) {
          float d = 0.f;
          for (int i = 0; i < D; ++i) d += qv[i] * bf(kb[(int64_t)j * D + i]);
          sc[j] = d * scale;
          if (sc[j] > mx) mx = sc[j];
        }
        float sum = 0.f, acc[512];
        for (int i = 0; i < D; ++i) acc[i] = 0.f;
        for (int j = 0; j < n; ++j) {
          const float e = expf(sc[j] - mx);
          sum += e;
          for (int i = 0; i < D; ++i) acc[i] += e * bf(vb[(int64_t)j * D + i]);
        }
        const float den = sum > 1e-12f ? sum : 1e-12f;
        float* ov = o + ((int64_t)r * hq + hh) * D;
        for (int i = 0; i < D; ++i) ov[i] = rbf(acc[i] / den);
        free(sc);
      }
    }
    linear(o, L, hq * D, m->w[wi + LO], m->s[wi + LO], m->b[wi + LO], H, G, t);
    for (int64_t i = 0; i < (int64_t)L * H; ++i) h[i] = rbf(h[i] + rbf(t[i]));
    for (int r = 0; r < L; ++r) rms_norm(h + (int64_t)r * H, m->ln2[li], H, m->eps, xn + (int64_t)r * H);
    linear(xn, L, H, m->w[wi + LG], m->s[wi + LG], m->b[wi + LG], F, G, gg);
    linear(xn, L, H, m->w[wi + LU], m->s[wi + LU], m->b[wi + LU], F, G, uu);
    for (int64_t i = 0; i < (int64_t)L * F; ++i) {
      const double g = rbf(gg[i]);
      const float u = rbf(uu[i]);
      t[i] = rbf((float)(g / (1.0 + exp(-g)) * u));
    }
    linear(t, L, F, m->w[wi + LD], m->s[wi + LD], m->b[wi + LD], H, G, xn);
    for (int64_t i = 0; i < (int64_t)L * H; ++i) h[i] = rbf(h[i] + rbf(xn[i]));
  }
  c->len = past + L;
  /* final norm and fp32 logits of the last row (double accumulation) */
  rms_norm(h + (int64_t)(L - 1) * H, m->norm, H, m->eps, xn);
  const uint16_t* head = m->lm_head ? m->lm_head : m->embed;
#pragma omp parallel for schedule(static)
  for (int n = 0; n < m->vocab; ++n) {
    const uint16_t* wr = head + (int64_t)n * H;
    double a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int k = 0; k < H; k += 8)
      for (int j = 0; j < 8; ++j) a[j] += (double)xn[k + j] * (double)bf(wr[k + j]);
    logits[n] = (float)(((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7])));
  }
  free(h); free(xn); free(q); free(kk); free(vv); free(o); free(t); free(gg); free(uu);
}

/*
 * Greedy generation for one sequence: out_ids[0 .. n_prompt+max_new) receives
 * the prompt followed by the generated ids.  margins (nullable) receives, per
 * generated token, the gap between the largest and second-largest logit;
 * last_logits (nullable) the [vocab] logits that chose the final token.
 * Returns 0, or -1 on an invalid argument.
 */
int oracle_llama_generate(const OracleLlama* m, const int64_t* prompt, int n_prompt, int max_new,
                          int64_t* out_ids, float* margins, float* last_logits) {
  if (!m || n_prompt <= 0 || max_new < 0 || m->hidden % m->heads || m->heads % m->kv_heads ||
      m->hidden % m->group || m->ffn % m->group || m->group % 8 || m->hidden / m->heads > 512)
    return -1;
  for (int i = 0; i < n_prompt; ++i) {
    if (prompt[i] < 0 || prompt[i] >= m->vocab) return -1;
    out_ids[i] = prompt[i];
  }
  if (max_new == 0) return 0;
  Cache c;
  c.m = m;
  c.cap = n_prompt + max_new;
  c.len = 0;
  const int D = m->hidden / m->heads;
  const size_t kvn = (size_t)m->layers * m->kv_heads * c.cap * D;
  c.k = (uint16_t*)calloc(kvn, 2);
  c.v = (uint16_t*)calloc(kvn, 2);
  float* lg = (float*)malloc(sizeof(float) * (size_t)m->vocab);
  const int64_t* in = prompt;
  int L = n_prompt;
  for (int step = 0; step < max_new; ++step) {
    forward(&c, in, L, lg);
    int best = 0;
    for (int n = 1; n < m->vocab; ++n)
      if (lg[n] > lg[best]) best = n;
    float second = -INFINITY;
    for (int n = 0; n < m->vocab; ++n)
      if (n != best && lg[n] > second) second = lg[n];
    if (margins) margins[step] = lg[best] - second;
    out_ids[n_prompt + step] = best;
    in = out_ids + n_prompt + step;
    L = 1;
  }
  if (last_logits) memcpy(last_logits, lg, sizeof(float) * (size_t)m->vocab);
  free(lg);
  free(c.k);
  free(c.v);
  return 0;
}
