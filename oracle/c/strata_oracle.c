/*
 * strata_oracle.c — plain-C restatement of the reference hot path
 * (TEST INFRASTRUCTURE / CPU BASELINE ONLY; never part of the product).
 *
 * oracle_q4_matmul   follows `_linear` -> mx.quantized_matmul(transpose=True)
 *                    (src/ollm/llama_mlx.py:53-74): y = x @ (s*q + b).T,
 *                    q = nibble k%8 of word k/8 (LSB first), fp32 accumulate
 *                    per group then summed in double per row.
 * oracle_decode_attn follows online_chunked_grouped_attention_mx for one query
 *                    per (batch, head) (src/ollm/backends/mlx_ops.py:32-152,
 *                    decode = one key block, llama_mlx.py:300-308), fp32.
 * Parallelised with OpenMP over output rows / heads.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static inline float bf16f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f2bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* x [M,K] (f32), w u32 [N,K/8], s/b bf16 [N,K/G]; y [M,N] f32. */
void oracle_q4_matmul(const float* x, int64_t M, int64_t K, const uint32_t* w, const uint16_t* s,
                      const uint16_t* b, int64_t N, int G, float* y) {
  const int64_t ng = K / G;
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t m = 0; m < M; ++m) {
      const float* xr = x + m * K;
      double acc = 0.0;
      for (int64_t g = 0; g < ng; ++g) {
        const float sc = bf16f(s[n * ng + g]), bi = bf16f(b[n * ng + g]);
        float dq = 0.f, xs = 0.f;
        for (int64_t k = g * G; k < (g + 1) * G; ++k) {
          const uint32_t q = (w[n * (K / 8) + k / 8] >> (4 * (k % 8))) & 15u;
          dq += xr[k] * (float)q;
          xs += xr[k];
        }
        acc += (double)sc * dq + (double)bi * xs;
      }
      y[m * N + n] = (float)acc;
    }
  }
}

/* Same as above with bf16 activations and bf16 output (the decode GEMV's I/O). */
void oracle_q4_gemv_bf16(const uint16_t* x, int64_t K, const uint32_t* w, const uint16_t* s,
                         const uint16_t* b, int64_t N, int G, uint16_t* y) {
  const int64_t ng = K / G;
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    float acc = 0.f;
    for (int64_t g = 0; g < ng; ++g) {
      const float sc = bf16f(s[n * ng + g]), bi = bf16f(b[n * ng + g]);
      float dq = 0.f, xs = 0.f;
      const uint32_t* wr = w + n * (K / 8) + g * (G / 8);
      for (int j = 0; j < G / 8; ++j) {
        const uint32_t word = wr[j];
        for (int e = 0; e < 8; ++e) {
          const float xv = bf16f(x[g * G + j * 8 + e]);
          dq += xv * (float)((word >> (4 * e)) & 15u);
          xs += xv;
        }
      }
      acc += sc * dq + bi * xs;
    }
    y[n] = f2bf16(acc);
  }
}

/* q [B,Hq,D] f32, k/v [B,Hkv,L,D] bf16 (cache), out [B,Hq,D] f32. */
void oracle_decode_attn(const float* q, const uint16_t* k, const uint16_t* v, int B, int Hq,
                        int Hkv, int L, int D, float* out) {
  const int G = Hq / Hkv;
  const float scale = 1.0f / sqrtf((float)D);
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b) {
    for (int h = 0; h < Hq; ++h) {
      const int hk = h / G;
      const float* qr = q + ((int64_t)b * Hq + h) * D;
      const uint16_t* kb = k + ((int64_t)b * Hkv + hk) * (int64_t)L * D;
      const uint16_t* vb = v + ((int64_t)b * Hkv + hk) * (int64_t)L * D;
      float m = -INFINITY, sum = 0.f;
      float acc[256];
      for (int d = 0; d < D; ++d) acc[d] = 0.f;
      for (int t = 0; t < L; ++t) {
        float sc = 0.f;
        for (int d = 0; d < D; ++d) sc += qr[d] * bf16f(kb[(int64_t)t * D + d]);
        sc *= scale;
        const float mn = sc > m ? sc : m;
        const float alpha = expf(m - mn), p = expf(sc - mn);
        sum = sum * alpha + p;
        for (int d = 0; d < D; ++d) acc[d] = acc[d] * alpha + p * bf16f(vb[(int64_t)t * D + d]);
        m = mn;
      }
      float* o = out + ((int64_t)b * Hq + h) * D;
      for (int d = 0; d < D; ++d) o[d] = acc[d] / (sum > 1e-12f ? sum : 1e-12f);
    }
  }
}

/* Dense bf16 GEMV y = W x (lm_head), W [N,K] bf16, x [K] bf16 -> y fp32. */
void oracle_bf16_gemv(const uint16_t* x, int64_t K, const uint16_t* w, int64_t N, float* y) {
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    float acc = 0.f;
    const uint16_t* wr = w + n * K;
    for (int64_t k = 0; k < K; ++k) acc += bf16f(wr[k]) * bf16f(x[k]);
    y[n] = acc;
  }
}
