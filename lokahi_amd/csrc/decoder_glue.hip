// Decoder glue around the hot path: RMSNorm (+ fused residual add), SiLU*up,
// residual add, embedding gather, greedy argmax and the q4 weight quantizer.
// These sit inside every decode step (src/ollm/llama_mlx.py:77-92, 399-407,
// 647-653, 724-738; src/ollm/generation.py:42-43).
#include "strata_internal.h"

// Products and sums are rounded separately (no FMA contraction) so the glue
// matches its CPU restatement operation by operation.
#pragma clang fp contract(off)

namespace {

// Block-wide sum for 256 threads.
__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  const float t = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return t;
}

// One workgroup per row.  If res != nullptr: x <- bf16(x + res) first.
// Vector path: each thread holds NV uint4 (8 bf16 each) of the row in
// registers, so x is read once; the generic path re-reads x.
template <int NV>
__global__ __launch_bounds__(256) void rmsnorm_vec_kernel(uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ res,
                                                          const uint16_t* __restrict__ w,
                                                          int64_t H, float eps,
                                                          uint16_t* __restrict__ y) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  uint4* xr = reinterpret_cast<uint4*>(x + row * H);
  const uint4* rr = res ? reinterpret_cast<const uint4*>(res + row * H) : nullptr;
  const uint4* wr = reinterpret_cast<const uint4*>(w);
  uint4* yr = reinterpret_cast<uint4*>(y + row * H);
  const int nvec = static_cast<int>(H >> 3);
  float v[NV][8];
  float ss = 0.f;
  uint4 xa[NV], ra[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int i = min((int)threadIdx.x + 256 * j, nvec - 1);
    xa[j] = xr[i];
    ra[j] = rr ? rr[i] : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int i = threadIdx.x + 256 * j;
    const uint32_t xu[4] = {xa[j].x, xa[j].y, xa[j].z, xa[j].w};
    const uint32_t ru[4] = {ra[j].x, ra[j].y, ra[j].z, ra[j].w};
    uint32_t hu[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float lo = __uint_as_float(xu[c] << 16), hi = __uint_as_float(xu[c] & 0xffff0000u);
      if (rr) {
        lo = bf16_to_f32(f32_to_bf16(lo + __uint_as_float(ru[c] << 16)));
        hi = bf16_to_f32(f32_to_bf16(hi + __uint_as_float(ru[c] & 0xffff0000u)));
      }
      hu[c] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
      v[j][2 * c] = lo;
      v[j][2 * c + 1] = hi;
    }
    if (i < nvec) {
      if (rr) xr[i] = make_uint4(hu[0], hu[1], hu[2], hu[3]);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(v[j][e], v[j][e], ss);
    }
  }
  const float tot = block_sum256(ss, red);
  const float r = 1.0f / sqrtf(tot / static_cast<float>(H) + eps);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int i = threadIdx.x + 256 * j;
    if (i >= nvec) continue;
    const uint4 wv = wr[i];
    const uint32_t wu[4] = {wv.x, wv.y, wv.z, wv.w};
    uint32_t o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float a = mul_rn(mul_rn(v[j][2 * c], r), __uint_as_float(wu[c] << 16));
      const float bb = mul_rn(mul_rn(v[j][2 * c + 1], r), __uint_as_float(wu[c] & 0xffff0000u));
      o[c] = static_cast<uint32_t>(f32_to_bf16(a)) | (static_cast<uint32_t>(f32_to_bf16(bb)) << 16);
    }
    yr[i] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

__global__ __launch_bounds__(256) void rmsnorm_kernel(uint16_t* __restrict__ x,
                                                      const uint16_t* __restrict__ res,
                                                      const uint16_t* __restrict__ w, int64_t H,
                                                      float eps, uint16_t* __restrict__ y) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  uint16_t* xr = x + row * H;
  const uint16_t* rr = res ? res + row * H : nullptr;
  uint16_t* yr = y + row * H;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < H; i += 256) {
    float v = bf16_to_f32(xr[i]);
    if (rr) {
      const uint16_t hb = f32_to_bf16(v + bf16_to_f32(rr[i]));
      xr[i] = hb;
      v = bf16_to_f32(hb);
    }
    ss = fmaf(v, v, ss);
  }
  const float tot = block_sum256(ss, red);
  const float r = 1.0f / sqrtf(tot / static_cast<float>(H) + eps);
  for (int64_t i = threadIdx.x; i < H; i += 256) {
    const float v = bf16_to_f32(xr[i]);
    yr[i] = f32_to_bf16(mul_rn(mul_rn(v, r), bf16_to_f32(w[i])));
  }
}

__device__ __forceinline__ uint16_t silu_mul1(uint16_t g, uint16_t u) {
  const float gv = bf16_to_f32(g);
  const float sg = gv / (1.0f + expf(-gv));
  return f32_to_bf16(mul_rn(sg, bf16_to_f32(u)));
}

// Elementwise over n values; with VEC the pointers are 16-byte aligned and
// n % 8 == 0, and each thread takes 8 values per 16-byte load (the same
// arithmetic per value).
template <bool VEC>
__global__ void silu_mul_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                                int64_t n, uint16_t* __restrict__ a) {
  if constexpr (VEC) {
    const int64_t n8 = n >> 3;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n8;
         i += (int64_t)gridDim.x * blockDim.x) {
      const uint4 gv = reinterpret_cast<const uint4*>(g)[i];
      const uint4 uv = reinterpret_cast<const uint4*>(u)[i];
      const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
      uint32_t o[4];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        o[c] = (uint32_t)silu_mul1((uint16_t)gw[c], (uint16_t)uw[c]) |
               ((uint32_t)silu_mul1((uint16_t)(gw[c] >> 16), (uint16_t)(uw[c] >> 16)) << 16);
      reinterpret_cast<uint4*>(a)[i] = make_uint4(o[0], o[1], o[2], o[3]);
    }
  } else {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
      a[i] = silu_mul1(g[i], u[i]);
  }
}

__global__ void add_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ r,
                           int64_t n, uint16_t* __restrict__ y) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    y[i] = f32_to_bf16(bf16_to_f32(x[i]) + bf16_to_f32(r[i]));
}

// Clears n bytes (a kernel, not hipMemsetAsync: memset nodes recorded into a
// captured graph have given wrong results on replays after the first).
__global__ void zero_fill_kernel(uint8_t* __restrict__ p, int64_t n) {
  const int64_t n16 = n >> 4;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n16;
       i += (int64_t)gridDim.x * blockDim.x)
    reinterpret_cast<uint4*>(p)[i] = make_uint4(0, 0, 0, 0);
  const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (t < (n & 15)) p[(n16 << 4) + t] = 0;
}

__global__ void embed_kernel(const uint16_t* __restrict__ table, int64_t V, int64_t H,
                             const int32_t* __restrict__ ids, uint16_t* __restrict__ y) {
  const int64_t t = blockIdx.x;
  int64_t id = ids[t];
  if (id < 0 || id >= V) id = 0;  // ids are validated on the host side
  for (int64_t i = threadIdx.x; i < H; i += blockDim.x) y[t * H + i] = table[id * H + i];
}

// Greedy argmax in two stages: grid (nb, rows) workgroups each reduce a
// slice of the row to (value, index); one workgroup per row reduces the nb
// partials.  Ties resolve to the lowest index.
__device__ __forceinline__ void argmax_pick(float& best, int& bi, float v, int i) {
  if (v > best || (v == best && i < bi)) { best = v; bi = i; }
}

__device__ __forceinline__ void argmax_block(float& best, int& bi, float* sv, int* si) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(best, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    argmax_pick(best, bi, ov, oi);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) { sv[wave] = best; si[wave] = bi; }
  __syncthreads();
  if (threadIdx.x == 0)
    for (int w = 1; w < 4; ++w) argmax_pick(best, bi, sv[w], si[w]);
}

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* __restrict__ logits,
                                                             int64_t V, float temperature,
                                                             int slice, float* __restrict__ pv,
                                                             int* __restrict__ pi) {
  __shared__ float sv[4];
  __shared__ int si[4];
  const int row = blockIdx.y;
  const float* lr = logits + (int64_t)row * V;
  const int64_t lo = (int64_t)blockIdx.x * slice;
  const int64_t hi = min(V, lo + slice);
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int64_t i = lo + threadIdx.x; i < hi; i += 256) {
    // argmax(logits / T) as generation.py:42-43 evaluates it (fp32 divide)
    const float v = temperature == 1.0f ? lr[i] : __fdiv_rn(lr[i], temperature);
    argmax_pick(best, bi, v, static_cast<int>(i));
  }
  argmax_block(best, bi, sv, si);
  if (threadIdx.x == 0) {
    pv[row * gridDim.x + blockIdx.x] = best;
    pi[row * gridDim.x + blockIdx.x] = bi;
  }
}

__global__ __launch_bounds__(256) void argmax_final_kernel(const float* __restrict__ pv,
                                                           const int* __restrict__ pi, int nb,
                                                           int32_t* __restrict__ out) {
  __shared__ float sv[4];
  __shared__ int si[4];
  const int row = blockIdx.x;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = threadIdx.x; i < nb; i += 256) argmax_pick(best, bi, pv[row * nb + i], pi[row * nb + i]);
  argmax_block(best, bi, sv, si);
  if (threadIdx.x == 0) out[row] = bi == 0x7fffffff ? 0 : bi;
}

// One thread per group of 64.
template <typename T>
__global__ void quantize_kernel(const T* __restrict__ src, int64_t N, int64_t K, int G,
                                uint32_t* __restrict__ w, uint16_t* __restrict__ sc,
                                uint16_t* __restrict__ bi) {
  const int64_t ngroups = N * (K / G);
  for (int64_t gi = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; gi < ngroups;
       gi += (int64_t)gridDim.x * blockDim.x) {
    const T* p = src + gi * G;  // groups are contiguous along K within a row
    float mn = INFINITY, mx = -INFINITY;
    for (int i = 0; i < G; ++i) {
      const float v = Elem<T>::load(p, i);
      mn = fminf(mn, v);
      mx = fmaxf(mx, v);
    }
    const float scale = fmaxf(__fdiv_rn(__fsub_rn(mx, mn), 15.0f), 1e-8f);
    const uint16_t sb = f32_to_bf16(scale), bb = f32_to_bf16(mn);
    sc[gi] = sb;
    bi[gi] = bb;
    const float s = bf16_to_f32(sb), b = bf16_to_f32(bb);
    uint32_t* wo = w + gi * (G / 8);
    for (int wd = 0; wd < G / 8; ++wd) {
      uint32_t word = 0;
      for (int j = 0; j < 8; ++j) {
        float qv = rintf(__fdiv_rn(__fsub_rn(Elem<T>::load(p, wd * 8 + j), b), s));
        qv = fminf(fmaxf(qv, 0.f), 15.f);
        word |= static_cast<uint32_t>(qv) << (4 * j);
      }
      wo[wd] = word;
    }
  }
}

inline int grid_for(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return static_cast<int>(g);
}

}  // namespace

int strata_rmsnorm_launch(void* x, const void* res, const uint16_t* w, int64_t rows, int64_t H,
                          float eps, void* y, void* stream) {
  const bool al = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(res) |
                    reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(y)) & 15u) == 0;
  if (al && H % 8 == 0 && H <= 8 * 256 * 4) {
    const int nv = static_cast<int>((H / 8 + 255) / 256);
    hipStream_t s = as_stream(stream);
    uint16_t* xx = reinterpret_cast<uint16_t*>(x);
    const uint16_t* rr = reinterpret_cast<const uint16_t*>(res);
    uint16_t* yy = reinterpret_cast<uint16_t*>(y);
    if (nv == 1) hipLaunchKernelGGL(rmsnorm_vec_kernel<1>, dim3(rows), dim3(256), 0, s, xx, rr, w, H, eps, yy);
    else if (nv == 2) hipLaunchKernelGGL(rmsnorm_vec_kernel<2>, dim3(rows), dim3(256), 0, s, xx, rr, w, H, eps, yy);
    else if (nv == 3) hipLaunchKernelGGL(rmsnorm_vec_kernel<3>, dim3(rows), dim3(256), 0, s, xx, rr, w, H, eps, yy);
    else hipLaunchKernelGGL(rmsnorm_vec_kernel<4>, dim3(rows), dim3(256), 0, s, xx, rr, w, H, eps, yy);
    STRATA_HIP_CHECK(hipGetLastError());
    return STRATA_OK;
  }
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<uint16_t*>(x), reinterpret_cast<const uint16_t*>(res), w, H,
                     eps, reinterpret_cast<uint16_t*>(y));
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}

int strata_silu_mul_launch(const void* g, const void* u, int64_t n, void* a, void* stream) {
  if (n % 8 == 0 && aligned16(g) && aligned16(u) && aligned16(a))
    hipLaunchKernelGGL(silu_mul_kernel<true>, dim3(grid_for(n / 8)), dim3(256), 0,
                       as_stream(stream), (const uint16_t*)g, (const uint16_t*)u, n, (uint16_t*)a);
  else
    hipLaunchKernelGGL(silu_mul_kernel<false>, dim3(grid_for(n)), dim3(256), 0, as_stream(stream),
                       (const uint16_t*)g, (const uint16_t*)u, n, (uint16_t*)a);
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}

int strata_add_launch(const void* x, const void* r, int64_t n, void* y, void* stream) {
  hipLaunchKernelGGL(add_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream),
                     (const uint16_t*)x, (const uint16_t*)r, n, (uint16_t*)y);
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}

int strata_zero_fill_launch(void* p, int64_t bytes, void* stream) {
  if (bytes <= 0) return STRATA_OK;
  STRATA_REQUIRE(aligned16(p), "zero fill: pointer must be 16-byte aligned");
  const int64_t n16 = (bytes >> 4) > 0 ? (bytes >> 4) : 1;
  hipLaunchKernelGGL(zero_fill_kernel, dim3(grid_for(n16)), dim3(256), 0, as_stream(stream),
                     (uint8_t*)p, bytes);
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}

int strata_embed_launch(const uint16_t* table, int64_t V, int64_t H, const int32_t* ids,
                        int64_t n, void* y, void* stream) {
  hipLaunchKernelGGL(embed_kernel, dim3(n), dim3(256), 0, as_stream(stream), table, V, H, ids,
                     (uint16_t*)y);
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}

int strata_argmax_launch(const float* logits, int64_t rows, int64_t V, float temperature,
                         int32_t* out, void* partial, void* stream) {
  // partial: rows * kArgmaxBlocks * 8 bytes (values then indices)
  const int nb = kArgmaxBlocks;
  const int slice = static_cast<int>((V + nb - 1) / nb);
  float* pv = reinterpret_cast<float*>(partial);
  int* pi = reinterpret_cast<int*>(pv + rows * nb);
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(argmax_partial_kernel, dim3(nb, rows), dim3(256), 0, s, logits, V,
                     temperature, slice, pv, pi);
  hipLaunchKernelGGL(argmax_final_kernel, dim3(rows), dim3(256), 0, s, pv, pi, nb, out);
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}

int strata_quantize_launch(const void* src, int dtype, int64_t N, int64_t K, int G, uint32_t* w,
                           uint16_t* s, uint16_t* b, void* stream) {
  const int64_t ng = N * (K / G);
  if (dtype == STRATA_BF16)
    hipLaunchKernelGGL((quantize_kernel<bf16_t>), dim3(grid_for(ng)), dim3(256), 0,
                       as_stream(stream), (const bf16_t*)src, N, K, G, w, s, b);
  else
    hipLaunchKernelGGL((quantize_kernel<float>), dim3(grid_for(ng)), dim3(256), 0,
                       as_stream(stream), (const float*)src, N, K, G, w, s, b);
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}

namespace {
// End of a decode step in one workgroup: the greedy token of each batch row
// from the argmax partials, recorded in ids and out[row, step]; the row's
// embedding gathered into h for the next step (llama_mlx.py:724-738); then
// the counters advance and the RoPE row of the new position is staged, as
// decode_advance_kernel does.
__global__ __launch_bounds__(256) void decode_tail_kernel(
    const float* __restrict__ pv, const int* __restrict__ pi, int nb, int B,
    int32_t* __restrict__ ids, int32_t* __restrict__ out, int out_stride,
    int* __restrict__ counters, const float2* __restrict__ rope_table, int lmax, int half,
    float2* __restrict__ rope_cur, const uint16_t* __restrict__ table, int64_t H, int vec,
    uint16_t* __restrict__ h) {
  __shared__ float sv[4];
  __shared__ int si[4];
  __shared__ int sid;
  const int step = counters[0];
  const int pos = counters[1] + 1;
  for (int b = 0; b < B; ++b) {
    float best = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = threadIdx.x; i < nb; i += 256) argmax_pick(best, bi, pv[b * nb + i], pi[b * nb + i]);
    argmax_block(best, bi, sv, si);
    if (threadIdx.x == 0) {
      const int id = bi == 0x7fffffff ? 0 : bi;
      ids[b] = id;
      out[(int64_t)b * out_stride + step] = id;
      sid = id;
    }
    __syncthreads();
    const int64_t id = sid;
    if (vec) {
      const uint4* src = reinterpret_cast<const uint4*>(table + id * H);
      uint4* dst = reinterpret_cast<uint4*>(h + (int64_t)b * H);
      for (int64_t i = threadIdx.x; i < H / 8; i += 256) dst[i] = src[i];
    } else {
      for (int64_t i = threadIdx.x; i < H; i += 256) h[(int64_t)b * H + i] = table[id * H + i];
    }
    __syncthreads();  // sv, si, sid are reused by the next row
  }
  if (rope_cur && pos >= 0 && pos < lmax)
    for (int t = threadIdx.x; t < half; t += 256) rope_cur[t] = rope_table[(int64_t)pos * half + t];
  __syncthreads();
  if (threadIdx.x == 0) {
    counters[0] = step + 1;
    counters[1] += 1;
    counters[2] += 1;
  }
}
}  // namespace

int strata_decode_tail_launch(const float* logits, int B, int64_t V, float temperature,
                              void* partial, int32_t* ids, int32_t* out_tokens, int out_stride,
                              int* counters, const float2* rope_table, int lmax, int half,
                              float2* rope_cur, const uint16_t* table, int64_t H, void* h,
                              void* stream) {
  const int nb = kArgmaxBlocks;
  const int slice = static_cast<int>((V + nb - 1) / nb);
  float* pv = reinterpret_cast<float*>(partial);
  int* pi = reinterpret_cast<int*>(pv + (int64_t)B * nb);
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(argmax_partial_kernel, dim3(nb, B), dim3(256), 0, s, logits, V, temperature,
                     slice, pv, pi);
  const int vec = H % 8 == 0 && ((reinterpret_cast<uintptr_t>(table) | reinterpret_cast<uintptr_t>(h)) & 15) == 0;
  hipLaunchKernelGGL(decode_tail_kernel, dim3(1), dim3(256), 0, s, pv, pi, nb, B, ids, out_tokens,
                     out_stride, counters, rope_table, lmax, half, rope_cur, table, H, vec,
                     (uint16_t*)h);
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}

namespace {
// End of a graph-replayed decode step: record the token chosen for each batch
// row, advance the device counters {step, position, key count}, and stage
// the RoPE (cos, sin) row of the new position for the next step's q/k/v
// epilogue (a position past the table is never used: nothing is staged).
__global__ void decode_advance_kernel(const int32_t* __restrict__ ids, int B,
                                      int32_t* __restrict__ out, int out_stride,
                                      int* __restrict__ counters,
                                      const float2* __restrict__ rope_table, int lmax, int half,
                                      float2* __restrict__ rope_cur) {
  const int step = counters[0];
  const int pos = counters[1] + 1;
  for (int b = threadIdx.x; b < B; b += blockDim.x) out[(int64_t)b * out_stride + step] = ids[b];
  if (rope_cur && pos >= 0 && pos < lmax)
    for (int t = threadIdx.x; t < half; t += blockDim.x) rope_cur[t] = rope_table[(int64_t)pos * half + t];
  __syncthreads();
  if (threadIdx.x == 0) {
    counters[0] = step + 1;
    counters[1] += 1;
    counters[2] += 1;
  }
}
}  // namespace

int strata_decode_advance_launch(const int32_t* ids, int B, int32_t* out_tokens, int out_stride,
                                 int* counters, const float2* rope_table, int lmax, int half,
                                 float2* rope_cur, void* stream) {
  hipLaunchKernelGGL(decode_advance_kernel, dim3(1), dim3(64), 0, as_stream(stream), ids, B,
                     out_tokens, out_stride, counters, rope_table, lmax, half, rope_cur);
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}
