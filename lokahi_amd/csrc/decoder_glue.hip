// Decoder glue around the hot path: RMSNorm (+ fused residual add), SiLU*up,
// residual add, embedding gather, greedy argmax and the q4 weight quantizer.
// These sit inside every decode step (src/ollm/llama_mlx.py:77-92, 399-407,
// 647-653, 724-738; src/ollm/generation.py:42-43).
#include "strata_common.h"

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

__global__ void silu_mul_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                                int64_t n, uint16_t* __restrict__ a) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float gv = bf16_to_f32(g[i]);
    const float sg = gv / (1.0f + expf(-gv));
    a[i] = f32_to_bf16(mul_rn(sg, bf16_to_f32(u[i])));
  }
}

__global__ void add_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ r,
                           int64_t n, uint16_t* __restrict__ y) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    y[i] = f32_to_bf16(bf16_to_f32(x[i]) + bf16_to_f32(r[i]));
}

__global__ void embed_kernel(const uint16_t* __restrict__ table, int64_t V, int64_t H,
                             const int32_t* __restrict__ ids, uint16_t* __restrict__ y) {
  const int64_t t = blockIdx.x;
  int64_t id = ids[t];
  if (id < 0 || id >= V) id = 0;  // ids are validated on the host side
  for (int64_t i = threadIdx.x; i < H; i += blockDim.x) y[t * H + i] = table[id * H + i];
}

// One workgroup per row; ties resolve to the lowest index.
__global__ __launch_bounds__(256) void argmax_kernel(const float* __restrict__ logits, int64_t V,
                                                     int32_t* __restrict__ out) {
  __shared__ float sv[4];
  __shared__ int si[4];
  const float* lr = logits + blockIdx.x * V;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int64_t i = threadIdx.x; i < V; i += 256) {
    const float v = lr[i];
    if (v > best) { best = v; bi = static_cast<int>(i); }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(best, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) { sv[wave] = best; si[wave] = bi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w)
      if (sv[w] > best || (sv[w] == best && si[w] < bi)) { best = sv[w]; bi = si[w]; }
    out[blockIdx.x] = bi == 0x7fffffff ? 0 : bi;
  }
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
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<uint16_t*>(x), reinterpret_cast<const uint16_t*>(res), w, H,
                     eps, reinterpret_cast<uint16_t*>(y));
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}

int strata_silu_mul_launch(const void* g, const void* u, int64_t n, void* a, void* stream) {
  hipLaunchKernelGGL(silu_mul_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream),
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

int strata_embed_launch(const uint16_t* table, int64_t V, int64_t H, const int32_t* ids,
                        int64_t n, void* y, void* stream) {
  hipLaunchKernelGGL(embed_kernel, dim3(n), dim3(256), 0, as_stream(stream), table, V, H, ids,
                     (uint16_t*)y);
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}

int strata_argmax_launch(const float* logits, int64_t rows, int64_t V, int32_t* out, void* stream) {
  hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(256), 0, as_stream(stream), logits, V, out);
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
