// RoPE and KV-cache append for gfx950.
//
// RoPE restates MLXRotaryEmbedding + apply_rotary_pos_emb_mlx / rotate_half
// (src/ollm/llama_mlx.py:95-182): inv_freq[i] = 1/theta^(2i/D),
// angle = fp32(fp32(pos) * inv_freq[i]), emb = [angle, angle], and
//   out[i]       = x[i]       * cos - x[i+D/2] * sin
//   out[i + D/2] = x[i + D/2] * cos + x[i]       * sin
// inv_freq, cos and sin are evaluated in double and rounded once to fp32;
// each product and the sum are rounded separately (no contraction), which
// makes the kernel bit-identical to the build's CPU restatement.
//
// The KV append replaces MLXKVCache.update's concatenate
// (src/ollm/mlx_kvcache.py:65-125) with an O(Lnew) write into a
// preallocated [B, Hkv, Lmax, D] buffer per layer.
#include <algorithm>

#include "strata_internal.h"

namespace {

// In-place RoPE on x [B, H, L, D]; one thread per (b, h, l, i < D/2).
template <typename T>
__global__ void rope_inplace(T* __restrict__ x, const int32_t* __restrict__ pos, int B, int H,
                             int L, int D, float theta) {
  const int half = D / 2;
  const int64_t total = (int64_t)B * H * L * half;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int i = idx % half;
    const int64_t r = idx / half;  // (b*H + h)*L + l
    const int l = r % L;
    const int b = (r / L) / H;
    float c, s;
    rope_cs(pos[(int64_t)b * L + l], i, D, theta, &c, &s);
    const int64_t off = r * D;
    float o1, o2;
    rotate_pair(Elem<T>::load(x, off + i), Elem<T>::load(x, off + i + half), c, s, &o1, &o2);
    Elem<T>::store(x, off + i, o1);
    Elem<T>::store(x, off + i + half, o2);
  }
}

// Append src [B, H, Lnew, D] into cache [B, H, Lmax, D] at pos0 (dtype convert).
template <typename TS, typename TC>
__global__ void kv_copy(const TS* __restrict__ src, TC* __restrict__ dst, int B, int H, int Lnew,
                        int Lmax, int D, int pos0) {
  const int64_t total = (int64_t)B * H * Lnew * D;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int d = idx % D;
    const int64_t r = idx / D;
    const int l = r % Lnew;
    const int64_t bh = r / Lnew;
    Elem<TC>::store(dst, (bh * Lmax + pos0 + l) * D + d, Elem<TS>::load(src, idx));
  }
}

// Fused: token-major projections q_src [B, L, Hq*D], k_src/v_src [B, L, Hkv*D]
// -> q_out [B, Hq, L, D] rotated, cache K[b,h,pos0+l,:] rotated, V copied.
// A thread owns (b, l, i < D/2) and the heads h = blockIdx.y + k * gridDim.y
// of the Hq + 2*Hkv (q, then k, then v): (cos, sin) of (pos, i) is computed
// once for all its heads, and a wave touches 128 contiguous bytes per head.
template <typename TS, typename TC>
__global__ void rope_kv_fused(const TS* __restrict__ qs, const TS* __restrict__ ks,
                              const TS* __restrict__ vs, int B, int Hq, int Hkv, int L, int D,
                              int Lmax, int pos0, const int* __restrict__ dpos, float theta,
                              TS* __restrict__ q_out, TC* __restrict__ kc, TC* __restrict__ vc,
                              const float2* __restrict__ table) {
  // dpos (device) overrides pos0: the decode step replayed from a HIP graph
  // reads its position from memory the previous step advanced.
  if (dpos) pos0 = *dpos;
  const int half = D / 2;
  const int NH = Hq + 2 * Hkv;
  const int64_t total = (int64_t)B * L * half;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int i = idx % half;
    const int64_t r = idx / half;
    const int l = r % L;
    const int b = r / L;
    const int pos = pos0 + l;
    float c = 0.f, s = 0.f;
    if ((int)blockIdx.y < Hq + Hkv) {
      if (table) {  // the same values, built once by rope_cs
        const float2 cs = table[(int64_t)pos * half + i];
        c = cs.x;
        s = cs.y;
      } else {
        rope_cs(pos, i, D, theta, &c, &s);
      }
    }
    for (int h = blockIdx.y; h < NH; h += gridDim.y) {
      if (h < Hq) {
        const int64_t so = ((int64_t)b * L + l) * Hq * D + (int64_t)h * D;
        float o1, o2;
        rotate_pair(Elem<TS>::load(qs, so + i), Elem<TS>::load(qs, so + i + half), c, s, &o1, &o2);
        const int64_t oo = (((int64_t)b * Hq + h) * L + l) * D;
        Elem<TS>::store(q_out, oo + i, o1);
        Elem<TS>::store(q_out, oo + i + half, o2);
      } else if (h < Hq + Hkv) {
        const int hk = h - Hq;
        const int64_t so = ((int64_t)b * L + l) * Hkv * D + (int64_t)hk * D;
        // K is rotated in the source dtype first (the projection output
        // dtype), then stored in the cache dtype.
        float o1, o2;
        rotate_pair(Elem<TS>::load(ks, so + i), Elem<TS>::load(ks, so + i + half), c, s, &o1, &o2);
        if constexpr (sizeof(TS) == 2) {
          o1 = bf16_to_f32(f32_to_bf16(o1));
          o2 = bf16_to_f32(f32_to_bf16(o2));
        }
        const int64_t co = (((int64_t)b * Hkv + hk) * Lmax + pos) * D;
        Elem<TC>::store(kc, co + i, o1);
        Elem<TC>::store(kc, co + i + half, o2);
      } else {
        const int hv = h - Hq - Hkv;
        const int64_t so = ((int64_t)b * L + l) * Hkv * D + (int64_t)hv * D;
        const int64_t co = (((int64_t)b * Hkv + hv) * Lmax + pos) * D;
        Elem<TC>::store(vc, co + i, Elem<TS>::load(vs, so + i));
        Elem<TC>::store(vc, co + i + half, Elem<TS>::load(vs, so + i + half));
      }
    }
  }
}

// The bf16 fused kernel with a (cos, sin) table, 8 pairs per thread: a
// thread owns (b, l, 8-pair chunk) and moves 16 bytes per load and store;
// the same arithmetic per pair as rope_kv_fused.  D % 16 == 0, 16-byte
// aligned operands.
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__global__ void rope_kv_fused_v8(const uint16_t* __restrict__ qs, const uint16_t* __restrict__ ks,
                                 const uint16_t* __restrict__ vs, int B, int Hq, int Hkv, int L,
                                 int D, int Lmax, int pos0, const int* __restrict__ dpos,
                                 uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc,
                                 uint16_t* __restrict__ vc, const float2* __restrict__ table) {
  if (dpos) pos0 = *dpos;
  const int half = D / 2, nc = half / 8;
  const int NH = Hq + 2 * Hkv;
  const int64_t total = (int64_t)B * L * nc;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int i0 = 8 * (int)(idx % nc);
    const int64_t r = idx / nc;
    const int l = r % L;
    const int b = r / L;
    const int pos = pos0 + l;
    float c[8], sn[8];
    if ((int)blockIdx.y < Hq + Hkv) {
      const float4* tp = reinterpret_cast<const float4*>(table + (int64_t)pos * half + i0);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 t = tp[q];
        c[2 * q] = t.x;
        sn[2 * q] = t.y;
        c[2 * q + 1] = t.z;
        sn[2 * q + 1] = t.w;
      }
    }
    for (int h = blockIdx.y; h < NH; h += gridDim.y) {
      const uint16_t* src;
      uint16_t* dst;
      int64_t so;
      if (h < Hq) {
        so = ((int64_t)b * L + l) * Hq * D + (int64_t)h * D;
        src = qs;
        dst = q_out + (((int64_t)b * Hq + h) * L + l) * D;
      } else {
        const int hk = h < Hq + Hkv ? h - Hq : h - Hq - Hkv;
        so = ((int64_t)b * L + l) * Hkv * D + (int64_t)hk * D;
        src = h < Hq + Hkv ? ks : vs;
        dst = (h < Hq + Hkv ? kc : vc) + (((int64_t)b * Hkv + hk) * Lmax + pos) * D;
      }
      const uint4 a = *reinterpret_cast<const uint4*>(src + so + i0);
      const uint4 e = *reinterpret_cast<const uint4*>(src + so + i0 + half);
      if (h >= Hq + Hkv) {  // V: copied
        *reinterpret_cast<uint4*>(dst + i0) = a;
        *reinterpret_cast<uint4*>(dst + i0 + half) = e;
        continue;
      }
      const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, ew[4] = {e.x, e.y, e.z, e.w};
      uint32_t o1w[4], o2w[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float p1, p2, r1, r2;
        rotate_pair(bf_lo(aw[q]), bf_lo(ew[q]), c[2 * q], sn[2 * q], &p1, &p2);
        rotate_pair(bf_hi(aw[q]), bf_hi(ew[q]), c[2 * q + 1], sn[2 * q + 1], &r1, &r2);
        o1w[q] = (uint32_t)f32_to_bf16(p1) | ((uint32_t)f32_to_bf16(r1) << 16);
        o2w[q] = (uint32_t)f32_to_bf16(p2) | ((uint32_t)f32_to_bf16(r2) << 16);
      }
      *reinterpret_cast<uint4*>(dst + i0) = make_uint4(o1w[0], o1w[1], o1w[2], o1w[3]);
      *reinterpret_cast<uint4*>(dst + i0 + half) = make_uint4(o2w[0], o2w[1], o2w[2], o2w[3]);
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

int strata_rope_launch(void* q, void* k, const int32_t* pos, int B, int Hq, int Hkv, int L, int D,
                       float theta, int dtype, void* stream) {
  hipStream_t s = as_stream(stream);
  struct Item { void* p; int H; } items[2] = {{q, Hq}, {k, Hkv}};
  for (const Item& it : items) {
    if (!it.p) continue;
    const int64_t n = (int64_t)B * it.H * L * (D / 2);
    if (dtype == STRATA_BF16)
      hipLaunchKernelGGL(rope_inplace<bf16_t>, dim3(grid_for(n)), dim3(256), 0, s,
                         reinterpret_cast<bf16_t*>(it.p), pos, B, it.H, L, D, theta);
    else
      hipLaunchKernelGGL(rope_inplace<float>, dim3(grid_for(n)), dim3(256), 0, s,
                         reinterpret_cast<float*>(it.p), pos, B, it.H, L, D, theta);
    STRATA_HIP_CHECK(hipGetLastError());
  }
  return STRATA_OK;
}

int strata_kv_copy_launch(const void* src, int src_dtype, void* dst, int dst_dtype, int B, int H,
                          int Lnew, int Lmax, int D, int pos0, void* stream) {
  hipStream_t s = as_stream(stream);
  const int64_t n = (int64_t)B * H * Lnew * D;
  const dim3 g(grid_for(n)), blk(256);
  if (src_dtype == STRATA_BF16 && dst_dtype == STRATA_BF16)
    hipLaunchKernelGGL((kv_copy<bf16_t, bf16_t>), g, blk, 0, s, (const bf16_t*)src, (bf16_t*)dst, B,
                       H, Lnew, Lmax, D, pos0);
  else if (src_dtype == STRATA_F32 && dst_dtype == STRATA_F32)
    hipLaunchKernelGGL((kv_copy<float, float>), g, blk, 0, s, (const float*)src, (float*)dst, B, H,
                       Lnew, Lmax, D, pos0);
  else if (src_dtype == STRATA_F32 && dst_dtype == STRATA_BF16)
    hipLaunchKernelGGL((kv_copy<float, bf16_t>), g, blk, 0, s, (const float*)src, (bf16_t*)dst, B,
                       H, Lnew, Lmax, D, pos0);
  else
    hipLaunchKernelGGL((kv_copy<bf16_t, float>), g, blk, 0, s, (const bf16_t*)src, (float*)dst, B,
                       H, Lnew, Lmax, D, pos0);
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}

int strata_rope_kv_fused_launch(const void* qs, const void* ks, const void* vs, int src_dtype,
                                int B, int Hq, int Hkv, int L, int D, int Lmax, int pos0,
                                const int* dpos, float theta, void* q_out, void* kc, void* vc,
                                int cache_dtype, void* stream, const void* rope_table) {
  hipStream_t s = as_stream(stream);
  // Heads are dealt over grid.y: all of them for short inputs (as many
  // threads as elements), slices of 6 from 256 rows, so (cos, sin) is
  // computed once per 6 heads.
  const int NH = Hq + 2 * Hkv;
  const int64_t rows = (int64_t)B * L;
  const int hy = rows >= 256 ? std::max(1, (NH + 5) / 6) : NH;
  const dim3 g(grid_for(rows * (D / 2)), hy), blk(256);
  const bool v8 = rope_table && D % 16 == 0 && aligned16(qs) && aligned16(ks) && aligned16(vs) &&
                  aligned16(q_out) && aligned16(kc) && aligned16(vc);
  if (src_dtype == STRATA_BF16 && cache_dtype == STRATA_BF16 && v8) {
    const dim3 g8(grid_for(rows * (D / 16)), hy);
    hipLaunchKernelGGL(rope_kv_fused_v8, g8, blk, 0, s, (const uint16_t*)qs, (const uint16_t*)ks,
                       (const uint16_t*)vs, B, Hq, Hkv, L, D, Lmax, pos0, dpos, (uint16_t*)q_out,
                       (uint16_t*)kc, (uint16_t*)vc, (const float2*)rope_table);
  } else if (src_dtype == STRATA_BF16 && cache_dtype == STRATA_BF16)
    hipLaunchKernelGGL((rope_kv_fused<bf16_t, bf16_t>), g, blk, 0, s, (const bf16_t*)qs,
                       (const bf16_t*)ks, (const bf16_t*)vs, B, Hq, Hkv, L, D, Lmax, pos0, dpos, theta,
                       (bf16_t*)q_out, (bf16_t*)kc, (bf16_t*)vc, (const float2*)rope_table);
  else if (src_dtype == STRATA_F32 && cache_dtype == STRATA_F32)
    hipLaunchKernelGGL((rope_kv_fused<float, float>), g, blk, 0, s, (const float*)qs,
                       (const float*)ks, (const float*)vs, B, Hq, Hkv, L, D, Lmax, pos0, dpos, theta,
                       (float*)q_out, (float*)kc, (float*)vc, (const float2*)rope_table);
  else
    return strata_set_error(STRATA_ENOTSUP,
                            "rope_kv_append: source and cache dtypes must match");
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}

namespace {
__global__ void rope_table_kernel(float2* __restrict__ table, int lmax, int D, float theta) {
  const int half = D >> 1;
  const int64_t n = (int64_t)lmax * half;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < n;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int pos = static_cast<int>(idx / half), i = static_cast<int>(idx % half);
    float c, s;
    rope_cs(pos, i, D, theta, &c, &s);
    table[idx] = make_float2(c, s);
  }
}
}  // namespace

int strata_rope_table_launch(float2* table, int lmax, int D, float theta, void* stream) {
  const int64_t n = (int64_t)lmax * (D / 2);
  const int blocks = static_cast<int>(std::min<int64_t>((n + 255) / 256, 4096));
  hipLaunchKernelGGL(rope_table_kernel, dim3(blocks), dim3(256), 0, as_stream(stream), table, lmax,
                     D, theta);
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}
