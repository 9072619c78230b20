// Decode-side quantized (q4 affine, group 64) and bf16 matrix-vector kernels.
//
// y[m, n] = sum_k x[m, k] * (s[n, k/64] * q[n, k] + b[n, k/64])
// (mx.quantized_matmul(transpose=True), src/ollm/llama_mlx.py:53-74)
//
// Design (HBM-bound streaming, gfx950 wave64):
//   * x for MT batch rows is staged once per workgroup into LDS, already
//     rearranged into bf16 pairs (x[8j+c], x[8j+c+4]) so that one AND-OR of a
//     packed word with the magic 0x43004300 yields the matching bf16 pair
//     (128+q[8j+c], 128+q[8j+c+4]) exactly; v_dot2_f32_bf16 then accumulates
//     x*(128+q) in fp32.  Per 32-element half group the offset is removed
//     with the precomputed LDS sum X = sum x:
//         acc += s * D + (b - 128 s) * X
//   * every lane streams one 16-byte uint4 (32 codes) per row per step, so a
//     wave reads 1 KiB contiguous per row per step (fully coalesced), R rows
//     at once to keep R*16 B per lane in flight and reuse the x reads;
//   * workgroups walk row blocks grid-stride; several linears that share x
//     (q/k/v, gate/up) are one launch ("problems" concatenated by row).
//   * lanes reduce with xor-butterflies at the end; results are deterministic.
#include "strata_common.h"

namespace {

constexpr int kMaxProblems = 8;
constexpr uint32_t kMagicPair = 0x43004300u;  // bf16 (128.0, 128.0)

struct Q4Problem {
  const uint4* w;      // [n, K/32] uint4  (== uint32 [n, K/8])
  const uint16_t* s;   // [n, K/64] bf16
  const uint16_t* b;   // [n, K/64] bf16
  void* y;             // [M, n]
  int n;
  int row0;
};

struct Q4Batch {
  Q4Problem p[kMaxProblems];
  int count;
  int total_rows;
};

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

template <typename YT>
__device__ __forceinline__ void store_y(void* y, int64_t idx, float v) {
  Elem<YT>::store(reinterpret_cast<YT*>(y), idx, v);
}

// Stage MT rows of x (bf16 or f32) into LDS.
//   bf16: xq[(mm*4 + j) * nv + i] = uint4 of the 4 bf16 pairs of word 4i+j,
//         xs[mm * nv + i]         = sum of the 32 x values of uint4 i.
//   f32 : xf[(mm*8 + c) * nv + i] = float4 of elements 32i+4c .. 32i+4c+3,
//         xs as above.
template <typename XT, int MT>
__device__ __forceinline__ void stage_x(const XT* __restrict__ x, int M, int K, int m0,
                                        uint4* smem, int nv) {
  float* xs;
  if constexpr (sizeof(XT) == 2) {
    uint4* xq = smem;
    xs = reinterpret_cast<float*>(smem + MT * 4 * nv);
    for (int idx = threadIdx.x; idx < MT * nv; idx += blockDim.x) {
      const int mm = idx / nv, i = idx - mm * nv;
      const int m = m0 + mm;
      float sum = 0.f;
      const uint4* xr = reinterpret_cast<const uint4*>(x) + ((int64_t)m * K + (int64_t)i * 32) / 8;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint4 v = make_uint4(0, 0, 0, 0);
        if (m < M) v = xr[j];
        uint4 pr;
        pr.x = (v.x & 0xffffu) | (v.z << 16);
        pr.y = (v.x >> 16) | (v.z & 0xffff0000u);
        pr.z = (v.y & 0xffffu) | (v.w << 16);
        pr.w = (v.y >> 16) | (v.w & 0xffff0000u);
        xq[(mm * 4 + j) * nv + i] = pr;
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int c = 0; c < 4; ++c)
          sum += __uint_as_float(u[c] << 16) + __uint_as_float(u[c] & 0xffff0000u);
      }
      xs[mm * nv + i] = sum;
    }
  } else {
    float4* xf = reinterpret_cast<float4*>(smem);
    xs = reinterpret_cast<float*>(smem + MT * 8 * nv);
    for (int idx = threadIdx.x; idx < MT * nv; idx += blockDim.x) {
      const int mm = idx / nv, i = idx - mm * nv;
      const int m = m0 + mm;
      float sum = 0.f;
      const float4* xr = reinterpret_cast<const float4*>(x + (int64_t)m * K + (int64_t)i * 32);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (m < M) v = xr[c];
        xf[(mm * 8 + c) * nv + i] = v;
        sum += (v.x + v.y) + (v.z + v.w);
      }
      xs[mm * nv + i] = sum;
    }
  }
}

template <int R, int MT, typename XT, typename YT>
__global__ __launch_bounds__(256) void q4_gemv_kernel(const XT* __restrict__ x, int M, int K,
                                                      Q4Batch batch) {
  extern __shared__ uint4 smem[];
  const int nv = K >> 5;  // uint4 (32 codes) per weight row
  const int m0 = blockIdx.y * MT;
  stage_x<XT, MT>(x, M, K, m0, smem, nv);
  __syncthreads();

  const float* xs = reinterpret_cast<const float*>(smem + MT * (sizeof(XT) == 2 ? 4 : 8) * nv);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rows_per_block = 4 * R;
  const int nrb = (batch.total_rows + rows_per_block - 1) / rows_per_block;

  for (int rb = blockIdx.x; rb < nrb; rb += gridDim.x) {
    const uint4* wp[R];
    const uint16_t* sp[R];
    const uint16_t* bp[R];
    int pid[R], nloc[R];
    bool valid[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = rb * rows_per_block + wave * R + r;
      valid[r] = row < batch.total_rows;
      int pi = 0;
#pragma unroll
      for (int t = 1; t < kMaxProblems; ++t)
        if (t < batch.count && row >= batch.p[t].row0) pi = t;
      const int n = valid[r] ? row - batch.p[pi].row0 : 0;
      pid[r] = pi;
      nloc[r] = n;
      wp[r] = batch.p[pi].w + (int64_t)n * nv;
      sp[r] = batch.p[pi].s + (int64_t)n * (nv >> 1);
      bp[r] = batch.p[pi].b + (int64_t)n * (nv >> 1);
    }

    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int mm = 0; mm < MT; ++mm) acc[r][mm] = 0.f;

    for (int i = lane; i < nv; i += 64) {
      uint4 wv[R];
      float sc[R], bc[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        wv[r] = valid[r] ? load_nt(wp[r] + i) : make_uint4(0, 0, 0, 0);
        sc[r] = valid[r] ? bf16_to_f32(sp[r][i >> 1]) : 0.f;
        bc[r] = valid[r] ? bf16_to_f32(bp[r][i >> 1]) : 0.f;
      }
#pragma unroll
      for (int mm = 0; mm < MT; ++mm) {
        const float xsum = xs[mm * nv + i];
        if constexpr (sizeof(XT) == 2) {
          const uint4* xq = smem;
          uint4 xa[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) xa[j] = xq[(mm * 4 + j) * nv + i];
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const uint32_t ww[4] = {wv[r].x, wv[r].y, wv[r].z, wv[r].w};
            float d = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const uint32_t w = ww[j];
              d = dot2_bf16((w & 0x000f000fu) | kMagicPair, xa[j].x, d);
              d = dot2_bf16(((w >> 4) & 0x000f000fu) | kMagicPair, xa[j].y, d);
              d = dot2_bf16(((w >> 8) & 0x000f000fu) | kMagicPair, xa[j].z, d);
              d = dot2_bf16(((w >> 12) & 0x000f000fu) | kMagicPair, xa[j].w, d);
            }
            acc[r][mm] = fmaf(sc[r], d, acc[r][mm]);
            acc[r][mm] = fmaf(fmaf(-128.f, sc[r], bc[r]), xsum, acc[r][mm]);
          }
        } else {
          const float4* xf = reinterpret_cast<const float4*>(smem);
          float4 xa[8];
#pragma unroll
          for (int c = 0; c < 8; ++c) xa[c] = xf[(mm * 8 + c) * nv + i];
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const uint32_t ww[4] = {wv[r].x, wv[r].y, wv[r].z, wv[r].w};
            float d = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const uint32_t lo = ww[j] & 0x0f0f0f0fu;         // codes 0,2,4,6
              const uint32_t hi = (ww[j] >> 4) & 0x0f0f0f0fu;  // codes 1,3,5,7
              const float4 xa0 = xa[2 * j], xa1 = xa[2 * j + 1];
              d = fmaf(xa0.x, (float)(lo & 0xff), d);
              d = fmaf(xa0.y, (float)(hi & 0xff), d);
              d = fmaf(xa0.z, (float)((lo >> 8) & 0xff), d);
              d = fmaf(xa0.w, (float)((hi >> 8) & 0xff), d);
              d = fmaf(xa1.x, (float)((lo >> 16) & 0xff), d);
              d = fmaf(xa1.y, (float)((hi >> 16) & 0xff), d);
              d = fmaf(xa1.z, (float)(lo >> 24), d);
              d = fmaf(xa1.w, (float)(hi >> 24), d);
            }
            acc[r][mm] = fmaf(sc[r], d, acc[r][mm]);
            acc[r][mm] = fmaf(bc[r], xsum, acc[r][mm]);
          }
        }
      }
    }

#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int mm = 0; mm < MT; ++mm) acc[r][mm] = wave_sum(acc[r][mm]);

#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int mm = 0; mm < MT; ++mm) {
        const int m = m0 + mm;
        if (lane == r * MT + mm && valid[r] && m < M) {
          const Q4Problem& p = batch.p[pid[r]];
          store_y<YT>(p.y, (int64_t)m * p.n + nloc[r], acc[r][mm]);
        }
      }
  }
}

// Dense bf16-weight GEMV (lm_head): y[m,n] = sum_k x[m,k] * W[n,k].
template <int R, int MT, typename YT>
__global__ __launch_bounds__(256) void bf16_gemv_kernel(const uint16_t* __restrict__ x, int M,
                                                        int K, const uint4* __restrict__ w,
                                                        int N, YT* __restrict__ y) {
  extern __shared__ uint4 smem[];
  const int nv = K >> 3;  // uint4 (8 bf16) per row
  const int m0 = blockIdx.y * MT;
  for (int idx = threadIdx.x; idx < MT * nv; idx += blockDim.x) {
    const int mm = idx / nv, i = idx - mm * nv;
    const int m = m0 + mm;
    smem[idx] = (m < M) ? reinterpret_cast<const uint4*>(x + (int64_t)m * K)[i]
                        : make_uint4(0, 0, 0, 0);
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nrb = (N + 4 * R - 1) / (4 * R);
  for (int rb = blockIdx.x; rb < nrb; rb += gridDim.x) {
    const int row0 = rb * 4 * R + wave * R;
    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int mm = 0; mm < MT; ++mm) acc[r][mm] = 0.f;
    for (int i = lane; i < nv; i += 64) {
      uint4 wv[R];
#pragma unroll
      for (int r = 0; r < R; ++r)
        wv[r] = (row0 + r < N) ? load_nt(w + (int64_t)(row0 + r) * nv + i)
                               : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int mm = 0; mm < MT; ++mm) {
        const uint4 xa = smem[mm * nv + i];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float d = acc[r][mm];
          d = dot2_bf16(wv[r].x, xa.x, d);
          d = dot2_bf16(wv[r].y, xa.y, d);
          d = dot2_bf16(wv[r].z, xa.z, d);
          d = dot2_bf16(wv[r].w, xa.w, d);
          acc[r][mm] = d;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int mm = 0; mm < MT; ++mm) acc[r][mm] = wave_sum(acc[r][mm]);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int mm = 0; mm < MT; ++mm) {
        const int m = m0 + mm;
        if (lane == r * MT + mm && row0 + r < N && m < M)
          Elem<YT>::store(y, (int64_t)m * N + row0 + r, acc[r][mm]);
      }
  }
}

template <int R, int MT, typename XT, typename YT>
int launch_q4(strata_ctx* ctx, const void* x, int M, int K, const Q4Batch& batch,
              hipStream_t stream) {
  const int nv = K / 32;
  const size_t lds = (size_t)MT * nv * (sizeof(XT) == 2 ? 64 : 128) + (size_t)MT * nv * 4;
  STRATA_REQUIRE((int64_t)lds <= ctx->max_lds_per_block,
                 "q4 GEMV: K=%d needs %zu B of LDS per batch tile, device allows %d", K, lds,
                 ctx->max_lds_per_block);
  const int nrb = (batch.total_rows + 4 * R - 1) / (4 * R);
  const int per_cu = lds <= 32768 ? 4 : (lds <= 53248 ? 3 : 2);
  const int gx = nrb < ctx->num_cus * per_cu ? nrb : ctx->num_cus * per_cu;
  dim3 grid(gx, (M + MT - 1) / MT);
  hipLaunchKernelGGL((q4_gemv_kernel<R, MT, XT, YT>), grid, dim3(256), lds, stream,
                     reinterpret_cast<const XT*>(x), M, K, batch);
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}

template <typename XT, typename YT>
int dispatch_q4_m(strata_ctx* ctx, const void* x, int M, int K, const Q4Batch& batch,
                  hipStream_t stream) {
  // Batch tile: as many x rows per pass as LDS allows (each pass re-streams
  // the weights, so small-M decode should fit in one pass).
  const size_t per_row = (size_t)(K / 32) * ((sizeof(XT) == 2 ? 64 : 128) + 4);
  const size_t cap = (size_t)ctx->max_lds_per_block;
  if (M >= 4 && 4 * per_row <= cap) return launch_q4<2, 4, XT, YT>(ctx, x, M, K, batch, stream);
  if (M >= 2 && 2 * per_row <= cap) return launch_q4<2, 2, XT, YT>(ctx, x, M, K, batch, stream);
  return launch_q4<4, 1, XT, YT>(ctx, x, M, K, batch, stream);
}

}  // namespace

int strata_q4_gemv(strata_ctx* ctx, const void* x, int x_dtype, int M, int K,
                   const strata_q4_weight* ws, int count, int y_dtype, void* stream) {
  Q4Batch batch{};
  batch.count = count;
  int rows = 0;
  for (int i = 0; i < count; ++i) {
    batch.p[i].w = reinterpret_cast<const uint4*>(ws[i].w);
    batch.p[i].s = ws[i].scales;
    batch.p[i].b = ws[i].biases;
    batch.p[i].y = ws[i].y;
    batch.p[i].n = static_cast<int>(ws[i].N);
    batch.p[i].row0 = rows;
    rows += static_cast<int>(ws[i].N);
  }
  batch.total_rows = rows;
  hipStream_t s = as_stream(stream);
  if (x_dtype == STRATA_BF16 && y_dtype == STRATA_BF16)
    return dispatch_q4_m<bf16_t, bf16_t>(ctx, x, M, K, batch, s);
  if (x_dtype == STRATA_BF16 && y_dtype == STRATA_F32)
    return dispatch_q4_m<bf16_t, float>(ctx, x, M, K, batch, s);
  if (x_dtype == STRATA_F32 && y_dtype == STRATA_F32)
    return dispatch_q4_m<float, float>(ctx, x, M, K, batch, s);
  if (x_dtype == STRATA_F32 && y_dtype == STRATA_BF16)
    return dispatch_q4_m<float, bf16_t>(ctx, x, M, K, batch, s);
  return strata_set_error(STRATA_EINVAL, "q4 GEMV: unsupported dtype pair (%d, %d)", x_dtype,
                          y_dtype);
}

int strata_bf16_gemv(strata_ctx* ctx, const void* x, int M, int K, const uint16_t* w, int N,
                     void* y, int y_dtype, void* stream) {
  constexpr int R = 4;
  const int MT = M >= 4 ? 4 : (M >= 2 ? 2 : 1);
  const size_t lds = (size_t)MT * K * 2;
  STRATA_REQUIRE((int64_t)lds <= ctx->max_lds_per_block, "bf16 GEMV: K=%d too large", K);
  const int nrb = (N + 4 * R - 1) / (4 * R);
  const int gx = nrb < ctx->num_cus * 4 ? nrb : ctx->num_cus * 4;
  dim3 grid(gx, (M + MT - 1) / MT);
  hipStream_t s = as_stream(stream);
  const uint16_t* xx = reinterpret_cast<const uint16_t*>(x);
  const uint4* ww = reinterpret_cast<const uint4*>(w);
#define STRATA_BF16_LAUNCH(MTV)                                                            \
  if (MT == MTV) {                                                                         \
    if (y_dtype == STRATA_F32)                                                             \
      hipLaunchKernelGGL((bf16_gemv_kernel<R, MTV, float>), grid, dim3(256), lds, s, xx, M, \
                         K, ww, N, reinterpret_cast<float*>(y));                           \
    else                                                                                   \
      hipLaunchKernelGGL((bf16_gemv_kernel<R, MTV, bf16_t>), grid, dim3(256), lds, s, xx,  \
                         M, K, ww, N, reinterpret_cast<bf16_t*>(y));                       \
  }
  STRATA_BF16_LAUNCH(1)
  STRATA_BF16_LAUNCH(2)
  STRATA_BF16_LAUNCH(4)
#undef STRATA_BF16_LAUNCH
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}
