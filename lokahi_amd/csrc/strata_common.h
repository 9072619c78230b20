// Shared device/host helpers for the Strata MI355X (gfx950) hot-path library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/strata_hip.h"

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Streaming (non-temporal) 16-byte load: weights are read exactly once.
__device__ __forceinline__ uint4 load_nt(const uint4* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// ---------------------------------------------------------- buffer loads
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer descriptor, gfx9 data format
typedef int v4i32_t __attribute__((ext_vector_type(4)));

// Raw buffer descriptor (wave-uniform) for `bytes` bytes at p.
__device__ __forceinline__ v4i32_t rsrc(const void* p, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  v4i32_t r = {(int)(uint32_t)a, (int)((a >> 32) & 0xffffu), (int)bytes, kRsrcWord3};
  r.x = __builtin_amdgcn_readfirstlane(r.x);
  r.y = __builtin_amdgcn_readfirstlane(r.y);
  return r;
}

// Direct global -> LDS loads (buffer_load ... lds): lane l of the wave writes
// its 16 (4) bytes at LDS byte address lds + 16 l (4 l).  Issued as inline
// assembly: the compiler does not track them, so it inserts no waits for
// them; the kernel waits with explicit s_waitcnt vmcnt.
__device__ __forceinline__ void dma16(uint32_t lds, uint32_t voff, v4i32_t r, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(lds), "v"(voff), "s"(r), "s"(soff) : "memory", "m0");
}
__device__ __forceinline__ void dma4(uint32_t lds, uint32_t voff, v4i32_t r, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds"
               :: "s"(lds), "v"(voff), "s"(r), "s"(soff) : "memory", "m0");
}

// ---------------------------------------------------------------- bf16 <-> f32
// bf16 values travel as uint16_t bit patterns (upper half of an IEEE f32).
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even (same rule as torch / MLX casts; NaN stays NaN):
// the hardware conversion, v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Correctly rounded product that can never be contracted into an FMA with a
// following add (the empty asm makes the product opaque to the optimizer).
__device__ __forceinline__ float mul_rn(float a, float b) {
  float p = a * b;
  asm volatile("" : "+v"(p));
  return p;
}

// RoPE (MLXRotaryEmbedding / rotate_half, src/ollm/llama_mlx.py:95-182):
// inv_freq and cos/sin in double rounded once to fp32, angle = fp32(pos *
// inv_freq), products and sums rounded separately (no FMA).
__device__ __forceinline__ void rope_cs(int pos, int i, int D, float theta, float* c, float* s) {
#pragma clang fp contract(off)
  const float inv = static_cast<float>(1.0 / pow(static_cast<double>(theta),
                                                 static_cast<double>(2 * i) / D));
  const float ang = mul_rn(static_cast<float>(pos), inv);
  double sd, cd;
  sincos(static_cast<double>(ang), &sd, &cd);
  *c = static_cast<float>(cd);
  *s = static_cast<float>(sd);
}

__device__ __forceinline__ void rotate_pair(float x1, float x2, float c, float s, float* o1,
                                            float* o2) {
#pragma clang fp contract(off)
  *o1 = mul_rn(x1, c) + mul_rn(-x2, s);
  *o2 = mul_rn(x2, c) + mul_rn(x1, s);
}

// Element access for the two activation dtypes the library computes with.
struct bf16_t { uint16_t bits; };

template <typename T> struct Elem;
template <> struct Elem<float> {
  static __device__ __forceinline__ float load(const float* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void store(float* p, int64_t i, float v) { p[i] = v; }
};
template <> struct Elem<bf16_t> {
  static __device__ __forceinline__ float load(const bf16_t* p, int64_t i) {
    return bf16_to_f32(p[i].bits);
  }
  static __device__ __forceinline__ void store(bf16_t* p, int64_t i, float v) {
    p[i].bits = f32_to_bf16(v);
  }
};

// ---------------------------------------------------------------- wave helpers
// Cross-lane sums on DPP (no LDS round trip): within quads by quad_perm, then
// 8- and 16-lane rows by row_half_mirror / row_mirror; wider groups finish
// with lane swaps (xor_sum).  After dpp_sum<W> every lane holds the sum of its
// aligned group of W lanes.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}

// v combined with the value of the lane OFF (16 or 32) lanes away, as
// v_permlane16_swap / v_permlane32_swap of v with itself: every lane ends up
// with its own value in one result and its partner's in the other (which one
// depends on the lane; sums and maxima do not care, and a + b == b + a
// exactly).  Two VALU instructions instead of an LDS-routed ds_bpermute.
// All 64 lanes must be active.
template <int OFF>
__device__ __forceinline__ float xor_sum(float v) {
  static_assert(OFF == 16 || OFF == 32, "lane distance");
  const uint32_t u = __float_as_uint(v);
  if constexpr (OFF == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}
template <int OFF>
__device__ __forceinline__ float xor_max(float v) {
  static_assert(OFF == 16 || OFF == 32, "lane distance");
  const uint32_t u = __float_as_uint(v);
  if constexpr (OFF == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
}

template <int W>
__device__ __forceinline__ float dpp_sum(float v) {
  static_assert(W == 1 || W == 2 || W == 4 || W == 8 || W == 16 || W == 32 || W == 64, "width");
  if constexpr (W >= 2) v += dpp_f<0xB1>(v);    // quad_perm [1,0,3,2]
  if constexpr (W >= 4) v += dpp_f<0x4E>(v);    // quad_perm [2,3,0,1]
  if constexpr (W >= 8) v += dpp_f<0x141>(v);   // row_half_mirror
  if constexpr (W >= 16) v += dpp_f<0x140>(v);  // row_mirror
  if constexpr (W >= 32) v = xor_sum<16>(v);
  if constexpr (W >= 64) v = xor_sum<32>(v);
  return v;
}

__device__ __forceinline__ float wave_sum(float v) { return dpp_sum<64>(v); }

// Maximum over the 64 lanes, same DPP pattern as dpp_sum.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  v = xor_max<16>(v);
  return xor_max<32>(v);
}

template <int W>
__device__ __forceinline__ float group_sum(float v) { return dpp_sum<W>(v); }

// ---------------------------------------------------------------- host helpers
// Thread-local error message; every entry point returns a status code and
// leaves the human-readable reason here (read with strata_last_error()).
int strata_set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

#define STRATA_HIP_CHECK(expr)                                                   \
  do {                                                                           \
    hipError_t _e = (expr);                                                      \
    if (_e != hipSuccess)                                                        \
      return strata_set_error(STRATA_EHIP, "%s failed: %s", #expr,               \
                              hipGetErrorString(_e));                            \
  } while (0)

#define STRATA_REQUIRE(cond, ...)                                                \
  do {                                                                           \
    if (!(cond)) return strata_set_error(STRATA_EINVAL, __VA_ARGS__);            \
  } while (0)

struct strata_ctx {
  int device;
  int num_cus;
  int max_lds_per_block;
  void* scratch;        // device scratch arena (split-K partials), grown on demand
  size_t scratch_bytes;
  float* fixed_scratch; // this device's copy of the library's static scratch array
};

// Returns a device scratch buffer of at least `bytes` (owned by ctx).
int strata_ctx_scratch(strata_ctx* ctx, size_t bytes, void** out, void* stream);

// Floats of decode split-K partials per (b, query head): o[nsplit][D] then
// (m, s)[nsplit]; a multiple of 4 (16-byte blocks) for D % 4 == 0.
__host__ __device__ constexpr int64_t part_stride(int nsplit, int D) {
  return (int64_t)nsplit * (D + 4);
}

// Optional inputs of the attention dispatcher used by the decoder engine.
struct AttnExtra {
  const int* dlen = nullptr;  // device key count (decode; overrides Lk, which is then capacity)
  float* part = nullptr;      // caller-owned split-K partials, B * Hq * part_stride(splits, D)
  int part_splits = 0;        // splits the partials buffer holds
  int out_tm = 0;             // prefill: write token-major [B, Lq, Hq, D]
};

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
