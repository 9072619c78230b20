// Plain-read floor of the decode GEMV's launches (measurement helper, no
// counterpart in the reference): a grid-stride stream of 16-byte loads with
// `U` loads in flight per lane and no other work.
#include <hip/hip_runtime.h>

#include "strata_common.h"

namespace {

template <int U>
__global__ __launch_bounds__(256) void bench_read_kernel(const uint4* __restrict__ p, int64_t n16,
                                                         uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t waves = (int64_t)gridDim.x * 4;
  uint32_t acc = 0;
  // each wave reads U contiguous KiB per step (one KiB per load instruction)
  for (int64_t base = wave * 64 * U; base < n16; base += waves * 64 * U) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = load_nt(p + min(base + u * 64 + lane, n16 - 1));
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9e3779b9u) sink[threadIdx.x & 3] = acc;
}

}  // namespace

extern "C" int strata_bench_read(strata_ctx* ctx, const void* p, int64_t bytes, int wg_per_cu,
                                 int unroll, void* sink, void* stream) {
  STRATA_REQUIRE(ctx != nullptr && p != nullptr && sink != nullptr, "bench_read: null argument");
  STRATA_REQUIRE(bytes > 0 && bytes % 16 == 0, "bench_read: bytes=%lld must be a positive multiple of 16",
                 (long long)bytes);
  STRATA_REQUIRE(wg_per_cu >= 1 && wg_per_cu <= 16, "bench_read: wg_per_cu=%d not in 1..16", wg_per_cu);
  const dim3 grid(ctx->num_cus * wg_per_cu), block(256);
  const uint4* src = static_cast<const uint4*>(p);
  uint32_t* out = static_cast<uint32_t*>(sink);
  hipStream_t st = as_stream(stream);
  switch (unroll) {
    case 4: hipLaunchKernelGGL(bench_read_kernel<4>, grid, block, 0, st, src, bytes / 16, out); break;
    case 8: hipLaunchKernelGGL(bench_read_kernel<8>, grid, block, 0, st, src, bytes / 16, out); break;
    case 16: hipLaunchKernelGGL(bench_read_kernel<16>, grid, block, 0, st, src, bytes / 16, out); break;
    default: return strata_set_error(STRATA_EINVAL, "bench_read: unroll=%d not in {4, 8, 16}", unroll);
  }
  STRATA_HIP_CHECK(hipGetLastError());
  return STRATA_OK;
}
