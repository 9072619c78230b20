// strata-hip-probe: the native evidence lane of the "hip" backend.
//
// The reference's MetalBackend runs a native probe executable and reads one
// JSON evidence envelope from its stdout (src/ollm/backends/metal_backend.py:
// 74-163: schema_version 1, backend, dispatch_success, device_name,
// operation, dtype, numerical_max_error, timing.average_dispatch_wall_time_ms,
// failure_reason; a non-zero exit status marks failure).  This executable
// produces the same envelope for the HIP library: it binds a context to the
// device (STRATA_HIP_DEVICE, default 0), runs the library's numerical self-test
// (a q4 GEMV against a closed-form host reference) and times repeated
// dispatches of that GEMV with HIP events.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "strata_hip.h"

namespace {

std::string escape(const char* s) {
  std::string out;
  for (; s && *s; ++s) {
    if (*s == '"' || *s == '\\') out += '\\';
    if (static_cast<unsigned char>(*s) >= 0x20) out += *s;
  }
  return out;
}

int fail(const std::string& device, const char* why) {
  std::printf("{\"schema_version\":1,\"backend\":\"hip\",\"device_name\":\"%s\","
              "\"operation\":\"linear_q4_gemv\",\"dtype\":\"bf16x_q4w_f32y\","
              "\"dispatch_success\":false,\"failure_reason\":\"%s\"}\n",
              escape(device.c_str()).c_str(), escape(why).c_str());
  return 1;
}

}  // namespace

int main() {
  const char* dev_env = std::getenv("STRATA_HIP_DEVICE");
  const int device = dev_env ? std::atoi(dev_env) : 0;
  hipDeviceProp_t prop;
  std::string device_name = "unknown";
  if (hipGetDeviceProperties(&prop, device) == hipSuccess)
    device_name = std::string(prop.name) + " (" + prop.gcnArchName + ")";
  strata_ctx* ctx = nullptr;
  if (strata_ctx_create(device, &ctx) != STRATA_OK) return fail(device_name, strata_last_error());

  char env[512];
  const int rc = strata_selftest(ctx, env, sizeof(env));
  // the self-test envelope carries the numerical result
  const char* key = "\"numerical_max_error\":";
  const char* at = std::strstr(env, key);
  const double max_err = at ? std::atof(at + std::strlen(key)) : -1.0;
  if (rc != STRATA_OK) {
    const std::string why = strata_last_error();
    strata_ctx_destroy(ctx);
    return fail(device_name, why.c_str());
  }

  // timing: the self-test's GEMV shape (N=64, K=128), 200 dispatches
  const int N = 64, K = 128, iters = 200;
  void *w = nullptr, *s = nullptr, *b = nullptr, *x = nullptr, *y = nullptr;
  hipEvent_t e0, e1;
  float ms = 0.f;
  bool timed = hipMalloc(&w, N * K / 2) == hipSuccess && hipMalloc(&s, N * K / 32) == hipSuccess &&
               hipMalloc(&b, N * K / 32) == hipSuccess && hipMalloc(&x, K * 2) == hipSuccess &&
               hipMalloc(&y, N * 4) == hipSuccess && hipMemset(w, 0, N * K / 2) == hipSuccess &&
               hipMemset(s, 0, N * K / 32) == hipSuccess && hipMemset(b, 0, N * K / 32) == hipSuccess &&
               hipMemset(x, 0, K * 2) == hipSuccess && hipEventCreate(&e0) == hipSuccess &&
               hipEventCreate(&e1) == hipSuccess;
  if (timed) {
    for (int i = 0; i < iters + 10 && timed; ++i) {
      if (i == 10) timed = hipEventRecord(e0, nullptr) == hipSuccess;
      timed = timed && strata_linear_q4(ctx, x, STRATA_BF16, 1, K, (const uint32_t*)w,
                                        (const uint16_t*)s, (const uint16_t*)b, N, 64, 4, y,
                                        STRATA_F32, nullptr) == STRATA_OK;
    }
    timed = timed && hipEventRecord(e1, nullptr) == hipSuccess &&
            hipEventSynchronize(e1) == hipSuccess && hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
  }
  (void)hipFree(w); (void)hipFree(s); (void)hipFree(b); (void)hipFree(x); (void)hipFree(y);
  strata_ctx_destroy(ctx);
  if (!timed) return fail(device_name, "timed dispatch of the q4 GEMV failed");
  std::printf("{\"schema_version\":1,\"backend\":\"hip\",\"device_name\":\"%s\","
              "\"operation\":\"linear_q4_gemv\",\"dtype\":\"bf16x_q4w_f32y\","
              "\"dispatch_success\":true,\"numerical_max_error\":%.9g,\"threshold\":1e-4,"
              "\"timing\":{\"iterations\":%d,\"average_dispatch_wall_time_ms\":%.6f}}\n",
              escape(device_name.c_str()).c_str(), max_err, iters, ms / iters);
  return 0;
}
