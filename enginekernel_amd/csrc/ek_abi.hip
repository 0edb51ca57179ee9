// Error strings and library identification for the C ABI.

#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstring>

#include "ek_abi_internal.h"
#include "ek_hip.h"

#include <atomic>

namespace {
thread_local char g_err[256] = {0};
std::atomic<int64_t> g_wait_limit{0};   // 0: each kernel's own default
}

int64_t ek_wait_limit(int64_t dflt) {
  const int64_t v = g_wait_limit.load(std::memory_order_relaxed);
  return v > 0 ? v : dflt;
}

hipError_t ek_fail(hipError_t code, const char* msg) {
  std::snprintf(g_err, sizeof(g_err), "%s", msg);
  return code;
}

void ek_clear_error() { g_err[0] = 0; }

extern "C" {

const char* ek_last_error(void) { return g_err; }

const char* ek_version(void) { return "enginekernel_amd 0.2 gfx950"; }

int64_t ek_set_wait_limit(int64_t polls) {
  return g_wait_limit.exchange(polls > 0 ? polls : 0, std::memory_order_relaxed);
}

// Report the device the current HIP context targets: compute units and the
// gfx architecture name (e.g. "gfx950"). Returns a hipError_t.
int ek_device_info(int* n_cu, char* arch, int arch_len) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) return e;
  if (n_cu) *n_cu = prop.multiProcessorCount;
  if (arch && arch_len > 0) std::snprintf(arch, (size_t)arch_len, "%s", prop.gcnArchName);
  return hipSuccess;
}

}  // extern "C"
