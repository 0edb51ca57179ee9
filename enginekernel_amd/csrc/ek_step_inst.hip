// Instantiations of the persistent decode-step kernel for one head dim:
// compiled once per head dim with -DEK_STEP_D=<32|64|128> so that the
// instantiations build in parallel.

#include "ek_step_impl.h"

#ifndef EK_STEP_D
#error "compile with -DEK_STEP_D=<head dim>"
#endif

namespace eks {

template <int D, int G, bool LONG>
static hipError_t launch_one(const StepArgs& a, int nwg, hipStream_t st) {
  const size_t lds = step_lds_bytes<D, G, LONG>(a.h, a.kpad_max, a.part_max, a.s_cap, a.lchunk);
  static bool attr_done = false;   // allow more than 64 KiB of dynamic LDS (gfx950 has 160 KiB per CU)
  if (!attr_done) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&step_kernel<D, G, LONG>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kStepDynLds);
    if (e != hipSuccess) {
      (void)hipGetLastError();   // do not leave the error for the next launch's check
      return e;
    }
    attr_done = true;
  }
  hipLaunchKernelGGL((step_kernel<D, G, LONG>), dim3(nwg), dim3(SNT), lds, st, a);
  return hipGetLastError();
}

template <int D, int G, bool LONG>
static int occupancy_one(size_t lds) {
  // a failed query leaves no error behind for the next launch's check
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(&step_kernel<D, G, LONG>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)kStepDynLds) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(&step_kernel<D, G, LONG>), SNT,
                                                   lds) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

template <bool LONG>
static int occupancy_g(int g, size_t lds) {
  switch (g) {
    case 2: return occupancy_one<EK_STEP_D, 2, LONG>(lds);
    case 4: return occupancy_one<EK_STEP_D, 4, LONG>(lds);
    default: return 0;
  }
}

template <bool LONG>
static hipError_t launch_g(const StepArgs& a, int g, int nwg, hipStream_t st) {
  switch (g) {
    case 2: return launch_one<EK_STEP_D, 2, LONG>(a, nwg, st);
    case 4: return launch_one<EK_STEP_D, 4, LONG>(a, nwg, st);
    default: return hipErrorInvalidValue;
  }
}

template <>
int step_occupancy<EK_STEP_D>(int g, bool lng, size_t lds) {
  return lng ? occupancy_g<true>(g, lds) : occupancy_g<false>(g, lds);
}

template <>
hipError_t launch_step<EK_STEP_D>(const StepArgs& a, int g, int nwg, hipStream_t st) {
  return a.lsplit > 0 ? launch_g<true>(a, g, nwg, st) : launch_g<false>(a, g, nwg, st);
}

}  // namespace eks
