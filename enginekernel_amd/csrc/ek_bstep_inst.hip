// Instantiations of the batch decode-step kernel for one row bound: compiled
// once per MB with -DEK_BSTEP_MB=<2|4|8> (head dim 128, the Qwen3 family's).

#include "ek_bstep_impl.h"

#ifndef EK_BSTEP_MB
#error "compile with -DEK_BSTEP_MB=<row bound>"
#endif

namespace eks {

template <int G>
static hipError_t launch_b(const StepArgs& a, int nwg, hipStream_t st) {
  constexpr int MB = EK_BSTEP_MB;
  const size_t lds = bstep_lds_bytes<128, G, MB>(a.h, a.nq * 128, a.part_max, a.lchunk, nwg);
  static bool attr_done = false;   // allow more than 64 KiB of dynamic LDS
  if (!attr_done) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&batch_step_kernel<128, G, MB>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kStepDynLds);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return e;
    }
    attr_done = true;
  }
  hipLaunchKernelGGL((batch_step_kernel<128, G, MB>), dim3(nwg), dim3(SNT), lds, st, a);
  return hipGetLastError();
}

template <int G>
static int occupancy_b(size_t lds) {
  constexpr int MB = EK_BSTEP_MB;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(&batch_step_kernel<128, G, MB>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)kStepDynLds) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(&batch_step_kernel<128, G, MB>),
                                                   SNT, lds) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

template <>
hipError_t launch_bstep<EK_BSTEP_MB>(const StepArgs& a, int g, int nwg, hipStream_t st) {
  switch (g) {
    case 2: return launch_b<2>(a, nwg, st);
    case 4: return launch_b<4>(a, nwg, st);
    default: return hipErrorInvalidValue;
  }
}

template <>
int bstep_occupancy<EK_BSTEP_MB>(int g, size_t lds) {
  switch (g) {
    case 2: return occupancy_b<2>(lds);
    case 4: return occupancy_b<4>(lds);
    default: return 0;
  }
}

}  // namespace eks
