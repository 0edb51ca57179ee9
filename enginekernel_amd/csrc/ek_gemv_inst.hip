// One (prologue, epilogue) pair of the GEMV family: the FMA kernel
// instantiated over batch tiles, chunks per lane and rows per wave, and the
// matrix-core kernel over batch tiles and ring depths. The build compiles this file
// once per pair with -DEK_PRO=<prologue> -DEK_EPI=<epilogue> so that the
// instantiations compile in parallel.

#include "ek_gemv_impl.h"

#ifndef EK_PRO
#error "compile with -DEK_PRO=<prologue> -DEK_EPI=<epilogue>"
#endif

namespace ekg {
namespace {

template <int PRO, int EPI, int BM, int KPL, int RPW>
hipError_t launch_t(const GemvParams& p, dim3 grid, size_t lds, hipStream_t st) {
  hipLaunchKernelGGL((gemv_kernel<PRO, EPI, BM, KPL, RPW>), grid, dim3(NTHR), lds, st, p);
  return hipGetLastError();
}

// Whole-row register blocks (KPL 8 and 19, K = 4096 and 9728) exist for one
// row per wave only: at 2 or 4 rows per wave they would not fit the register
// file (the compiler spills them), so those launches take the generic
// 4-chunk block loop, which is correct for any K.
template <int PRO, int EPI, int BM, int RPW>
hipError_t launch_k(const GemvParams& p, int kpl, dim3 grid, size_t lds, hipStream_t st) {
  switch (kpl) {
    case 1: return launch_t<PRO, EPI, BM, 1, RPW>(p, grid, lds, st);
    case 5: return launch_t<PRO, EPI, BM, 5, RPW>(p, grid, lds, st);
    default: break;
  }
  if constexpr (RPW == 1) {
    if (kpl == 8) return launch_t<PRO, EPI, BM, 8, RPW>(p, grid, lds, st);
    if (kpl == 19) return launch_t<PRO, EPI, BM, 19, RPW>(p, grid, lds, st);
  }
  return launch_t<PRO, EPI, BM, 4, RPW>(p, grid, lds, st);
}

// 8 batch rows x 4 rows per wave (x2 for the gate/up pairs) is more
// accumulators than the register file holds: such launches run 2 rows per wave
template <int PRO, int EPI, int BM>
hipError_t launch_r(const GemvParams& p, int kpl, int rpw, dim3 grid, size_t lds, hipStream_t st) {
  if (rpw == 1) return launch_k<PRO, EPI, BM, 1>(p, kpl, grid, lds, st);
  if constexpr (BM == 8) {
    return launch_k<PRO, EPI, BM, 2>(p, kpl, grid, lds, st);
  } else {
    if (rpw == 2) return launch_k<PRO, EPI, BM, 2>(p, kpl, grid, lds, st);
    return launch_k<PRO, EPI, BM, 4>(p, kpl, grid, lds, st);
  }
}

template <int PRO, int EPI>
hipError_t launch_b(const GemvParams& p, int bm, int kpl, int rpw, dim3 grid, size_t lds, hipStream_t st) {
  switch (bm) {
    case 1: return launch_r<PRO, EPI, 1>(p, kpl, rpw, grid, lds, st);
    case 2: return launch_r<PRO, EPI, 2>(p, kpl, rpw, grid, lds, st);
    case 4: return launch_r<PRO, EPI, 4>(p, kpl, rpw, grid, lds, st);
    default: return launch_r<PRO, EPI, 8>(p, kpl, rpw, grid, lds, st);
  }
}

template <int PRO, int EPI, int BM, int NB>
hipError_t launch_m(const GemvParams& p, dim3 grid, size_t lds, hipStream_t st) {
  hipLaunchKernelGGL((gemv_mfma_kernel<PRO, EPI, BM, NB>), grid, dim3(mfma_threads(EPI)), lds, st, p);
  return hipGetLastError();
}

// ring depths (mfma_nb in ek_gemv.hip): up to 20 for single row tiles, up
// to 10 for the gate/up pairs
template <int PRO, int EPI, int BM>
hipError_t launch_mn(const GemvParams& p, int nb, dim3 grid, size_t lds, hipStream_t st) {
  if constexpr (EPI != EPI_SWIGLU) {
    switch (nb) {
      case 20: return launch_m<PRO, EPI, BM, 20>(p, grid, lds, st);
      case 19: return launch_m<PRO, EPI, BM, 19>(p, grid, lds, st);
      case 16: return launch_m<PRO, EPI, BM, 16>(p, grid, lds, st);
      default: break;
    }
  }
  switch (nb) {
    case 10: return launch_m<PRO, EPI, BM, 10>(p, grid, lds, st);
    case 8: return launch_m<PRO, EPI, BM, 8>(p, grid, lds, st);
    case 5: return launch_m<PRO, EPI, BM, 5>(p, grid, lds, st);
    case 4: return launch_m<PRO, EPI, BM, 4>(p, grid, lds, st);
    case 1: return launch_m<PRO, EPI, BM, 1>(p, grid, lds, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

template <>
hipError_t launch_mfma_pair<EK_PRO, EK_EPI>(const GemvParams& p, int bm, int nb, dim3 grid, size_t lds,
                                            hipStream_t st) {
  switch (bm) {
    case 2: return launch_mn<EK_PRO, EK_EPI, 2>(p, nb, grid, lds, st);
    case 4: return launch_mn<EK_PRO, EK_EPI, 4>(p, nb, grid, lds, st);
    default: return launch_mn<EK_PRO, EK_EPI, 8>(p, nb, grid, lds, st);
  }
}

template <>
hipError_t launch_pair<EK_PRO, EK_EPI>(const GemvParams& p, int bm, int kpl, int rpw, dim3 grid, size_t lds,
                                       hipStream_t st) {
  return launch_b<EK_PRO, EK_EPI>(p, bm, kpl, rpw, grid, lds, st);
}

}  // namespace ekg
