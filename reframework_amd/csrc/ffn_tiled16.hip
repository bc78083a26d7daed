// One instance of ffn_tiled16_kernel's launcher (the 256-row tiled grouped
// GEMM on v_mfma_f32_16x16x32, ffn_tiled.h), chosen at compile time:
// MOE355_TILED16_T is bf16 or f16 and MOE355_TILED16_GATE_UP true or false.
// The Makefile builds this file once per combination.
#include "ffn_tiled.h"

namespace moe355 {

template <typename T, bool kGateUp>
hipError_t launch_tiled16(const FfnArgs& a, hipStream_t s) {
  if (a.ragged)
    ffn_tiled16_kernel<T, kGateUp, true><<<dim3(a.grid), dim3(kThreads), 0, s>>>(a);
  else
    ffn_tiled16_kernel<T, kGateUp, false><<<dim3(a.grid), dim3(kThreads), 0, s>>>(a);
  return hipGetLastError();
}

template hipError_t launch_tiled16<MOE355_TILED16_T, MOE355_TILED16_GATE_UP>(const FfnArgs&, hipStream_t);

}  // namespace moe355
