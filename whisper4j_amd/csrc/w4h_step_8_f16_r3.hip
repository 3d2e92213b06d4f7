// Step kernel instance: up to 8 rows, f16 weights, 3 register rounds of 16-byte chunks
// per lane for GEMVs over d.
#include "w4h_kernels.h"

namespace w4h {
hipError_t launch_step_8_f16_r3(const StepParams& p, int grid, size_t lds, hipStream_t st) {
  return launch_step_t<kMaxRows, 0, 3>(p, grid, lds, st);
}
}  // namespace w4h
