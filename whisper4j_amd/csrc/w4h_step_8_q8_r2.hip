// Step kernel instance: up to 8 rows, q8_0 weights, 2 register rounds of 16-byte chunks
// per lane for GEMVs over d.
#include "w4h_kernels.h"

namespace w4h {
hipError_t launch_step_8_q8_r2(const StepParams& p, int grid, size_t lds, hipStream_t st) {
  return launch_step_t<kMaxRows, 1, 2>(p, grid, lds, st);
}
}  // namespace w4h
