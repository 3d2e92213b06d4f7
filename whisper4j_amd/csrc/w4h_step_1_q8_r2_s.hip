// Step kernel instance for sampled runs (the token drawn inside the launch): one row, q8_0 weights, 2 register rounds.
#include "w4h_kernels.h"

namespace w4h {
hipError_t launch_step_1_q8_r2_s(const StepParams& p, int grid, size_t lds, hipStream_t st) {
  return launch_step_t<1, 1, 2, 1>(p, grid, lds, st);
}
}  // namespace w4h
