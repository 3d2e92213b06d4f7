// MFMA operand helpers shared by the gfx950 GEMM kernels (v_mfma_f32_16x16x32_f16).
//
// Lane layout of v_mfma_f32_16x16x32_f16 (checked on the device against a CPU product): lane i
// holds A row i % 16 and B column i % 16, each at k = 8 * (i / 16) + [0, 8); the fp32 result D
// holds rows 4 * (i / 16) + [0, 4) of column i % 16.
#pragma once

#include "w4h_kernels.h"

namespace w4h {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kPadH = 8;  // halves of padding per LDS operand row (16 bytes: spreads banks)

DEV half8 as_half8(uint4 u) {
  half8 h;
  __builtin_memcpy(&h, &u, 16);
  return h;
}

// 8 int8 values (two dwords) to 8 exact f16 values.
DEV half8 i8x8_to_h8(uint2 u) {
  half8 h;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h[j] = (_Float16)(float)(int8_t)((u.x >> (8 * j)) & 0xff);
    h[4 + j] = (_Float16)(float)(int8_t)((u.y >> (8 * j)) & 0xff);
  }
  return h;
}

}  // namespace w4h
