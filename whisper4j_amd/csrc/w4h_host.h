// Host-side helpers shared by the runtime translation units (not part of the public C ABI).
#pragma once

#include <stdint.h>

#include "../../include/w4h.h"

namespace w4h {
int fail(int code, const char* fmt, ...);
float half_to_float(uint16_t h);
uint16_t float_to_half(float f);
int session_rows(const w4h_session* s);
w4h_dims session_dims(const w4h_session* s);
}  // namespace w4h
