// Shared helpers for the RFSN HIP kernels (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <string>

#include "rfsn_abi.h"

namespace rfsn {

typedef _Float16 f16;

// ---- error reporting across the C ABI ---------------------------------------
void set_error(const std::string& msg);
int fail(int status, const std::string& msg);
int check_launch(const char* what);

#define RFSN_REQUIRE(cond, msg)                                   \
  do {                                                            \
    if (!(cond)) return ::rfsn::fail(RFSN_ERR_INVALID, (msg));    \
  } while (0)

// ---- device helpers ------------------------------------------------------------
__device__ __forceinline__ float h2f(uint16_t bits) {
  return (float)__builtin_bit_cast(f16, bits);
}
__device__ __forceinline__ uint16_t f2h(float v) {
  return __builtin_bit_cast(uint16_t, (f16)v);  // round to nearest even
}
// fp16(fl32(a) + fl32(b)) for fp16 bit patterns.
__device__ __forceinline__ uint16_t hadd_bits(uint16_t a, uint16_t b) {
  return f2h(h2f(a) + h2f(b));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

constexpr float kMaskFill = -1e30f;  // storage.py:16

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace rfsn
