// Shared helpers of the gfx950 Veda kernels: error reporting, bf16 bit
// handling and the MFMA operand types.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/veda_hip.h"

namespace veda {

constexpr int kTile = 128;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Thread-local message of the last failure, read by veda_last_error().
void set_error(const char* fmt, ...);

// Returns VEDA_ELAUNCH (with a message) if the last launch failed.
int check_launch(const char* what);

#define VEDA_REQUIRE(cond, ...)          \
  do {                                   \
    if (!(cond)) {                       \
      ::veda::set_error(__VA_ARGS__);    \
      return VEDA_EINVAL;                \
    }                                    \
  } while (0)

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits (NaN kept quiet).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Two fp32 -> packed bf16x2 (low half = a), round to nearest even.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v = __builtin_convertvector(f32x2_t{a, b}, bf16x2_t);
  return __builtin_bit_cast(uint32_t, v);
}

}  // namespace veda
