// Shared helpers for the gfx950 kernels of libnanoserve_hip.so: bf16 bit conversions, wave64
// reductions, and the per-thread error slot behind ns_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/nanoserve_hip.h"

namespace ns {

typedef uint16_t bf16_t;  // raw bf16 storage

// bf16 -> fp32 is exact: the bf16 bits are the high half of the fp32 bits.
__device__ __forceinline__ float bf16_to_f32(bf16_t h) { return __uint_as_float(uint32_t(h) << 16); }

// fp32 -> bf16, round to nearest, ties to even, on the integer bits (the textbook method: add
// 0x7FFF plus the lowest kept bit, then truncate). NaN maps to the canonical quiet NaN. Integer
// arithmetic keeps the rounding point explicit: no contraction can merge it into a neighbour.
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return bf16_t(0x7fc0);
  u += 0x7fffu + ((u >> 16) & 1u);
  return bf16_t(u >> 16);
}

// Value of f rounded to bf16, kept in fp32.
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Sum / max over the 64 lanes of a wavefront (butterfly; every lane receives the result).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Host side: error slot and launch checking.
void set_error(const char* fmt, ...);
int check_launch(const char* what);

}  // namespace ns

#define NS_REQUIRE(cond, ...)          \
  do {                                 \
    if (!(cond)) {                     \
      ::ns::set_error(__VA_ARGS__);    \
      return NS_E_INVALID;             \
    }                                  \
  } while (0)
