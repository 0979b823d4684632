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

// torch.argmax order: a beats b for a larger value, or NaN over a number, or the same value (or both NaN)
// and a smaller index.
__device__ __forceinline__ bool better(float av, int ai, float bv, int bi) {
  const bool an = av != av, bn = bv != bv;
  if (an || bn) return an && (!bn || ai < bi);
  return av > bv || (av == bv && ai < bi);
}
// The same order as one unsigned 64-bit key (so an atomic max picks the winner): high word the value's
// rank (every NaN highest, -0 equal to +0, then the IEEE order as unsigned bits), low word ~index.
__device__ __forceinline__ unsigned long long argmax_key(float v, int i) {
  uint32_t u = __float_as_uint(v == 0.f ? 0.f : v);
  u = v != v ? 0xffffffffu : ((u & 0x80000000u) ? ~u : (u | 0x80000000u));
  return (static_cast<unsigned long long>(u) << 32) | static_cast<uint32_t>(~uint32_t(i));
}

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

// Hand-off of data between workgroups of one launch without device-scope fences. On gfx950 an
// agent-scope release/acquire fence writes back / invalidates the whole L2 of the XCD, which costs
// tens of nanoseconds per workgroup, serialised. Instead the data itself moves through agent-scope
// atomic stores and loads, which are coherent across XCDs (they bypass the non-coherent L2), and
// ordering comes from waiting for those stores to complete before the counter update that
// publishes them (release side), and from the counter's returned value being consumed before the
// data loads issue (acquire side). This is the publication scheme rocPRIM's look-back scan uses on
// gfx942/gfx950.
__device__ __forceinline__ void publish_store(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish_store(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float publish_load(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t publish_load(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16-byte forms: two 8-byte agent-scope atomic accesses each, which the compiler sees, orders and waits
// for itself. (A written-out vector store or load would hide its register use from the compiler's hazard
// and wait bookkeeping: a store could read its data registers before a preceding accumulator move has
// written them, and a load's destination could be copied before the data has arrived.)
typedef __attribute__((ext_vector_type(4))) unsigned int pub_u32x4_t;
__device__ __forceinline__ void publish_store16(void* p, pub_u32x4_t v) {
  uint64_t* q = static_cast<uint64_t*>(p);
  __hip_atomic_store(q, uint64_t(v[0]) | (uint64_t(v[1]) << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(q + 1, uint64_t(v[2]) | (uint64_t(v[3]) << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ pub_u32x4_t publish_load16(const void* p) {
  uint64_t* q = static_cast<uint64_t*>(const_cast<void*>(p));
  const uint64_t lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return pub_u32x4_t{uint32_t(lo), uint32_t(lo >> 32), uint32_t(hi), uint32_t(hi >> 32)};
}
// Every vector memory operation this wave issued so far has completed (s_waitcnt vmcnt(0)); with the
// workgroup-scope fence the compiler keeps the preceding stores before it.
__device__ __forceinline__ void publish_complete() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt and lgkmcnt left at their maxima
}
// Counter update of a publication: returns the previous value (one lane per workgroup calls it).
__device__ __forceinline__ unsigned publish_count(unsigned* c) {
  return __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish_reset(unsigned* c) {
  __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// After a counter read that says every publisher is done: no later load may move above it.
__device__ __forceinline__ void acquire_published() {
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Split-K workspaces (decode and prefill attention, argmax) start with a fixed region of arrival counters,
// one 32-bit word per merged unit. Only the counter protocol (increment, reset by the last arriver) ever
// touches it, so every call leaves it zero and calls of different shapes can share one buffer; the
// partial results of any call start after it.
constexpr size_t WS_COUNTER_BYTES = size_t(NS_WS_COUNTER_BYTES);
constexpr int WS_MAX_COUNTERS = int(WS_COUNTER_BYTES / 4);
// Words between two arrival counters of one launch: a 128-byte line each when the region holds them so,
// since the atomics of many workgroups on one line queue behind each other at the memory side (measured:
// 0.25 us per decode-attention launch); packed otherwise.
constexpr int WS_COUNTER_LINE = 32;
static inline int ws_counter_stride(size_t n_counters, size_t capacity_words) {
  return n_counters * WS_COUNTER_LINE <= capacity_words ? WS_COUNTER_LINE : 1;
}
// The last WS_AM_FUSED_WORDS words of an argmax workspace's counter region belong to the LM head with the
// argmax fused (ns_gemm_argmax): its arrival counter (word WS_AM_FUSED_OFF) and one 8-byte key per row
// (from word WS_AM_FUSED_OFF + 2), which that launch leaves at zero like the counters; the split argmax
// kernel's per-row counters stay below WS_AM_FUSED_OFF.
constexpr int WS_AM_FUSED_WORDS = 256;
constexpr int WS_AM_FUSED_OFF = WS_MAX_COUNTERS - WS_AM_FUSED_WORDS;

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
