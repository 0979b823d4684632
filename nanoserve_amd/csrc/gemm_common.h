// Device helpers shared by the GEMM translation units (gemm.hip: row-major weights; packed_gemm.hip:
// fragment-packed weights): vector types, bf16 packing, and the RMSNorm statistics and "norm on load" of
// normalised activations.
#pragma once

#include "ns_common.h"

namespace ns {

typedef __attribute__((ext_vector_type(8))) __bf16 g_bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float g_float4_t;
typedef __attribute__((ext_vector_type(4))) unsigned int g_u32x4_t;   // native vector: stays in registers

enum GemmEpi { EPI_STORE = 0, EPI_SILU = 1, EPI_RESNORM = 2, EPI_ROPE = 3 };

constexpr int G_MAX_M = 64;
constexpr int G_NORM_ROWS = NS_NORM_ROWS;   // row stride of a row-statistics buffer
constexpr int G_NORM_COLS = 16;   // columns per row-sum partial of the RMSNorm statistics

// Two fp32 -> packed bf16, round to nearest even, by the hardware conversion (v_cvt_pk_bf16_f32): the same
// bits as f32_to_bf16 for every non-NaN value, in one instruction instead of a dozen integer ones.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __attribute__((ext_vector_type(2))) __bf16 g_bf16x2_t;
  g_bf16x2_t r;
  r[0] = static_cast<__bf16>(lo);
  r[1] = static_cast<__bf16>(hi);
  return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ void store_bf16x8(bf16_t* p, const float (&v)[8]) {
  g_u32x4_t u;
  u[0] = pack_bf16x2(v[0], v[1]);
  u[1] = pack_bf16x2(v[2], v[3]);
  u[2] = pack_bf16x2(v[4], v[5]);
  u[3] = pack_bf16x2(v[6], v[7]);
  *reinterpret_cast<g_u32x4_t*>(p) = u;
}
__device__ __forceinline__ void load_bf16x8(const bf16_t* p, float (&v)[8]) {
  const g_u32x4_t u = *reinterpret_cast<const g_u32x4_t*>(p);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[2 * e] = __uint_as_float(u[e] << 16);
    v[2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u);
  }
}

// inv of rows 0 .. M-1 into s_inv (LDS), for a whole workgroup, in two steps, so that the loads go out
// ahead of the kernel's weight stream and waiting for them never waits for it (vector loads complete in
// issue order). Thread (row, g) = (tid / 4, tid % 4) of the first ceil(M / 16) waves adds the partials
// p = g, g + 4, g + 8, ... in increasing p, then the four combine as (g0 + g1) + (g2 + g3) -- the same
// operations in the same order as rms_norm_row_inv, so the bits agree. row_stats_issue loads the thread's
// first RS_PRE partials (all of them for K <= 2048) with clamped, branch-free addresses; row_stats_finish
// adds them (and, for longer rows, the rest) and writes s_inv; the caller synchronises before reading it.
constexpr int RS_PRE = 32;
__device__ __forceinline__ void row_stats_issue(const float* sumsq, int ptiles, int M, float (&v)[RS_PRE]) {
  const int tid = threadIdx.x, m = min(tid >> 2, M - 1), g = tid & 3;
#pragma unroll
  for (int e = 0; e < RS_PRE; ++e) v[e] = sumsq[int64_t(min(g + 4 * e, ptiles - 1)) * G_NORM_ROWS + m];
}
__device__ __forceinline__ void row_stats_finish(const float* sumsq, int ptiles, int M, int K, float eps,
                                                 const float (&v)[RS_PRE], float* s_inv) {
  const int tid = threadIdx.x, m = tid >> 2, g = tid & 3;
  float part = 0.f;
#pragma unroll
  for (int e = 0; e < RS_PRE; ++e)
    if (g + 4 * e < ptiles) part += v[e];
  for (int p = g + 4 * RS_PRE; p < ptiles; p += 4) part += sumsq[int64_t(p) * G_NORM_ROWS + min(m, M - 1)];
  part += __shfl_xor(part, 1, 64);
  part += __shfl_xor(part, 2, 64);
  if (m < M && g == 0) s_inv[m] = rsqrtf(part / float(K) + eps);
}

// 8 bf16 of r (one X fragment) -> 8 bf16 of h = round(w * round(r * inv))
__device__ __forceinline__ g_u32x4_t norm_fragment(g_u32x4_t r, g_u32x4_t w, float inv) {
  g_u32x4_t o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float r0 = __uint_as_float(r[e] << 16), r1 = __uint_as_float(r[e] & 0xffff0000u);
    const float w0 = __uint_as_float(w[e] << 16), w1 = __uint_as_float(w[e] & 0xffff0000u);
    const uint32_t hp = pack_bf16x2(r0 * inv, r1 * inv);   // round(r * inv), both halves
    o[e] = pack_bf16x2(w0 * __uint_as_float(hp << 16), w1 * __uint_as_float(hp & 0xffff0000u));
  }
  return o;
}

}  // namespace ns
