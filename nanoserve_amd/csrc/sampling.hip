// Greedy token selection on gfx950: row-wise argmax of the logits (nanoserve/engine.py:239,
// `logits.argmax(-1)`). Semantics of torch.argmax: the index of the first maximal value, NaN counting
// as larger than every number (the first NaN wins).
//
// One workgroup per row, each thread scans a strided part of the row with 16-byte loads (8 bf16, eight
// loads in flight), keeps (value, index) with first-index tie breaking, then a wave64 shuffle reduction
// and a cross-wave step.
#include "ns_common.h"

namespace ns {

// a beats b: larger value, or NaN over a number, or same value (or both NaN) and smaller index
__device__ __forceinline__ bool better(float av, int ai, float bv, int bi) {
  const bool an = av != av, bn = bv != bv;
  if (an || bn) return an && (!bn || ai < bi);
  return av > bv || (av == bv && ai < bi);
}

template <typename T>
__device__ __forceinline__ float ldf(const T* p, int64_t i);
template <>
__device__ __forceinline__ float ldf<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float ldf<bf16_t>(const bf16_t* p, int64_t i) { return bf16_to_f32(p[i]); }

template <typename T>
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const T* __restrict__ x, int64_t ld, int n,
                                                           int64_t* __restrict__ out) {
  const int64_t row = blockIdx.x;
  const T* r = x + row * ld;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  constexpr int VEC = 16 / sizeof(T);
  const bool vec_ok = (reinterpret_cast<uintptr_t>(r) % 16) == 0;
  const int nv = vec_ok ? n / VEC : 0;
  // U vectors in flight per thread: a row is one workgroup's, so its bandwidth comes from memory-level
  // parallelism inside the workgroup, not from more workgroups. Indices still rise within each thread,
  // so first-index tie breaking is kept.
  constexpr int U = 8;
  const int stride = int(blockDim.x);
  for (int v0 = threadIdx.x; v0 < nv; v0 += U * stride) {
    uint4 u[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int v = v0 + k * stride;
      u[k] = v < nv ? reinterpret_cast<const uint4*>(r)[v] : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int v = v0 + k * stride;
      if (v < nv) {
        const T* e = reinterpret_cast<const T*>(&u[k]);
#pragma unroll
        for (int q = 0; q < VEC; ++q) {
          float f;
          if constexpr (sizeof(T) == 2) f = bf16_to_f32(reinterpret_cast<const bf16_t*>(e)[q]);
          else f = reinterpret_cast<const float*>(e)[q];
          const int i = v * VEC + q;
          if (better(f, i, bv, bi)) { bv = f; bi = i; }
        }
      }
    }
  }
  for (int i = nv * VEC + threadIdx.x; i < n; i += blockDim.x) {
    const float f = ldf<T>(r, i);
    if (better(f, i, bv, bi)) { bv = f; bi = i; }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  __shared__ float sv[16];
  __shared__ int si[16];
  const int wv = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wv] = bv;
    si[wv] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = sv[0];
    int i = si[0];
    for (int q = 1; q < int(blockDim.x) / 64; ++q)
      if (better(sv[q], si[q], v, i)) { v = sv[q]; i = si[q]; }
    out[row] = i == 0x7fffffff ? 0 : i;
  }
}

}  // namespace ns

using namespace ns;

extern "C" int ns_argmax_rows(const void* x, int64_t ld, int64_t rows, int n, int dtype, int64_t* out, void* stream) {
  NS_REQUIRE(dtype == NS_DTYPE_F32 || dtype == NS_DTYPE_BF16, "argmax_rows: dtype %d not supported", dtype);
  NS_REQUIRE(rows >= 0 && rows < (int64_t(1) << 31) && n >= 1 && ld >= n, "argmax_rows: rows=%lld n=%d ld=%lld",
             (long long)rows, n, (long long)ld);
  if (rows == 0) return NS_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (dtype == NS_DTYPE_BF16)
    hipLaunchKernelGGL(argmax_rows_kernel<bf16_t>, dim3(unsigned(rows)), dim3(1024), 0, s, static_cast<const bf16_t*>(x),
                       ld, n, out);
  else
    hipLaunchKernelGGL(argmax_rows_kernel<float>, dim3(unsigned(rows)), dim3(1024), 0, s, static_cast<const float*>(x), ld,
                       n, out);
  return check_launch("argmax_rows");
}
