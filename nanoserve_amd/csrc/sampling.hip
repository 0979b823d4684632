// Greedy token selection on gfx950: row-wise argmax of the logits (nanoserve/engine.py:239,
// `logits.argmax(-1)`). Semantics of torch.argmax: the index of the first maximal value, NaN counting
// as larger than every number (the first NaN wins).
//
// With a workspace, each row is split over several workgroups whose partial results merge in the same
// launch (argmax_split_kernel); without one, one workgroup per row: each thread scans a strided part of the
// row with 16-byte loads (8 bf16, eight loads in flight), keeps (value, index) with first-index tie
// breaking, then a wave64 shuffle reduction and a cross-wave step.
#include "ns_common.h"

namespace ns {

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

// Split rows: row r is scanned by `splits` workgroups of 256 threads, split k covering vectors
// [k nv / splits, (k + 1) nv / splits). Each publishes its (value, index) with agent-scope stores, waits
// for them and counts itself in on the row's counter; the last to arrive combines the splits (by the same
// order: larger value, NaN first, then the smaller index, so the result is the single-pass one), writes
// out[r] and resets the counter.
constexpr int AM_THREADS = 256;
constexpr int AM_MAX_SPLITS = 64;

template <typename T>
__global__ __launch_bounds__(AM_THREADS) void argmax_split_kernel(const T* __restrict__ x, int64_t ld, int n,
                                                                  int splits, int64_t* __restrict__ out,
                                                                  unsigned* __restrict__ cnt,
                                                                  uint32_t* __restrict__ part) {
  const int row = blockIdx.x / splits, k = blockIdx.x - (blockIdx.x / splits) * splits;
  const T* r = x + int64_t(row) * ld;
  constexpr int VEC = 16 / sizeof(T);
  const int nv = n / VEC;   // the host checks 16-byte alignment of every row
  const int v0 = int(int64_t(k) * nv / splits), v1 = int(int64_t(k + 1) * nv / splits);
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  constexpr int U = 8;
  for (int vb = v0 + threadIdx.x; vb < v1; vb += U * AM_THREADS) {
    uint4 u[U];
#pragma unroll
    for (int q = 0; q < U; ++q) {
      const int v = vb + q * AM_THREADS;
      u[q] = v < v1 ? reinterpret_cast<const uint4*>(r)[v] : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int q = 0; q < U; ++q) {
      const int v = vb + q * AM_THREADS;
      if (v < v1) {
        const T* e = reinterpret_cast<const T*>(&u[q]);
#pragma unroll
        for (int c = 0; c < VEC; ++c) {
          float f;
          if constexpr (sizeof(T) == 2) f = bf16_to_f32(reinterpret_cast<const bf16_t*>(e)[c]);
          else f = reinterpret_cast<const float*>(e)[c];
          const int i = v * VEC + c;
          if (better(f, i, bv, bi)) { bv = f; bi = i; }
        }
      }
    }
  }
  if (k == splits - 1)   // the scalar tail past the last whole vector
    for (int i = nv * VEC + threadIdx.x; i < n; i += AM_THREADS) {
      const float f = ldf<T>(r, i);
      if (better(f, i, bv, bi)) { bv = f; bi = i; }
    }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  __shared__ float sv[AM_THREADS / 64];
  __shared__ int si[AM_THREADS / 64];
  __shared__ unsigned s_last;
  const int wv = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wv] = bv;
    si[wv] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = sv[0];
    int i = si[0];
#pragma unroll
    for (int q = 1; q < AM_THREADS / 64; ++q)
      if (better(sv[q], si[q], v, i)) { v = sv[q]; i = si[q]; }
    uint32_t* my = part + (int64_t(row) * AM_MAX_SPLITS + k) * 2;
    publish_store(my, __float_as_uint(v));
    publish_store(my + 1, uint32_t(i));
    publish_complete();
    const unsigned prev = publish_count(cnt + row);
    const unsigned last = prev == unsigned(splits - 1);
    if (last) publish_reset(cnt + row);
    s_last = last;
  }
  __syncthreads();
  if (s_last == 0u) return;
  acquire_published();
  // the last split: one lane per split, then a shuffle reduction
  if (threadIdx.x < 64) {
    float v = -INFINITY;
    int i = 0x7fffffff;
    if (int(threadIdx.x) < splits) {
      const uint32_t* pp = part + (int64_t(row) * AM_MAX_SPLITS + threadIdx.x) * 2;
      v = __uint_as_float(publish_load(pp));
      i = int(publish_load(pp + 1));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(v, o, 64);
      const int oi = __shfl_xor(i, o, 64);
      if (better(ov, oi, v, i)) { v = ov; i = oi; }
    }
    if (threadIdx.x == 0) out[row] = i == 0x7fffffff ? 0 : i;
  }
}

static int argmax_splits(int64_t rows, int n) {
  // about 512 workgroups, at least 2048 elements each
  int s = int((512 + rows - 1) / rows);
  const int by_len = n / 2048;
  if (s > by_len) s = by_len;
  if (s > AM_MAX_SPLITS) s = AM_MAX_SPLITS;
  return s < 1 ? 1 : s;
}

}  // namespace ns

using namespace ns;

// Workspace: the fixed counter region (one arrival counter per row; shared safely by calls with any row
// count), then each row's per-split (value, index) partials.
extern "C" size_t ns_argmax_workspace_bytes(int64_t rows, int n) {
  if (rows <= 0 || n <= 0 || rows > WS_AM_FUSED_OFF) return 0;
  return WS_COUNTER_BYTES + size_t(rows) * AM_MAX_SPLITS * 8;
}

extern "C" int ns_argmax_rows(const void* x, int64_t ld, int64_t rows, int n, int dtype, int64_t* out, void* workspace,
                              size_t workspace_bytes, void* stream) {
  NS_REQUIRE(dtype == NS_DTYPE_F32 || dtype == NS_DTYPE_BF16, "argmax_rows: dtype %d not supported", dtype);
  NS_REQUIRE(rows >= 0 && rows < (int64_t(1) << 31) && n >= 1 && ld >= n, "argmax_rows: rows=%lld n=%d ld=%lld",
             (long long)rows, n, (long long)ld);
  if (rows == 0) return NS_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int esz = dtype == NS_DTYPE_BF16 ? 2 : 4;
  const bool aligned = (reinterpret_cast<uintptr_t>(x) % 16) == 0 && (ld * esz) % 16 == 0;
  const int splits = argmax_splits(rows, n);
  if (workspace != nullptr && aligned && splits > 1 && rows <= WS_AM_FUSED_OFF) {
    NS_REQUIRE(workspace_bytes >= ns_argmax_workspace_bytes(rows, n) && reinterpret_cast<uintptr_t>(workspace) % 256 == 0,
               "argmax_rows: a zero-initialised, 256-byte aligned workspace of %zu bytes is needed, got %zu",
               ns_argmax_workspace_bytes(rows, n), workspace_bytes);
    unsigned* cnt = static_cast<unsigned*>(workspace);
    uint32_t* part = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + WS_COUNTER_BYTES);
    const dim3 grid(unsigned(rows * splits));
    if (dtype == NS_DTYPE_BF16)
      hipLaunchKernelGGL(argmax_split_kernel<bf16_t>, grid, dim3(AM_THREADS), 0, s, static_cast<const bf16_t*>(x), ld,
                         n, splits, out, cnt, part);
    else
      hipLaunchKernelGGL(argmax_split_kernel<float>, grid, dim3(AM_THREADS), 0, s, static_cast<const float*>(x), ld, n,
                         splits, out, cnt, part);
    return check_launch("argmax_rows(split)");
  }
  if (dtype == NS_DTYPE_BF16)
    hipLaunchKernelGGL(argmax_rows_kernel<bf16_t>, dim3(unsigned(rows)), dim3(1024), 0, s, static_cast<const bf16_t*>(x),
                       ld, n, out);
  else
    hipLaunchKernelGGL(argmax_rows_kernel<float>, dim3(unsigned(rows)), dim3(1024), 0, s, static_cast<const float*>(x), ld,
                       n, out);
  return check_launch("argmax_rows");
}
