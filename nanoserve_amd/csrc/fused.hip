// Token-wise fused kernels of the decode step for gfx950: RMSNorm (+ residual add), SiLU*mul, RoPE on the
// merged QKV projection with the paged KV write, and the step's embedding + RoPE tables.
//
// Every kernel rounds to the tensor dtype exactly where PyTorch's unfused ops round, so bf16
// outputs equal the unfused ops bit for bit apart from RMSNorm's fp32 sum order (<= 1 bf16 ulp).
// Semantics follow nanoserve/kernels/fused.py (rms_norm :26-59, silu_mul :63-83, rope_qkv
// :87-175); this file is built with -ffp-contract=off so no product is fused into an add.
#include "ns_common.h"

namespace ns {

// ------------------------------------------------------------------------------------------ RMSNorm
// One workgroup of 256 threads (4 waves) per row. Each thread holds VEC consecutive elements per
// pass (16-byte loads for bf16); rows up to 256 * VEC * NPASS elements stay in registers, so x is
// read from HBM once and written once.
template <typename T>
struct io;
template <>
struct io<float> {
  static __device__ __forceinline__ float ld(const float* p) { return *p; }
  static __device__ __forceinline__ void st(float* p, float v) { *p = v; }
  static __device__ __forceinline__ float rnd(float v) { return v; }
};
template <>
struct io<bf16_t> {
  static __device__ __forceinline__ float ld(const bf16_t* p) { return bf16_to_f32(*p); }
  static __device__ __forceinline__ void st(bf16_t* p, float v) { *p = f32_to_bf16(v); }
  static __device__ __forceinline__ float rnd(float v) { return round_bf16(v); }
};

constexpr int RMS_THREADS = 256;
constexpr int RMS_MAX_PER_THREAD = 16;  // n <= 4096 elements per row

template <typename T>
__global__ __launch_bounds__(RMS_THREADS) void rms_norm_kernel(const T* __restrict__ x, const T* __restrict__ res,
                                                               const T* __restrict__ w, T* __restrict__ out,
                                                               T* __restrict__ res_out, int n, float eps) {
  const int64_t row = blockIdx.x;
  const T* xr = x + row * n;
  float v[RMS_MAX_PER_THREAD];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < RMS_MAX_PER_THREAD; ++i) {
    const int c = i * RMS_THREADS + threadIdx.x;
    float a = 0.f;
    if (c < n) {
      a = io<T>::ld(xr + c);
      if (res != nullptr) {
        // residual + x, rounded to the dtype (PyTorch's `x + a`), kept for the next layer.
        a = io<T>::rnd(io<T>::ld(res + row * n + c) + a);
        io<T>::st(res_out + row * n + c, a);
      }
    }
    v[i] = a;
    ss += a * a;
  }
  __shared__ float part[RMS_THREADS / 64];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < RMS_THREADS / 64; ++i) tot += part[i];
  const float inv = rsqrtf(tot / float(n) + eps);
#pragma unroll
  for (int i = 0; i < RMS_MAX_PER_THREAD; ++i) {
    const int c = i * RMS_THREADS + threadIdx.x;
    if (c < n) {
      const float y = io<T>::rnd(v[i] * inv);  // HF casts back BEFORE the weight multiply
      io<T>::st(out + row * n + c, io<T>::ld(w + c) * y);
    }
  }
}

// bf16 rows with n % 8 == 0 and 16-byte aligned operands: one wave per row, 8 consecutive elements (16 bytes)
// per lane per pass, every pass's loads issued before any arithmetic. The sum of squares is the lane's
// elements in pass order, then a butterfly over the wave. Same roundings as rms_norm_kernel.
constexpr int RMSV_MAX_PASS = 8;   // n <= 8 * 512
typedef __attribute__((ext_vector_type(4))) unsigned int f_u32x4_t;

__device__ __forceinline__ void unpack8(const f_u32x4_t& u, float (&f)[8]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = __uint_as_float(u[e] << 16);
    f[2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u);
  }
}
__device__ __forceinline__ f_u32x4_t pack8(const float (&f)[8]) {
  f_u32x4_t u;
#pragma unroll
  for (int e = 0; e < 4; ++e) u[e] = uint32_t(f32_to_bf16(f[2 * e])) | (uint32_t(f32_to_bf16(f[2 * e + 1])) << 16);
  return u;
}

__global__ __launch_bounds__(256) void rms_norm_bf16_rows_kernel(const bf16_t* __restrict__ x,
                                                                 const bf16_t* __restrict__ res,
                                                                 const bf16_t* __restrict__ w, bf16_t* __restrict__ out,
                                                                 bf16_t* __restrict__ res_out, int64_t rows, int n,
                                                                 float eps) {
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;   // wave-uniform, and nothing below synchronises the workgroup
  const int lane = threadIdx.x & 63;
  const bf16_t* xr = x + row * n;
  f_u32x4_t xv[RMSV_MAX_PASS], rv[RMSV_MAX_PASS], wv[RMSV_MAX_PASS];
#pragma unroll
  for (int p = 0; p < RMSV_MAX_PASS; ++p) {
    const int c = p * 512 + lane * 8;
    if (c < n) {
      xv[p] = *reinterpret_cast<const f_u32x4_t*>(xr + c);
      if (res != nullptr) rv[p] = *reinterpret_cast<const f_u32x4_t*>(res + row * n + c);
      wv[p] = *reinterpret_cast<const f_u32x4_t*>(w + c);
    }
  }
  float v[RMSV_MAX_PASS][8];
  float ss = 0.f;
#pragma unroll
  for (int p = 0; p < RMSV_MAX_PASS; ++p) {
    const int c = p * 512 + lane * 8;
    if (c < n) {
      unpack8(xv[p], v[p]);
      if (res != nullptr) {
        float r[8];
        unpack8(rv[p], r);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[p][e] = round_bf16(r[e] + v[p][e]);   // residual + x, rounded
        *reinterpret_cast<f_u32x4_t*>(res_out + row * n + c) = pack8(v[p]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[p][e] * v[p][e];
    }
  }
  ss = wave_sum(ss);
  const float inv = rsqrtf(ss / float(n) + eps);
#pragma unroll
  for (int p = 0; p < RMSV_MAX_PASS; ++p) {
    const int c = p * 512 + lane * 8;
    if (c < n) {
      float wf[8], o[8];
      unpack8(wv[p], wf);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = wf[e] * round_bf16(v[p][e] * inv);   // cast back before the weight
      *reinterpret_cast<f_u32x4_t*>(out + row * n + c) = pack8(o);
    }
  }
}

// ------------------------------------------------------------------------------------------ SiLU*mul
// Elementwise over [rows, n] outputs; each thread produces 8 consecutive outputs when n % 8 == 0.
template <typename T>
__global__ __launch_bounds__(256) void silu_mul_kernel(const T* __restrict__ x, T* __restrict__ out, int64_t rows,
                                                       int n) {
  const int64_t total = rows * int64_t(n);
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / n;
    const int64_t c = i - r * n;
    const float g = io<T>::ld(x + r * 2 * n + c);
    const float u = io<T>::ld(x + r * 2 * n + n + c);
    const float s = io<T>::rnd(g / (1.0f + expf(-g)));  // F.silu: fp32 math, rounded to the dtype
    io<T>::st(out + i, s * u);
  }
}

// bf16 fast path: 8 outputs per thread with 16-byte loads and stores.
__global__ __launch_bounds__(256) void silu_mul_bf16x8_kernel(const uint4* __restrict__ x, uint4* __restrict__ out,
                                                              int64_t rows, int n8) {
  const int64_t total = rows * int64_t(n8);
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / n8;
    const int64_t c = i - r * n8;
    const uint4 gv = x[r * 2 * n8 + c];
    const uint4 uv = x[r * 2 * n8 + n8 + c];
    const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
    const uint32_t uw[4] = {uv.x, uv.y, uv.z, uv.w};
    uint32_t ow[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float o2[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float g = bf16_to_f32(bf16_t(gw[j] >> (16 * h)));
        const float u = bf16_to_f32(bf16_t(uw[j] >> (16 * h)));
        const float s = round_bf16(g / (1.0f + expf(-g)));
        o2[h] = s * u;
      }
      ow[j] = uint32_t(f32_to_bf16(o2[0])) | (uint32_t(f32_to_bf16(o2[1])) << 16);
    }
    out[i] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
  }
}

// ------------------------------------------------------------------------------------- RoPE + cache
// One workgroup per token. Work item = (head, d) with d < hd/2 for the rotated q and k heads (the
// pair d, d + hd/2 is produced together), then (head, d) < n_kv * hd for the value copy.
// rotate_half(x) = [-x_hi, x_lo], so with lo/hi halves of each head:
//   out_lo = x_lo*cos_lo - x_hi*sin_lo,   out_hi = x_hi*cos_hi + x_lo*sin_hi
// with a rounding after each product and after the sum (PyTorch's q*c + rotate_half(q)*s in bf16).
template <typename T>
__global__ __launch_bounds__(256) void rope_qkv_kernel(const T* __restrict__ qkv, const T* __restrict__ cosb,
                                                       const T* __restrict__ sinb, T* __restrict__ q,
                                                       T* __restrict__ k, T* __restrict__ v, T* __restrict__ kc,
                                                       T* __restrict__ vc, const int64_t* __restrict__ slots, int nh,
                                                       int nkv, int hd) {
  const int64_t t = blockIdx.x;
  const int half = hd >> 1;
  const int width = (nh + 2 * nkv) * hd;
  const T* row = qkv + t * width;
  const T* cr = cosb + t * hd;
  const T* sr = sinb + t * hd;
  const int64_t slot = kc != nullptr ? slots[t] : 0;
  const int n_rot = (nh + nkv) * half;
  for (int i = threadIdx.x; i < n_rot; i += blockDim.x) {
    const int head = i / half;
    const int d = i - head * half;
    const float xl = io<T>::ld(row + head * hd + d);
    const float xh = io<T>::ld(row + head * hd + half + d);
    const float cl = io<T>::ld(cr + d), ch = io<T>::ld(cr + half + d);
    const float sl = io<T>::ld(sr + d), sh = io<T>::ld(sr + half + d);
    const float lo = io<T>::rnd(io<T>::rnd(xl * cl) - io<T>::rnd(xh * sl));
    const float hi = io<T>::rnd(io<T>::rnd(xh * ch) + io<T>::rnd(xl * sh));
    if (head < nh) {
      T* dst = q + (t * nh + head) * hd;
      io<T>::st(dst + d, lo);
      io<T>::st(dst + half + d, hi);
    } else {
      const int kh = head - nh;
      T* dst = k + (t * nkv + kh) * hd;
      io<T>::st(dst + d, lo);
      io<T>::st(dst + half + d, hi);
      if (kc != nullptr) {
        T* cd = kc + (slot * nkv + kh) * hd;
        io<T>::st(cd + d, lo);
        io<T>::st(cd + half + d, hi);
      }
    }
  }
  const int n_v = nkv * hd;
  const T* vrow = row + (nh + nkv) * hd;
  for (int i = threadIdx.x; i < n_v; i += blockDim.x) {
    const T val = vrow[i];
    v[t * n_v + i] = val;
    if (vc != nullptr) vc[slot * n_v + i] = val;
  }
}

// bf16 with head_dim % 16 == 0 and 16-byte aligned operands: one workgroup per token, a thread's item is 8 dims
// of a rotated head's low half with their rotate-half partners (16-byte loads and stores), or 8 dims of a
// value head -- one pass for up to 256 items (the 1.5B and 3B shapes have 144 and 176). Same roundings as
// rope_qkv_kernel.
__global__ __launch_bounds__(256) void rope_qkv_bf16x8_kernel(const bf16_t* __restrict__ qkv,
                                                              const bf16_t* __restrict__ cosb,
                                                              const bf16_t* __restrict__ sinb, bf16_t* __restrict__ q,
                                                              bf16_t* __restrict__ k, bf16_t* __restrict__ v,
                                                              bf16_t* __restrict__ kc, bf16_t* __restrict__ vc,
                                                              const int64_t* __restrict__ slots, int nh, int nkv,
                                                              int hd) {
  const int64_t t = blockIdx.x;
  const int half = hd >> 1, per_head = half >> 3;
  const bf16_t* row = qkv + t * int64_t((nh + 2 * nkv) * hd);
  const bf16_t* cr = cosb + t * hd;
  const bf16_t* sr = sinb + t * hd;
  const int64_t slot = kc != nullptr ? slots[t] : 0;
  const int n_rot = (nh + nkv) * per_head, n_v = nkv * (hd >> 3);
  for (int i = threadIdx.x; i < n_rot + n_v; i += 256) {
    if (i < n_rot) {
      const int head = i / per_head, d0 = (i - head * per_head) * 8;
      float xl[8], xh[8], cl[8], ch[8], sl[8], sh[8], lo[8], hi[8];
      unpack8(*reinterpret_cast<const f_u32x4_t*>(row + head * hd + d0), xl);
      unpack8(*reinterpret_cast<const f_u32x4_t*>(row + head * hd + half + d0), xh);
      unpack8(*reinterpret_cast<const f_u32x4_t*>(cr + d0), cl);
      unpack8(*reinterpret_cast<const f_u32x4_t*>(cr + half + d0), ch);
      unpack8(*reinterpret_cast<const f_u32x4_t*>(sr + d0), sl);
      unpack8(*reinterpret_cast<const f_u32x4_t*>(sr + half + d0), sh);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        lo[e] = round_bf16(xl[e] * cl[e]) - round_bf16(xh[e] * sl[e]);
        hi[e] = round_bf16(xh[e] * ch[e]) + round_bf16(xl[e] * sh[e]);
      }
      const f_u32x4_t plo = pack8(lo), phi = pack8(hi);
      bf16_t* dst;
      bf16_t* cd = nullptr;
      if (head < nh) {
        dst = q + (t * nh + head) * hd;
      } else {
        const int kh = head - nh;
        dst = k + (t * nkv + kh) * hd;
        if (kc != nullptr) cd = kc + (slot * nkv + kh) * hd;
      }
      *reinterpret_cast<f_u32x4_t*>(dst + d0) = plo;
      *reinterpret_cast<f_u32x4_t*>(dst + half + d0) = phi;
      if (cd != nullptr) {
        *reinterpret_cast<f_u32x4_t*>(cd + d0) = plo;
        *reinterpret_cast<f_u32x4_t*>(cd + half + d0) = phi;
      }
    } else {
      const int c = (i - n_rot) * 8;   // element of the row's value heads
      const f_u32x4_t val = *reinterpret_cast<const f_u32x4_t*>(row + (nh + nkv) * hd + c);
      *reinterpret_cast<f_u32x4_t*>(v + t * (nkv * hd) + c) = val;
      if (vc != nullptr) *reinterpret_cast<f_u32x4_t*>(vc + slot * (nkv * hd) + c) = val;
    }
  }
}

// ------------------------------------------------------------------------- embedding + RoPE tables
// The first ops of a forward step in one launch (nanoserve/model.py:337-342 F.embedding and :212-217
// rope): x[i] = embed[token_ids[i]]; cos/sin[i] = cat(f, f).cos()/.sin() rounded to the dtype with
// f = float(positions[i]) * inv_freq (fp32). With row_sumsq given (decode batches, <= NS_NORM_ROWS rows) it also
// writes the statistics the first RMSNorm takes on load: row_sumsq[p][i] = sum over columns 16p .. 16p+15
// of x[i]^2. A token id outside [0, vocab) yields a zero row. One workgroup of 256 threads per token.
template <typename T>
__global__ __launch_bounds__(256) void embed_rope_kernel(const int64_t* __restrict__ ids, const int64_t* __restrict__ pos,
                                                         const T* __restrict__ embed, int64_t vocab, int hidden,
                                                         const float* __restrict__ inv_freq, int head_dim,
                                                         T* __restrict__ x, T* __restrict__ cosb, T* __restrict__ sinb,
                                                         float* __restrict__ row_sumsq) {
  const int64_t i = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t id = ids[i];
  const bool ok = id >= 0 && id < vocab;
  const T* src = embed + (ok ? id : 0) * int64_t(hidden);
  T* dst = x + i * int64_t(hidden);
  constexpr int VEC = 16 / sizeof(T);   // elements per 16-byte chunk
  // 16-column groups are VEC == 8 ? two threads : four threads; the group's sum is formed by shuffles
  constexpr int TPG = 16 / VEC;
  for (int c0 = 0; c0 < hidden; c0 += 256 * VEC) {
    const int c = c0 + tid * VEC;
    float ss = 0.f;
    if (c < hidden) {
      uint4 u = *reinterpret_cast<const uint4*>(src + c);
      if (!ok) u = make_uint4(0u, 0u, 0u, 0u);
      *reinterpret_cast<uint4*>(dst + c) = u;
      const T* e = reinterpret_cast<const T*>(&u);
#pragma unroll
      for (int q = 0; q < VEC; ++q) {
        const float f = io<T>::ld(e + q);
        ss += f * f;
      }
    }
#pragma unroll
    for (int o = 1; o < TPG; o <<= 1) ss += __shfl_xor(ss, o, 64);
    if (row_sumsq != nullptr && c < hidden && (tid % TPG) == 0) row_sumsq[int64_t(c / 16) * NS_NORM_ROWS + i] = ss;
  }
  const int half = head_dim >> 1;
  if (tid < half) {
    const float f = float(pos[i]) * inv_freq[tid];
    const float cv = cosf(f), sv = sinf(f);
    T* cr = cosb + i * int64_t(head_dim);
    T* sr = sinb + i * int64_t(head_dim);
    io<T>::st(cr + tid, cv);
    io<T>::st(cr + half + tid, cv);
    io<T>::st(sr + tid, sv);
    io<T>::st(sr + half + tid, sv);
  }
}

}  // namespace ns

using namespace ns;

extern "C" int ns_rms_norm(const void* x, const void* residual, const void* weight, void* out, void* res_out,
                           int64_t rows, int n, float eps, int dtype, void* stream) {
  NS_REQUIRE(dtype == NS_DTYPE_F32 || dtype == NS_DTYPE_BF16, "rms_norm: dtype %d not supported", dtype);
  NS_REQUIRE(n > 0 && n <= RMS_THREADS * RMS_MAX_PER_THREAD, "rms_norm: row length %d outside 1..%d", n,
             RMS_THREADS * RMS_MAX_PER_THREAD);
  NS_REQUIRE(residual == nullptr || res_out != nullptr, "rms_norm: residual given without res_out");
  NS_REQUIRE(rows >= 0 && rows < (int64_t(1) << 31), "rms_norm: rows %lld out of range", (long long)rows);
  if (rows == 0) return NS_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool vec = dtype == NS_DTYPE_BF16 && n % 8 == 0 && n <= RMSV_MAX_PASS * 512 &&
                   ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(residual) |
                     reinterpret_cast<uintptr_t>(weight) | reinterpret_cast<uintptr_t>(out) |
                     reinterpret_cast<uintptr_t>(res_out)) % 16) == 0;
  if (vec)
    hipLaunchKernelGGL(rms_norm_bf16_rows_kernel, dim3(unsigned((rows + 3) / 4)), dim3(256), 0, s,
                       static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(residual),
                       static_cast<const bf16_t*>(weight), static_cast<bf16_t*>(out), static_cast<bf16_t*>(res_out),
                       rows, n, eps);
  else if (dtype == NS_DTYPE_BF16)
    hipLaunchKernelGGL(rms_norm_kernel<bf16_t>, dim3(unsigned(rows)), dim3(RMS_THREADS), 0, s,
                       static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(residual),
                       static_cast<const bf16_t*>(weight), static_cast<bf16_t*>(out), static_cast<bf16_t*>(res_out),
                       n, eps);
  else
    hipLaunchKernelGGL(rms_norm_kernel<float>, dim3(unsigned(rows)), dim3(RMS_THREADS), 0, s,
                       static_cast<const float*>(x), static_cast<const float*>(residual),
                       static_cast<const float*>(weight), static_cast<float*>(out), static_cast<float*>(res_out), n,
                       eps);
  return check_launch("rms_norm");
}

extern "C" int ns_silu_mul(const void* x, void* out, int64_t rows, int n, int dtype, void* stream) {
  NS_REQUIRE(dtype == NS_DTYPE_F32 || dtype == NS_DTYPE_BF16, "silu_mul: dtype %d not supported", dtype);
  NS_REQUIRE(n > 0 && rows >= 0, "silu_mul: bad shape rows=%lld n=%d", (long long)rows, n);
  if (rows == 0) return NS_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool vec = dtype == NS_DTYPE_BF16 && n % 8 == 0 && (reinterpret_cast<uintptr_t>(x) % 16) == 0 &&
                   (reinterpret_cast<uintptr_t>(out) % 16) == 0;
  const int64_t items = vec ? rows * (n / 8) : rows * int64_t(n);
  int64_t blocks = (items + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (vec)
    hipLaunchKernelGGL(silu_mul_bf16x8_kernel, dim3(unsigned(blocks)), dim3(256), 0, s,
                       static_cast<const uint4*>(x), static_cast<uint4*>(out), rows, n / 8);
  else if (dtype == NS_DTYPE_BF16)
    hipLaunchKernelGGL(silu_mul_kernel<bf16_t>, dim3(unsigned(blocks)), dim3(256), 0, s,
                       static_cast<const bf16_t*>(x), static_cast<bf16_t*>(out), rows, n);
  else
    hipLaunchKernelGGL(silu_mul_kernel<float>, dim3(unsigned(blocks)), dim3(256), 0, s,
                       static_cast<const float*>(x), static_cast<float*>(out), rows, n);
  return check_launch("silu_mul");
}

extern "C" int ns_rope_qkv(const void* qkv, const void* cos, const void* sin, void* q, void* k, void* v,
                           void* k_cache, void* v_cache, const int64_t* slots, int64_t n_tok, int n_heads,
                           int n_kv_heads, int head_dim, int dtype, void* stream) {
  NS_REQUIRE(dtype == NS_DTYPE_F32 || dtype == NS_DTYPE_BF16, "rope_qkv: dtype %d not supported", dtype);
  NS_REQUIRE(n_heads > 0 && n_kv_heads > 0 && head_dim > 0 && head_dim % 2 == 0,
             "rope_qkv: bad heads nh=%d nkv=%d hd=%d", n_heads, n_kv_heads, head_dim);
  NS_REQUIRE((k_cache == nullptr) == (v_cache == nullptr), "rope_qkv: give both caches or neither");
  NS_REQUIRE(k_cache == nullptr || slots != nullptr, "rope_qkv: cache write needs slots");
  NS_REQUIRE(n_tok >= 0 && n_tok < (int64_t(1) << 31), "rope_qkv: n_tok %lld out of range", (long long)n_tok);
  if (n_tok == 0) return NS_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool vec = dtype == NS_DTYPE_BF16 && head_dim % 16 == 0 &&
                   ((reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(cos) |
                     reinterpret_cast<uintptr_t>(sin) | reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                     reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(k_cache) |
                     reinterpret_cast<uintptr_t>(v_cache)) % 16) == 0;
  if (vec)
    hipLaunchKernelGGL(rope_qkv_bf16x8_kernel, dim3(unsigned(n_tok)), dim3(256), 0, s,
                       static_cast<const bf16_t*>(qkv), static_cast<const bf16_t*>(cos),
                       static_cast<const bf16_t*>(sin), static_cast<bf16_t*>(q), static_cast<bf16_t*>(k),
                       static_cast<bf16_t*>(v), static_cast<bf16_t*>(k_cache), static_cast<bf16_t*>(v_cache), slots,
                       n_heads, n_kv_heads, head_dim);
  else if (dtype == NS_DTYPE_BF16)
    hipLaunchKernelGGL(rope_qkv_kernel<bf16_t>, dim3(unsigned(n_tok)), dim3(256), 0, s,
                       static_cast<const bf16_t*>(qkv), static_cast<const bf16_t*>(cos),
                       static_cast<const bf16_t*>(sin), static_cast<bf16_t*>(q), static_cast<bf16_t*>(k),
                       static_cast<bf16_t*>(v), static_cast<bf16_t*>(k_cache), static_cast<bf16_t*>(v_cache), slots,
                       n_heads, n_kv_heads, head_dim);
  else
    hipLaunchKernelGGL(rope_qkv_kernel<float>, dim3(unsigned(n_tok)), dim3(256), 0, s,
                       static_cast<const float*>(qkv), static_cast<const float*>(cos), static_cast<const float*>(sin),
                       static_cast<float*>(q), static_cast<float*>(k), static_cast<float*>(v),
                       static_cast<float*>(k_cache), static_cast<float*>(v_cache), slots, n_heads, n_kv_heads,
                       head_dim);
  return check_launch("rope_qkv");
}

extern "C" int ns_embed_rope(const int64_t* token_ids, const int64_t* positions, int64_t n_tokens, const void* embed,
                             int64_t vocab, int hidden, const float* inv_freq, int head_dim, void* x_out, void* cos_out,
                             void* sin_out, float* row_sumsq, int dtype, void* stream) {
  NS_REQUIRE(dtype == NS_DTYPE_F32 || dtype == NS_DTYPE_BF16, "embed_rope: dtype %d not supported", dtype);
  const int vec = dtype == NS_DTYPE_BF16 ? 8 : 4;
  NS_REQUIRE(hidden > 0 && hidden % 16 == 0, "embed_rope: hidden %d must be a positive multiple of 16", hidden);
  NS_REQUIRE(head_dim > 0 && head_dim % 2 == 0 && head_dim <= 512, "embed_rope: head_dim %d (even, <= 512)", head_dim);
  NS_REQUIRE(n_tokens >= 0 && n_tokens < (int64_t(1) << 31), "embed_rope: n_tokens %lld", (long long)n_tokens);
  NS_REQUIRE(row_sumsq == nullptr || n_tokens <= NS_NORM_ROWS, "embed_rope: row statistics need <= %d tokens, got %lld", NS_NORM_ROWS,
             (long long)n_tokens);
  NS_REQUIRE((reinterpret_cast<uintptr_t>(embed) | reinterpret_cast<uintptr_t>(x_out)) % 16 == 0,
             "embed_rope: embed and x_out must be 16-byte aligned");
  (void)vec;
  if (n_tokens == 0) return NS_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (dtype == NS_DTYPE_BF16)
    hipLaunchKernelGGL(embed_rope_kernel<bf16_t>, dim3(unsigned(n_tokens)), dim3(256), 0, s, token_ids, positions,
                       static_cast<const bf16_t*>(embed), vocab, hidden, inv_freq, head_dim, static_cast<bf16_t*>(x_out),
                       static_cast<bf16_t*>(cos_out), static_cast<bf16_t*>(sin_out), row_sumsq);
  else
    hipLaunchKernelGGL(embed_rope_kernel<float>, dim3(unsigned(n_tokens)), dim3(256), 0, s, token_ids, positions,
                       static_cast<const float*>(embed), vocab, hidden, inv_freq, head_dim, static_cast<float*>(x_out),
                       static_cast<float*>(cos_out), static_cast<float*>(sin_out), row_sumsq);
  return check_launch("embed_rope");
}

// ------------------------------------------------------------------------------------------ row gather
// dst[i] = src[rows[i]] for rows of row_bytes bytes (16-byte pieces), the rows the LM head scores
// (nanoserve/model.py:353-356: x[:, logits, :] or each sequence's last row). A row index outside [0, n_src)
// yields a zero row. One workgroup of 64 threads per output row.
namespace ns {
__global__ __launch_bounds__(64) void gather_rows_kernel(const unsigned char* __restrict__ src, int64_t src_stride,
                                                         int64_t n_src, const int64_t* __restrict__ rows,
                                                         int64_t row_bytes, unsigned char* __restrict__ dst,
                                                         int64_t dst_stride) {
  const int64_t i = blockIdx.x, r = rows[i];
  const bool ok = r >= 0 && r < n_src;
  const f_u32x4_t* s = reinterpret_cast<const f_u32x4_t*>(src + (ok ? r : 0) * src_stride);
  f_u32x4_t* d = reinterpret_cast<f_u32x4_t*>(dst + i * dst_stride);
  for (int64_t c = threadIdx.x; c < row_bytes / 16; c += 64) d[c] = ok ? s[c] : f_u32x4_t{0u, 0u, 0u, 0u};
}
}  // namespace ns

extern "C" int ns_gather_rows(const void* src, int64_t src_stride_bytes, int64_t n_src, const int64_t* rows,
                              int64_t n_rows, int64_t row_bytes, void* dst, int64_t dst_stride_bytes, void* stream) {
  NS_REQUIRE(n_rows >= 0 && n_rows < (int64_t(1) << 31), "gather_rows: n_rows %lld out of range", (long long)n_rows);
  NS_REQUIRE(row_bytes > 0 && row_bytes % 16 == 0 && src_stride_bytes % 16 == 0 && dst_stride_bytes % 16 == 0,
             "gather_rows: row_bytes %lld and strides must be positive multiples of 16", (long long)row_bytes);
  NS_REQUIRE(src_stride_bytes >= row_bytes && dst_stride_bytes >= row_bytes, "gather_rows: strides below row_bytes");
  NS_REQUIRE(src != nullptr && dst != nullptr && rows != nullptr && n_src >= 0, "gather_rows: null operand");
  NS_REQUIRE((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) % 16 == 0,
             "gather_rows: src and dst must be 16-byte aligned");
  if (n_rows == 0) return NS_OK;
  hipLaunchKernelGGL(ns::gather_rows_kernel, dim3(unsigned(n_rows)), dim3(64), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<const unsigned char*>(src), src_stride_bytes, n_src, rows, row_bytes,
                     static_cast<unsigned char*>(dst), dst_stride_bytes);
  return check_launch("gather_rows");
}
