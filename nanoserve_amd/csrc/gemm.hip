// Skinny GEMMs of the decode step on gfx950: Y[M, N] = X[M, K] . W[N, K]^T with M <= 64 (the decode
// batch), bf16 in, fp32 accumulate. At M = 32 each weight byte feeds 32 multiply-adds, so the product is
// bound by streaming W once from HBM; the kernels are built to keep that stream full and to fold the
// token-wise ops around each projection into its epilogue.
//
// Main kernel (one workgroup = 4 waves = one 64-column tile x one K slice):
//   * MFMA 16x16x32 bf16: B operand = 16 weight rows x 8 consecutive k per lane (a 16-byte load straight
//     from W), A operand = 16 activation rows x 8 k (16-byte load from X, which stays in L2). A wave owns
//     all 64 columns of the tile (4 n-tiles), so every 16-byte X load feeds 4 MFMAs and weight bytes are
//     2x the activation bytes per k-step at M = 32.
//   * each wave takes a contiguous quarter of the tile's k-steps and issues a batch of U k-steps of loads
//     before its MFMAs; the waves' partial tiles are summed through LDS in a fixed order (deterministic).
//   * small N: the K range is split over KSPLIT workgroups (deterministic: partials go to a workspace and
//     an epilogue kernel sums them in order). The host picks KSPLIT so that ~256 workgroups run.
// Modes:
//   PLAIN    y = round(acc + bias)                                   (LM head, generic)
//   PARTIAL  ws[s] = acc (fp32)                                      (split-K, fused epilogues below)
//   SILU     paired gate/up tiles: 32 output columns = gate rows t*32.., up rows N/2 + t*32..;
//            out = round(round(silu(round(g))) * round(u))            (merged gate/up + SiLU*mul)
// Epilogue kernels (sum partials in order, then):
//   bias                 y = round(sum + bias)
//   residual + RMSNorm   o = round(sum); r = round(res + o) -> res_out; h = round(w * round(r * rsqrt(mean r^2 + eps)))
//   bias + RoPE + KV     qkv = round(sum + bias), then the rope_qkv contract (fused.hip) incl. the cache write
// Rounding points are PyTorch's for F.linear (+bias), x + y, rms_norm and silu(g) * u in bf16, so the
// fused step equals the unfused ops up to the fp32 summation order of the products.
#include <cstdlib>
#include <type_traits>

#include "ns_common.h"

namespace ns {

typedef __attribute__((ext_vector_type(8))) __bf16 g_bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float g_float4_t;
typedef __attribute__((ext_vector_type(4))) unsigned int g_u32x4_t;   // native vector: stays in registers

enum GemmMode { GEMM_PLAIN = 0, GEMM_PARTIAL = 1, GEMM_SILU = 2 };

constexpr int G_WAVES = 4;
constexpr int G_TN = 4;          // 16-row n-tiles per workgroup tile: 64 weight rows
constexpr int G_KC = 256;        // k per chunk: 512 bytes of each weight row
constexpr int G_SC = 3;          // chunks whose weight loads are in flight together (a super chunk)
constexpr int G_PAIR = 1040;     // LDS bytes of one row pair (rows p and p+8 of an n-tile) + 16 B pad
constexpr int G_NTB = 8 * G_PAIR;  // LDS bytes of one n-tile (16 rows) of a chunk
constexpr int G_STAGE = G_TN * G_NTB;

// Weight row of n-tile j, row r (0..15) of the tile (clamped; rows past the matrix are dropped later).
template <int MODE>
__device__ __forceinline__ int tile_row(int tile, int j, int r, int N) {
  if constexpr (MODE == GEMM_SILU) {
    const int half = N >> 1;
    const int row = (j < 2 ? 0 : half) + tile * 32 + 16 * (j & 1) + r;
    return min(row, (j < 2 ? half : N) - 1);
  } else {
    return min(tile * 64 + 16 * j + r, N - 1);
  }
}

// Main kernel. Workgroup = 4 waves = one 64-row weight tile x one K slice (chunks [c0, c1) of 256 k).
// Weight path: HBM -> registers -> LDS -> MFMA B fragments. Wave j loads n-tile j: instruction p (0..7)
// reads 512 contiguous bytes of row p (lanes 0-31) and of row p+8 (lanes 32-63) of the chunk, so every
// load instruction covers two long row segments; the LDS pitch of 1040 bytes per row pair makes both the
// stores and the 16-lane fragment reads bank-conflict free. Activation path: X fragments straight from L2.
// The 4 waves split each chunk's 8 k-steps (2 each) and reduce their partial tiles through LDS.
template <int TM, int MODE>
__global__ __launch_bounds__(G_WAVES * 64) void skinny_gemm_kernel(const bf16_t* __restrict__ x, const bf16_t* __restrict__ w,
                                                                   const bf16_t* __restrict__ bias, bf16_t* __restrict__ y,
                                                                   float* __restrict__ ws, int M, int N, int K, int ksplit) {
  constexpr int RED_BYTES = G_WAVES * TM * G_TN * 4 * 64 * 4;
  constexpr int LDS_BYTES = RED_BYTES > G_STAGE ? RED_BYTES : G_STAGE;
  __shared__ __align__(16) unsigned char lds[LDS_BYTES];
  const int tile = blockIdx.x, s = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int c16 = lane & 15, r4 = lane >> 4;
  const int nchunks = (K + G_KC - 1) / G_KC;
  const int c0 = int((int64_t(nchunks) * s) / ksplit), c1 = int((int64_t(nchunks) * (s + 1)) / ksplit);

  // this lane's weight rows: n-tile wv, rows p (lanes 0-31) / p + 8 (lanes 32-63), p = 0..7
  const int half_sel = lane >> 5, col16 = lane & 31;
  const bf16_t* wbase[8];
#pragma unroll
  for (int p = 0; p < 8; ++p)
    wbase[p] = w + int64_t(tile_row<MODE>(tile, wv, p + 8 * half_sel, N)) * K + 8 * col16;
  const int st_off = wv * G_NTB + half_sel * 512 + col16 * 16;       // + p * G_PAIR
  const int fr_off = (c16 & 7) * G_PAIR + (c16 >> 3) * 512 + r4 * 16;  // + j * G_NTB + kstep * 64
  const bf16_t* xrow[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) xrow[i] = x + int64_t(min(16 * i + c16, M - 1)) * K + 8 * r4;

  g_float4_t acc[TM][G_TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < G_TN; ++j) acc[i][j] = g_float4_t{0.f, 0.f, 0.f, 0.f};

  for (int sc = c0; sc < c1; sc += G_SC) {
    // issue every weight load of up to G_SC chunks, and this wave's activation fragments (k-steps 2wv,
    // 2wv+1 of each chunk); k beyond K reads a clamped in-bounds address and is masked below
    g_u32x4_t wr[G_SC][8], xf[G_SC][2][TM];
#pragma unroll
    for (int q = 0; q < G_SC; ++q) {
      const int kc = min(sc + q, c1 - 1) * G_KC;
#pragma unroll
      for (int p = 0; p < 8; ++p) wr[q][p] = *reinterpret_cast<const g_u32x4_t*>(wbase[p] + min(kc, K - 8 * col16 - 8));
    }
#pragma unroll
    for (int q = 0; q < G_SC; ++q) {
      const int kc = min(sc + q, c1 - 1) * G_KC;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < TM; ++i)
          xf[q][t][i] = *reinterpret_cast<const g_u32x4_t*>(xrow[i] + min(kc + 32 * (2 * wv + t), K - 32));
    }
    __builtin_amdgcn_sched_barrier(0);
    // one chunk at a time through the LDS stage; q is a compile-time constant so wr/xf stay in registers
    auto chunk = [&](auto qc) {
      constexpr int q = decltype(qc)::value;
      if (sc + q >= c1) return;   // uniform
      const int kc = (sc + q) * G_KC;
      __syncthreads();   // the stage is free (previous chunk consumed)
#pragma unroll
      for (int p = 0; p < 8; ++p) *reinterpret_cast<g_u32x4_t*>(lds + st_off + p * G_PAIR) = wr[q][p];
      __syncthreads();
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int ks = 2 * wv + t;
        if (kc + 32 * ks < K) {   // uniform
          g_bf16x8_t bfr[G_TN];
#pragma unroll
          for (int j = 0; j < G_TN; ++j)
            bfr[j] = __builtin_bit_cast(g_bf16x8_t, *reinterpret_cast<const g_u32x4_t*>(lds + j * G_NTB + ks * 64 + fr_off));
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < G_TN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(g_bf16x8_t, xf[q][t][i]), bfr[j],
                                                                  acc[i][j], 0, 0, 0);
        }
      }
    };
    static_assert(G_SC == 3, "chunk() is expanded for three chunks");
    chunk(std::integral_constant<int, 0>{});
    chunk(std::integral_constant<int, 1>{});
    chunk(std::integral_constant<int, 2>{});
  }

  // sum the 4 waves' partial tiles through LDS (fixed order); element e = ((i*4 + j)*4 + r)*64 + lane
  __syncthreads();
  float* sm = reinterpret_cast<float*>(lds);
  constexpr int PER_WAVE = TM * G_TN * 4 * 64;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < G_TN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) sm[wv * PER_WAVE + ((i * G_TN + j) * 4 + r) * 64 + lane] = acc[i][j][r];
  __syncthreads();

  if constexpr (MODE == GEMM_SILU) {
    const int half = N >> 1;
    for (int e = tid; e < TM * 2 * 4 * 64; e += G_WAVES * 64) {
      const int l = e & 63, r = (e >> 6) & 3, j = (e >> 8) & 1, i = e >> 9;
      const int eg = ((i * G_TN + j) * 4 + r) * 64 + l, eu = ((i * G_TN + j + 2) * 4 + r) * 64 + l;
      float g = 0.f, u = 0.f;
#pragma unroll
      for (int qw = 0; qw < G_WAVES; ++qw) {
        g += sm[qw * PER_WAVE + eg];
        u += sm[qw * PER_WAVE + eu];
      }
      const int m = 16 * i + 4 * (l >> 4) + r, n = tile * 32 + 16 * j + (l & 15);
      if (m < M && n < half) {
        const float gb = round_bf16(g), ub = round_bf16(u);
        const float sv = round_bf16(gb / (1.0f + expf(-gb)));
        y[int64_t(m) * half + n] = f32_to_bf16(sv * ub);
      }
    }
  } else {
    for (int e = tid; e < PER_WAVE; e += G_WAVES * 64) {
      const int l = e & 63, r = (e >> 6) & 3, j = (e >> 8) & 3, i = e >> 10;
      float v = 0.f;
#pragma unroll
      for (int qw = 0; qw < G_WAVES; ++qw) v += sm[qw * PER_WAVE + e];
      const int m = 16 * i + 4 * (l >> 4) + r, n = tile * 64 + 16 * j + (l & 15);
      if (m < M && n < N) {
        if constexpr (MODE == GEMM_PARTIAL) {
          ws[(int64_t(s) * M + m) * N + n] = v;
        } else {
          if (bias != nullptr) v += bf16_to_f32(bias[n]);
          y[int64_t(m) * N + n] = f32_to_bf16(v);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------- split-K epilogues
// Partials ws[s][m][n] (fp32) are summed in order s = 0, 1, ... Every thread owns one group of 4 columns of
// a row and loads its KMAX partial float4s at once (steps past ksplit read a valid slice and are weighted
// 0), so an epilogue costs one memory latency.
constexpr int KMAX = 16;   // largest K split the host picks

__device__ __forceinline__ float4 sum_partials(const float* __restrict__ ws, int64_t total, int64_t off, int ksplit) {
  float4 p[KMAX];
#pragma unroll
  for (int s = 0; s < KMAX; ++s) p[s] = *reinterpret_cast<const float4*>(ws + min(s, ksplit - 1) * total + off);
  float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int s = 0; s < KMAX; ++s) {
    if (s < ksplit) {
      a.x += p[s].x;
      a.y += p[s].y;
      a.z += p[s].z;
      a.w += p[s].w;
    }
  }
  return a;
}

// grid (ceil(N/4 / 256), M): y = round(sum + bias)
__global__ __launch_bounds__(256) void splitk_bias_kernel(const float* __restrict__ ws, const bf16_t* __restrict__ bias,
                                                          bf16_t* __restrict__ y, int M, int N, int ksplit) {
  const int m = blockIdx.y, c4 = blockIdx.x * 256 + threadIdx.x;
  if (4 * c4 >= N) return;
  const int64_t total = int64_t(M) * N, off = int64_t(m) * N + 4 * c4;
  const float4 a = sum_partials(ws, total, off, ksplit);
  const float v[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float b = bias != nullptr ? bf16_to_f32(bias[4 * c4 + e]) : 0.f;
    y[off + e] = f32_to_bf16(v[e] + b);
  }
}

constexpr int EPI_THREADS = 1024;   // one workgroup per row, one thread per 4 columns: rows up to 4096

// One workgroup of ceil(N/4) threads (rounded up to a wave) per row: o = round(sum); r = round(res + o)
// -> res_out; with a norm weight, h = rms_norm(r) (fp32 statistics, the rms_norm kernel's rounding).
__global__ __launch_bounds__(EPI_THREADS) void splitk_residual_rmsnorm_kernel(
    const float* __restrict__ ws, const bf16_t* __restrict__ res, bf16_t* __restrict__ res_out,
    const bf16_t* __restrict__ nw, bf16_t* __restrict__ h, int M, int N, int ksplit, float eps) {
  const int m = blockIdx.x, c4 = threadIdx.x;
  const bool live = 4 * c4 < N;
  const int64_t total = int64_t(M) * N, off = int64_t(m) * N + 4 * (live ? c4 : 0);
  const float4 a = sum_partials(ws, total, off, ksplit);
  const float o[4] = {a.x, a.y, a.z, a.w};
  float r[4];
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    r[e] = live ? round_bf16(bf16_to_f32(res[off + e]) + round_bf16(o[e])) : 0.f;
    if (live) res_out[off + e] = f32_to_bf16(r[e]);
    ss += r[e] * r[e];
  }
  if (nw == nullptr) return;
  __shared__ float part[EPI_THREADS / 64];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
  for (int i = 0; i < int(blockDim.x) / 64; ++i) tot += part[i];
  const float inv = rsqrtf(tot / float(N) + eps);
  if (live)
#pragma unroll
    for (int e = 0; e < 4; ++e) h[off + e] = f32_to_bf16(bf16_to_f32(nw[4 * c4 + e]) * round_bf16(r[e] * inv));
}

// One workgroup per token: qkv row = round(sum + bias) staged in LDS, then RoPE + KV write exactly as
// the rope_qkv kernel (out_lo = r(r(xl cl) - r(xh sl)), out_hi = r(r(xh ch) + r(xl sh)), v copied).
constexpr int ROPE_MAX_WIDTH = 4096;
__global__ __launch_bounds__(ROPE_MAX_WIDTH / 4) void splitk_bias_rope_kernel(
    const float* __restrict__ ws, const bf16_t* __restrict__ bias, const bf16_t* __restrict__ cosb,
    const bf16_t* __restrict__ sinb, bf16_t* __restrict__ q, bf16_t* __restrict__ k, bf16_t* __restrict__ v,
    bf16_t* __restrict__ kc, bf16_t* __restrict__ vc, const int64_t* __restrict__ slots, int M, int nh, int nkv,
    int hd, int ksplit) {
  const int t = blockIdx.x;
  const int width = (nh + 2 * nkv) * hd, half = hd >> 1;
  const int64_t total = int64_t(M) * width;
  __shared__ float row[ROPE_MAX_WIDTH];
  {
    const int c4 = threadIdx.x;
    if (4 * c4 < width) {
      const float4 a = sum_partials(ws, total, int64_t(t) * width + 4 * c4, ksplit);
      const float vv[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        row[4 * c4 + e] = round_bf16(vv[e] + (bias != nullptr ? bf16_to_f32(bias[4 * c4 + e]) : 0.f));
    }
  }
  __syncthreads();
  const bf16_t* cr = cosb + int64_t(t) * hd;
  const bf16_t* sr = sinb + int64_t(t) * hd;
  const int64_t slot = kc != nullptr ? slots[t] : 0;
  const int n_rot = (nh + nkv) * half;
  for (int i = threadIdx.x; i < n_rot; i += blockDim.x) {
    const int head = i / half, d = i - head * half;
    const float xl = row[head * hd + d], xh = row[head * hd + half + d];
    const float cl = bf16_to_f32(cr[d]), ch = bf16_to_f32(cr[half + d]);
    const float sl = bf16_to_f32(sr[d]), sh = bf16_to_f32(sr[half + d]);
    const bf16_t lo = f32_to_bf16(round_bf16(xl * cl) - round_bf16(xh * sl));
    const bf16_t hi = f32_to_bf16(round_bf16(xh * ch) + round_bf16(xl * sh));
    if (head < nh) {
      bf16_t* dst = q + (int64_t(t) * nh + head) * hd;
      dst[d] = lo;
      dst[half + d] = hi;
    } else {
      const int kh = head - nh;
      bf16_t* dst = k + (int64_t(t) * nkv + kh) * hd;
      dst[d] = lo;
      dst[half + d] = hi;
      if (kc != nullptr) {
        bf16_t* cd = kc + (slot * nkv + kh) * hd;
        cd[d] = lo;
        cd[half + d] = hi;
      }
    }
  }
  const int n_v = nkv * hd;
  for (int i = threadIdx.x; i < n_v; i += blockDim.x) {
    const bf16_t val = f32_to_bf16(row[(nh + nkv) * hd + i]);
    v[int64_t(t) * n_v + i] = val;
    if (vc != nullptr) vc[slot * n_v + i] = val;
  }
}

// ------------------------------------------------------------------------------------------- host side
static int target_workgroups() {
  static int target = [] {
    const char* e = getenv("NS_GEMM_TARGET_WGS");
    const int v = e != nullptr ? atoi(e) : 0;
    return v > 0 ? v : 256;
  }();
  return target;
}

static int pick_ksplit(int tiles, int K) {
  const int nchunks = (K + G_KC - 1) / G_KC;
  int k = (target_workgroups() + tiles - 1) / tiles;
  const int one_round = (nchunks + G_SC - 1) / G_SC;   // slices that fit one super chunk of loads
  if (k > 1 && k < one_round) k = one_round;            // when K is split anyway, one load round per slice
  if (k < 1) k = 1;
  if (k > nchunks) k = nchunks;     // every slice holds at least one chunk
  if (k > KMAX) k = KMAX;
  return k;
}

template <int MODE>
static int launch_main(const bf16_t* x, const bf16_t* w, const bf16_t* bias, bf16_t* y, float* ws, int M, int N,
                       int K, int tiles, int ksplit, hipStream_t st) {
  const dim3 grid(tiles, ksplit);
  if (M <= 16)
    hipLaunchKernelGGL((skinny_gemm_kernel<1, MODE>), grid, dim3(G_WAVES * 64), 0, st, x, w, bias, y, ws, M, N, K, ksplit);
  else if (M <= 32)
    hipLaunchKernelGGL((skinny_gemm_kernel<2, MODE>), grid, dim3(G_WAVES * 64), 0, st, x, w, bias, y, ws, M, N, K, ksplit);
  else
    hipLaunchKernelGGL((skinny_gemm_kernel<4, MODE>), grid, dim3(G_WAVES * 64), 0, st, x, w, bias, y, ws, M, N, K, ksplit);
  return check_launch("skinny_gemm");
}

static int check_common(const void* x, const void* w, int M, int N, int K, int dtype) {
  NS_REQUIRE(dtype == NS_DTYPE_BF16, "skinny gemm: bf16 only (dtype %d)", dtype);
  NS_REQUIRE(M >= 1 && M <= 64, "skinny gemm: M=%d outside 1..64", M);
  NS_REQUIRE(N >= 1 && K >= 32 && K % 32 == 0, "skinny gemm: N=%d K=%d (K must be a positive multiple of 32)", N, K);
  NS_REQUIRE(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) % 16) == 0,
             "skinny gemm: x and w must be 16-byte aligned");
  return NS_OK;
}

static int need_ws(void* ws, size_t ws_bytes, int ksplit, int M, int N) {
  const size_t need = size_t(ksplit) * M * N * sizeof(float);
  if (ws == nullptr || ws_bytes < need) {
    set_error("skinny gemm: workspace of %zu bytes needed, got %zu", need, ws == nullptr ? size_t(0) : ws_bytes);
    return NS_E_WORKSPACE;
  }
  return NS_OK;
}

}  // namespace ns

using namespace ns;

extern "C" size_t ns_gemm_workspace_bytes(int M, int N, int K) {
  if (M < 1 || N < 1 || K < 32) return 0;
  const int ksplit = pick_ksplit((N + 63) / 64, K);
  return size_t(ksplit) * M * N * sizeof(float);
}

extern "C" int ns_gemm(const void* x, const void* w, const void* bias, void* y, int M, int N, int K, int dtype,
                       void* ws, size_t ws_bytes, void* stream) {
  int st = check_common(x, w, M, N, K, dtype);
  if (st != NS_OK) return st;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int tiles = (N + 63) / 64;
  const int ksplit = pick_ksplit(tiles, K);
  if (ksplit == 1)
    return launch_main<GEMM_PLAIN>(static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(w),
                                   static_cast<const bf16_t*>(bias), static_cast<bf16_t*>(y), nullptr, M, N, K, tiles, 1, s);
  if ((st = need_ws(ws, ws_bytes, ksplit, M, N)) != NS_OK) return st;
  st = launch_main<GEMM_PARTIAL>(static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(w), nullptr, nullptr,
                                 static_cast<float*>(ws), M, N, K, tiles, ksplit, s);
  if (st != NS_OK) return st;
  NS_REQUIRE(N % 4 == 0, "gemm: split-K needs N %% 4 == 0 (N=%d)", N);
  hipLaunchKernelGGL(splitk_bias_kernel, dim3(unsigned((N / 4 + 255) / 256), unsigned(M)), dim3(256), 0, s,
                     static_cast<const float*>(ws), static_cast<const bf16_t*>(bias), static_cast<bf16_t*>(y), M, N,
                     ksplit);
  return check_launch("gemm split-K epilogue");
}

extern "C" int ns_gemm_silu_mul(const void* x, const void* w_gate_up, void* out, int M, int N2, int K, int dtype,
                                void* stream) {
  int st = check_common(x, w_gate_up, M, N2, K, dtype);
  if (st != NS_OK) return st;
  NS_REQUIRE(N2 % 2 == 0, "gemm_silu_mul: merged gate/up rows %d must be even", N2);
  const int tiles = (N2 / 2 + 31) / 32;
  return launch_main<GEMM_SILU>(static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(w_gate_up), nullptr,
                                static_cast<bf16_t*>(out), nullptr, M, N2, K, tiles, 1, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int ns_gemm_residual_rms_norm(const void* x, const void* w, const void* residual, void* res_out,
                                         const void* norm_w, void* h, float eps, int M, int N, int K, int dtype,
                                         void* ws, size_t ws_bytes, void* stream) {
  int st = check_common(x, w, M, N, K, dtype);
  if (st != NS_OK) return st;
  NS_REQUIRE(N % 4 == 0 && N <= 4 * EPI_THREADS, "gemm_residual_rms_norm: row length %d (multiple of 4, <= %d)", N,
             4 * EPI_THREADS);
  NS_REQUIRE(residual != nullptr && res_out != nullptr, "gemm_residual_rms_norm: residual and res_out required");
  NS_REQUIRE(norm_w == nullptr || h != nullptr, "gemm_residual_rms_norm: norm weight given without output");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int tiles = (N + 63) / 64;
  const int ksplit = pick_ksplit(tiles, K);
  if ((st = need_ws(ws, ws_bytes, ksplit, M, N)) != NS_OK) return st;
  st = launch_main<GEMM_PARTIAL>(static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(w), nullptr, nullptr,
                                 static_cast<float*>(ws), M, N, K, tiles, ksplit, s);
  if (st != NS_OK) return st;
  hipLaunchKernelGGL(splitk_residual_rmsnorm_kernel, dim3(M), dim3(unsigned((N / 4 + 63) / 64 * 64)), 0, s, static_cast<const float*>(ws),
                     static_cast<const bf16_t*>(residual), static_cast<bf16_t*>(res_out),
                     static_cast<const bf16_t*>(norm_w), static_cast<bf16_t*>(h), M, N, ksplit, eps);
  return check_launch("gemm residual/rms_norm epilogue");
}

extern "C" int ns_gemm_rope_qkv(const void* x, const void* w, const void* bias, const void* cos, const void* sin,
                                void* q, void* k, void* v, void* k_cache, void* v_cache, const int64_t* slots, int M,
                                int K, int n_heads, int n_kv_heads, int head_dim, int dtype, void* ws, size_t ws_bytes,
                                void* stream) {
  const int N = (n_heads + 2 * n_kv_heads) * head_dim;
  int st = check_common(x, w, M, N, K, dtype);
  if (st != NS_OK) return st;
  NS_REQUIRE(head_dim % 2 == 0 && N % 4 == 0 && N <= ROPE_MAX_WIDTH, "gemm_rope_qkv: width %d / head_dim %d unsupported",
             N, head_dim);
  NS_REQUIRE((k_cache == nullptr) == (v_cache == nullptr) && (k_cache == nullptr || slots != nullptr),
             "gemm_rope_qkv: give both caches and slots, or none");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int tiles = (N + 63) / 64;
  const int ksplit = pick_ksplit(tiles, K);
  if ((st = need_ws(ws, ws_bytes, ksplit, M, N)) != NS_OK) return st;
  st = launch_main<GEMM_PARTIAL>(static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(w), nullptr, nullptr,
                                 static_cast<float*>(ws), M, N, K, tiles, ksplit, s);
  if (st != NS_OK) return st;
  hipLaunchKernelGGL(splitk_bias_rope_kernel, dim3(M), dim3(unsigned((N / 4 + 63) / 64 * 64)), 0, s, static_cast<const float*>(ws),
                     static_cast<const bf16_t*>(bias), static_cast<const bf16_t*>(cos), static_cast<const bf16_t*>(sin),
                     static_cast<bf16_t*>(q), static_cast<bf16_t*>(k), static_cast<bf16_t*>(v),
                     static_cast<bf16_t*>(k_cache), static_cast<bf16_t*>(v_cache), slots, M, n_heads, n_kv_heads,
                     head_dim, ksplit);
  return check_launch("gemm rope/qkv epilogue");
}
