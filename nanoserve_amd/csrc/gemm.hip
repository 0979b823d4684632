// Skinny GEMMs of the decode step on gfx950: Y[M, N] = X[M, K] . W[N, K]^T with M <= 64 (the decode
// batch), bf16 in, fp32 accumulate, one launch per projection with the token-wise op that follows it
// fused into the epilogue. At M = 32 each weight byte feeds 32 multiply-adds, so a projection is bound
// by streaming W once from HBM; everything here serves keeping that stream full.
//
// Work split: the weight matrix is cut into 64-row tiles and K into 256-k chunks. Each workgroup owns one
// segment -- a whole tile, or one of ks K-slices of a tile -- so it flushes exactly once, at its end.
// With many tiles every workgroup takes a whole tile (two resident per CU, so one's epilogue overlaps
// the other's streaming). With fewer tiles than twice the CU count, the first CU-count tiles go whole
// and the remainder are sliced, so the last round is spread over the GPU instead of running on a few
// CUs; with fewer tiles than CUs every tile is sliced. A sliced tile's workgroups publish their fp32
// partial tiles; the last slice to arrive (a per-tile counter) sums them in slice order -- a fixed
// order, so results are deterministic -- and runs the epilogue. One launch, no epilogue kernel.
//
// Inside a workgroup (4 waves, one 64-row tile at a time):
//   * weights stream HBM -> registers -> LDS -> MFMA B fragments. Wave j loads n-tile j (16 rows) of the
//     chunk: instruction p (0..7) reads 512 contiguous bytes of row p (lanes 0-31) and of row p+8 (lanes
//     32-63). The LDS pitch of 1040 bytes per row pair keeps the stores and the 16-lane fragment reads free
//     of bank conflicts. Row-contiguous loads stream markedly faster than MFMA-layout loads (16 rows x
//     64 bytes per instruction).
//   * a rolling pipeline keeps D chunks of loads in flight per wave (register slots refilled as soon as
//     their chunk is staged); the LDS stage is double-buffered, one barrier per chunk.
//   * the 4 waves split each chunk's 8 k-steps (2 each) for all 4 n-tiles (mfma_f32_16x16x32_bf16,
//     A = X fragments straight from L2, B = weight fragments from LDS); at the end of a tile the waves'
//     partial tiles are summed through LDS in wave order.
// Epilogues (rounding points are PyTorch's for the unfused ops each one replaces):
//   STORE    y = round(acc + bias)                                        (F.linear; LM head)
//   SILU     tile = 32 gate rows + the matching 32 up rows;
//            out = round(round(silu(round(g))) * round(u))                 (silu_mul(F.linear(x, Wgu)))
//   RESNORM  o = round(acc); r = round(residual + o) -> res_out, and the row sums of r^2 over each 16
//            columns -> row_sumsq[column group][row] (fp32): the statistics of the RMSNorm that follows
// Normalised activations ("norm on load"): a projection whose input is rms_norm(r) takes r itself plus
// the producer's row_sumsq and the norm weight, and normalises each X fragment as it loads it:
//   h = round(w * round(r * inv)), inv = rsqrt(sum(row_sumsq) / K + eps)
// with the row sums added in one fixed order (rms_norm_row_inv), so every consumer -- and
// ns_rms_norm_apply, which materialises h where a tensor is needed -- sees bitwise the same h.
//   ROPE     tile = 32 dims of a head and the 32 dims half a head further (the rotate-half partners);
//            qkv = round(acc + bias), then out_lo = r(r(xl cl) - r(xh sl)), out_hi = r(r(xh ch) + r(xl sh))
//            for q and k heads, v copied; k and v also stored at the token's cache slot
// Cross-workgroup data moves through agent-scope atomic stores/loads (ns_common.h: publish_*).
#include <climits>
#include <cstdlib>
#include <type_traits>

#include "gemm_common.h"

namespace ns {

constexpr int G_WAVES = 4;
constexpr int G_TN = 4;            // 16-row n-tiles per tile: 64 weight rows
constexpr int G_KC = 256;          // k per chunk: 512 bytes of each weight row
constexpr int G_PAIR = 1040;       // LDS bytes of one row pair (rows p and p+8 of an n-tile) + 16 B pad
constexpr int G_NTB = 8 * G_PAIR;  // LDS bytes of one n-tile (16 rows) of a chunk
constexpr int G_STAGE = G_TN * G_NTB;
constexpr int G_RED = 65;          // floats per tile row in the cross-wave reduction (64 + 1 pad)
constexpr int G_NX_MAX_K = 4096;  // longest normalised input the 64-row kernel stages its norm weight for
// The arrival counters sit at the start of every workspace, in a region no other data ever uses, so the
// "all counters are zero between calls" invariant holds whatever shapes share the buffer.
constexpr int G_MAX_TILES = 8191;
constexpr size_t G_CNT_BYTES = sizeof(unsigned) * (G_MAX_TILES + 1);

struct GemmArgs {
  const bf16_t* x;
  const bf16_t* w;
  int M, N, K;              // N: rows of w
  int tiles, chunks;        // tiles, 256-k chunks per tile
  int mblocks;              // STORE above 64 rows: 64-row token blocks, each a whole plan of its own
  int whole, ks;            // tiles [0, whole) get one workgroup each; every later tile is cut into ks
                            // K slices, one workgroup each, summed by the last slice to finish
  // epilogue operands
  const bf16_t* bias;
  bf16_t* y;
  const bf16_t* residual;
  bf16_t* res_out;
  float* sumsq_out;         // RESNORM: [ceil(N/16)][64] row sums of r^2 over 16 columns
  // normalised input: x holds r; xsq [ceil(K/16)][64] its row sums of r^2, xnw the norm weight [K]
  const float* xsq;
  const bf16_t* xnw;
  float xeps;
  const bf16_t* cosb;
  const bf16_t* sinb;
  bf16_t* q;
  bf16_t* k;
  bf16_t* v;
  bf16_t* kc;
  bf16_t* vc;
  const int64_t* slots;
  int nh, nkv, hd;
  // workspace (zeroed once by the owner; every launch leaves the counters at zero)
  unsigned* cnt;    // arrival counters of the sliced tiles, cstride words apart (start of the workspace)
  int cstride;
  float* part;      // [(tiles - whole) * ks][64 rows][64] published partial tiles of the sliced tiles
  // fused argmax of the persistent kernel: tokens [M], per-row keys [M] and the arrival counter (left zero)
  int64_t* am_out;
  unsigned long long* am_key;
  unsigned* am_cnt;
};

// Weight row of n-tile j, row r (0..15) of tile t (clamped inside the matrix / its half).
template <int EPI>
__device__ __forceinline__ int tile_row(const GemmArgs& a, int t, int j, int r) {
  if constexpr (EPI == EPI_SILU) {
    const int half = a.N >> 1;
    const int row = (j < 2 ? 0 : half) + t * 32 + 16 * (j & 1) + r;
    return min(row, (j < 2 ? half : a.N) - 1);
  } else if constexpr (EPI == EPI_ROPE) {
    const int tph = a.hd >> 6;   // tiles per head
    const int head = t / tph, hf = t - head * tph;
    return head * a.hd + hf * (a.hd >> 2) + 16 * (j & 1) + (j >> 1) * (a.hd >> 1) + r;
  } else {
    return min(t * 64 + 16 * j + r, a.N - 1);
  }
}


// Values of 8 consecutive tile columns [col, col + 8) of tile row m: from the LDS reduction buffer
// (sum of the 4 waves in order) or from the published partials of the tile's ks slices (in order).
struct TileSource {
  const float* red;      // LDS [wave][R][G_RED]
  int R;
  bool from_parts;
  int ks;
  const float* part;     // slice 0 of this tile; slice s at + s * G_MAX_M * 64
};
constexpr int G_MAXC = 8;   // slices whose partials are in flight together

__device__ __forceinline__ void tile_values(const TileSource& s, int m, int col, float (&v)[8]) {
  if (!s.from_parts) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = 0.f;
#pragma unroll
      for (int w = 0; w < G_WAVES; ++w) acc += s.red[(w * s.R + m) * G_RED + col + e];
      v[e] = acc;
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = 0.f;
  for (int s0 = 0; s0 < s.ks; s0 += G_MAXC) {
    float x[G_MAXC][8];
#pragma unroll
    for (int k = 0; k < G_MAXC; ++k) {
      // partial slice layout [e][row * 8 + column group]: lanes hit consecutive words
      const float* p = s.part + int64_t(min(s0 + k, s.ks - 1)) * G_MAX_M * 64 + m * 8 + (col >> 3);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[k][e] = publish_load(p + e * G_MAX_M * 8);
    }
#pragma unroll
    for (int k = 0; k < G_MAXC; ++k)
      if (s0 + k < s.ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] += x[k][e];
  }
}

// Per-thread work items of an epilogue, unrolled to their compile-time maximum so that no loop with a
// data-dependent trip count (and memory operations) sits inside the streaming loop: the compiler's
// wait counts for the in-flight weight loads then stay exact across a tile flush.
template <int TM>
constexpr int g_items8() { return (16 * TM * 8 + G_WAVES * 64 - 1) / (G_WAVES * 64); }   // (row, 8 columns)
template <int TM>
constexpr int g_items4() { return (16 * TM * 4 + G_WAVES * 64 - 1) / (G_WAVES * 64); }   // (row, 8 lo + 8 hi)

// Drain this wave's memory operations after a loop whose trip count depends on data: with nothing left
// in flight, the compiler's wait counts for the prefetched slots are exact again.
__device__ __forceinline__ void drain_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// RESNORM's residual fragments of this thread's epilogue items (row m, 8 columns), loaded at kernel start
// with clamped addresses, so the epilogue waits for no round trip of its own.
template <int TM, int EPI>
__device__ __forceinline__ void res_prefetch(const GemmArgs& a, int t, g_u32x4_t (&pre)[g_items8<4>()]) {
  if constexpr (EPI == EPI_RESNORM) {
#pragma unroll
    for (int it = 0; it < g_items8<TM>(); ++it) {
      const int idx = threadIdx.x + it * G_WAVES * 64;
      const int m = min(idx >> 3, a.M - 1), n0 = min(t * 64 + 8 * (idx & 7), a.N - 8);
      pre[it] = *reinterpret_cast<const g_u32x4_t*>(a.residual + int64_t(m) * a.N + n0);
    }
  }
}

// pre: RESNORM's residual fragments of this thread's items, loaded at kernel start (res_prefetch)
template <int TM, int EPI>
__device__ __forceinline__ void tile_epilogue(const GemmArgs& a, const TileSource& src, int t,
                                              const g_u32x4_t (&pre)[g_items8<4>()]) {
  const int tid = threadIdx.x, M = a.M;
  if constexpr (EPI == EPI_STORE) {
#pragma unroll
    for (int it = 0; it < g_items8<TM>(); ++it) {
      const int idx = tid + it * G_WAVES * 64;
      const int m = idx >> 3, cq = idx & 7, n0 = t * 64 + 8 * cq;
      if (m < M && n0 < a.N) {
        float v[8];
        tile_values(src, m, 8 * cq, v);
        if (a.bias != nullptr)
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] += n0 + e < a.N ? bf16_to_f32(a.bias[n0 + e]) : 0.f;
        bf16_t* dst = a.y + int64_t(m) * a.N + n0;
        if ((a.N & 7) == 0) {
          store_bf16x8(dst, v);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (n0 + e < a.N) dst[e] = f32_to_bf16(v[e]);
        }
      }
    }
  } else if constexpr (EPI == EPI_SILU) {
    const int half = a.N >> 1;
#pragma unroll
    for (int it = 0; it < g_items4<TM>(); ++it) {
      const int idx = tid + it * G_WAVES * 64;
      const int m = idx >> 2, cq = idx & 3, n0 = t * 32 + 8 * cq;
      if (m < M && n0 < half) {
        float gv[8], uv[8], o[8];
        tile_values(src, m, 8 * cq, gv);
        tile_values(src, m, 32 + 8 * cq, uv);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float gb = round_bf16(gv[e]), ub = round_bf16(uv[e]);
          o[e] = round_bf16(gb / (1.0f + expf(-gb))) * ub;
        }
        bf16_t* dst = a.y + int64_t(m) * half + n0;
        if ((half & 7) == 0) {
          store_bf16x8(dst, o);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (n0 + e < half) dst[e] = f32_to_bf16(o[e]);
        }
      }
    }
  } else if constexpr (EPI == EPI_ROPE) {
    const int tph = a.hd >> 6, head = t / tph, hf = t - head * tph, hh = a.hd >> 1;
#pragma unroll
    for (int it = 0; it < g_items4<TM>(); ++it) {
      const int idx = tid + it * G_WAVES * 64;
      const int m = idx >> 2, cq = idx & 3;
      if (m < M) {
        const int d0 = hf * (a.hd >> 2) + 8 * cq;             // dims d0..d0+7 and d0+hd/2..
        float xl[8], xh[8], lo[8], hi[8];
        tile_values(src, m, 8 * cq, xl);
        tile_values(src, m, 32 + 8 * cq, xh);
        const int rl = head * a.hd + d0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          xl[e] = round_bf16(xl[e] + (a.bias != nullptr ? bf16_to_f32(a.bias[rl + e]) : 0.f));
          xh[e] = round_bf16(xh[e] + (a.bias != nullptr ? bf16_to_f32(a.bias[rl + hh + e]) : 0.f));
        }
        if (head < a.nh + a.nkv) {
          float cl[8], ch[8], sl[8], sh[8];
          load_bf16x8(a.cosb + int64_t(m) * a.hd + d0, cl);
          load_bf16x8(a.cosb + int64_t(m) * a.hd + d0 + hh, ch);
          load_bf16x8(a.sinb + int64_t(m) * a.hd + d0, sl);
          load_bf16x8(a.sinb + int64_t(m) * a.hd + d0 + hh, sh);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            lo[e] = round_bf16(xl[e] * cl[e]) - round_bf16(xh[e] * sl[e]);
            hi[e] = round_bf16(xh[e] * ch[e]) + round_bf16(xl[e] * sh[e]);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            lo[e] = xl[e];
            hi[e] = xh[e];
          }
        }
        bf16_t* dst;
        bf16_t* cdst = nullptr;
        if (head < a.nh) {
          dst = a.q + (int64_t(m) * a.nh + head) * a.hd;
        } else if (head < a.nh + a.nkv) {
          const int kh = head - a.nh;
          dst = a.k + (int64_t(m) * a.nkv + kh) * a.hd;
          if (a.kc != nullptr) cdst = a.kc + (a.slots[m] * a.nkv + kh) * a.hd;
        } else {
          const int vh = head - a.nh - a.nkv;
          dst = a.v + (int64_t(m) * a.nkv + vh) * a.hd;
          if (a.vc != nullptr) cdst = a.vc + (a.slots[m] * a.nkv + vh) * a.hd;
        }
        store_bf16x8(dst + d0, lo);
        store_bf16x8(dst + d0 + hh, hi);
        if (cdst != nullptr) {
          store_bf16x8(cdst + d0, lo);
          store_bf16x8(cdst + d0 + hh, hi);
        }
      }
    }
  } else {  // EPI_RESNORM
    const int N = a.N;
    // res_out and the row sums of r^2 over each 16 columns (8 threads per row: lanes 8k .. 8k+7)
#pragma unroll
    for (int it = 0; it < g_items8<TM>(); ++it) {
      const int idx = tid + it * G_WAVES * 64;
      const int m = idx >> 3, cq = idx & 7, n0 = t * 64 + 8 * cq;
      const bool live = m < M;
      float ss = 0.f;
      if (live && n0 < N) {
        float o[8], rs[8], r[8];
        tile_values(src, m, 8 * cq, o);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          rs[2 * e] = __uint_as_float(pre[it][e] << 16);
          rs[2 * e + 1] = __uint_as_float(pre[it][e] & 0xffff0000u);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          r[e] = round_bf16(rs[e] + round_bf16(o[e]));
          ss += r[e] * r[e];
        }
        store_bf16x8(a.res_out + int64_t(m) * N + n0, r);
      }
      ss += __shfl_xor(ss, 1, 64);   // columns 16p .. 16p+15 (two 8-column groups)
      if (live && (cq & 1) == 0 && n0 < N && a.sumsq_out != nullptr)
        a.sumsq_out[int64_t(4 * t + (cq >> 1)) * G_NORM_ROWS + m] = ss;
    }
  }
}

// inv of row m for normalised inputs: lane group r4 (the 4 lanes of one row) adds the row sums of
// producer tiles r4, r4+4, ... in order, then the groups combine as (g0 + g1) + (g2 + g3) through two
// butterfly steps, which gives every lane of the 4 the same bits. Called by all 64 lanes of a wave.
__device__ __forceinline__ float rms_norm_row_inv(const float* sumsq, int ptiles, int m, int r4, int K, float eps) {
  float part = 0.f;
  for (int p0 = r4; p0 < ptiles; p0 += 32) {   // 8 loads in flight, added in tile order
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = p0 + 4 * e < ptiles ? sumsq[int64_t(p0 + 4 * e) * G_NORM_ROWS + m] : 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) part += v[e];
  }
  part += __shfl_xor(part, 16, 64);
  part += __shfl_xor(part, 32, 64);
  return rsqrtf(part / float(K) + eps);
}


template <int TM, int EPI, bool NX>
__global__ __launch_bounds__(G_WAVES * 64) void skinny_gemm_kernel(GemmArgs a) {
  __shared__ __align__(16) unsigned char lds[2 * G_STAGE];
  __shared__ unsigned s_flag;
  constexpr int R = 16 * TM;
  // this workgroup's segment: chunks [c0, c1) of tile t (slice s of ks)
  int b = blockIdx.x;
  if constexpr (EPI == EPI_STORE || EPI == EPI_RESNORM) {
    if (a.mblocks > 1) {   // token block mb: rows 64 mb .. 64 mb + 63, with its own counters and partials
      const int per = a.whole + (a.tiles - a.whole) * a.ks, mb = b / per;
      b -= mb * per;
      a.x += int64_t(G_MAX_M) * mb * a.K;
      if constexpr (EPI == EPI_STORE) {
        a.y += int64_t(G_MAX_M) * mb * a.N;
      } else {
        a.residual += int64_t(G_MAX_M) * mb * a.N;
        a.res_out += int64_t(G_MAX_M) * mb * a.N;
        if (a.sumsq_out != nullptr) a.sumsq_out += G_MAX_M * mb;
      }
      a.M = min(G_MAX_M, a.M - G_MAX_M * mb);
      a.cnt += mb * (a.tiles - a.whole) * a.cstride;
      a.part += int64_t(mb) * (a.tiles - a.whole) * a.ks * G_MAX_M * 64;
    }
  }
  const int C = a.chunks, K = a.K;
  int t, s, ks;
  if (b < a.whole) {
    t = b;
    s = 0;
    ks = 1;
  } else {
    ks = a.ks;
    t = a.whole + (b - a.whole) / ks;
    s = (b - a.whole) - (t - a.whole) * ks;
  }
  const int c0 = s * C / ks, c1 = (s + 1) * C / ks;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int c16 = lane & 15, r4 = lane >> 4;
  const int half_sel = lane >> 5, col16 = lane & 31;
  const int st_off = wv * G_NTB + half_sel * 512 + col16 * 16;        // + p * G_PAIR
  const int fr_off = (c16 & 7) * G_PAIR + (c16 >> 3) * 512 + r4 * 16;   // + j * G_NTB + kstep * 64
  const bf16_t* wbase[8];
#pragma unroll
  for (int p = 0; p < 8; ++p) wbase[p] = a.w + int64_t(tile_row<EPI>(a, t, wv, p + 8 * half_sel)) * K + 8 * col16;
  const bf16_t* xrow[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) xrow[i] = a.x + int64_t(min(16 * i + c16, a.M - 1)) * K + 8 * r4;
  float xinv[TM];   // normalised input: inv of this lane's X rows (computed once the first loads are out)

  g_float4_t acc[TM][G_TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < G_TN; ++j) acc[i][j] = g_float4_t{0.f, 0.f, 0.f, 0.f};

  // Rolling pipeline: register slot q holds the weight rows (and this wave's X fragments) of chunk
  // c0 + q (mod D); while one chunk is staged through LDS and multiplied, the loads of the next D-1 are
  // in flight, and a slot is refilled with chunk c + D as soon as its chunk has been staged. Refills past
  // the segment re-load its last chunk (an L2 hit), so every path issues the same load sequence and the
  // compiler's wait counts stay exact (vmcnt leaves the other slots' loads in flight).
  // Epilogue operands and row statistics go out before the weight stream (waiting for them never waits
  // for it); a normalised input's norm weight is staged through LDS once (a per-fragment load would cost a
  // 1 KB wave access for 64 distinct bytes).
  g_u32x4_t pre[g_items8<4>()];
  res_prefetch<TM, EPI>(a, t, pre);
  const bool stat_wave = wv < TM;   // threads 0 .. 64 TM - 1 hold the (row, group) pairs
  const int ptiles = (K + G_NORM_COLS - 1) / G_NORM_COLS;
  float rs[RS_PRE];
  constexpr int NW_PER_THREAD = G_NX_MAX_K / 2 / (G_WAVES * 64);
  uint32_t nw_word[NW_PER_THREAD];
  if constexpr (NX) {
    if (stat_wave) row_stats_issue(a.xsq, ptiles, a.M, rs);
#pragma unroll
    for (int j = 0; j < NW_PER_THREAD; ++j)
      nw_word[j] = reinterpret_cast<const uint32_t*>(a.xnw)[min(tid + j * G_WAVES * 64, (K >> 1) - 1)];
  }
  constexpr int D = (TM <= 2 && !NX) ? 3 : 2;
  g_u32x4_t wr[D][8], xf[D][2][TM];
  __shared__ __align__(16) uint32_t s_nw[NX ? G_NX_MAX_K / 2 : 4];
  const int clast = c1 - 1;
  auto load_w = [&](auto qc, int c) __attribute__((always_inline)) {
    constexpr int q = decltype(qc)::value;
    const int kc = min(c * G_KC, K - 8 * col16 - 8);   // k beyond K: a clamped in-bounds address, masked below
#pragma unroll
    for (int p = 0; p < 8; ++p) wr[q][p] = *reinterpret_cast<const g_u32x4_t*>(wbase[p] + kc);
  };
  auto load_x = [&](auto qc, int c) __attribute__((always_inline)) {
    constexpr int q = decltype(qc)::value;
    const int kc = c * G_KC;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int k = min(kc + 32 * (2 * wv + h), K - 32);
#pragma unroll
      for (int i = 0; i < TM; ++i) xf[q][h][i] = *reinterpret_cast<const g_u32x4_t*>(xrow[i] + k);
    }
  };
  int buf = 0;
  auto step = [&](auto qc, int c, int next) __attribute__((always_inline)) {
    constexpr int q = decltype(qc)::value;
    unsigned char* stage = lds + buf * G_STAGE;
#pragma unroll
    for (int p = 0; p < 8; ++p) *reinterpret_cast<g_u32x4_t*>(stage + st_off + p * G_PAIR) = wr[q][p];
    load_w(qc, next);
    __syncthreads();   // the chunk's 64 rows are in this buffer; every wave is done with the other one
    const int kc = c * G_KC;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int kstep = 2 * wv + h;
      if (kc + 32 * kstep < K) {   // uniform
        g_u32x4_t w8;
        if constexpr (NX) w8 = *reinterpret_cast<const g_u32x4_t*>(s_nw + ((kc + 32 * kstep + 8 * r4) >> 1));
        g_bf16x8_t bfr[G_TN];
#pragma unroll
        for (int j = 0; j < G_TN; ++j)
          bfr[j] = __builtin_bit_cast(g_bf16x8_t, *reinterpret_cast<const g_u32x4_t*>(stage + j * G_NTB + kstep * 64 + fr_off));
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          g_u32x4_t xa = xf[q][h][i];
          if constexpr (NX) xa = norm_fragment(xa, w8, xinv[i]);
#pragma unroll
          for (int j = 0; j < G_TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(g_bf16x8_t, xa), bfr[j], acc[i][j], 0,
                                                                0, 0);
        }
      }
    }
    load_x(qc, next);
    buf ^= 1;
  };
  using Q0 = std::integral_constant<int, 0>;
  using Q1 = std::integral_constant<int, 1>;
  using Q2 = std::integral_constant<int, 2>;
  load_w(Q0{}, c0);
  load_x(Q0{}, c0);
  load_w(Q1{}, min(c0 + 1, clast));
  load_x(Q1{}, min(c0 + 1, clast));
  if constexpr (D > 2) {
    load_w(Q2{}, min(c0 + 2, clast));
    load_x(Q2{}, min(c0 + 2, clast));
  }
  if constexpr (NX) {   // the statistics' and norm weight's round trip overlaps the first chunks' loads
    __shared__ float s_inv[G_MAX_M];
    if (stat_wave) row_stats_finish(a.xsq, ptiles, a.M, K, a.xeps, rs, s_inv);
#pragma unroll
    for (int j = 0; j < NW_PER_THREAD; ++j)
      if (tid + j * G_WAVES * 64 < (K >> 1)) s_nw[tid + j * G_WAVES * 64] = nw_word[j];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TM; ++i) xinv[i] = s_inv[min(16 * i + c16, a.M - 1)];
  }
  int c = c0;
  for (; c + D <= c1; c += D) {   // whole rounds only: no path into the loop header skips a step
    step(Q0{}, c, min(c + D, clast));
    step(Q1{}, c + 1, min(c + 1 + D, clast));
    if constexpr (D > 2) step(Q2{}, c + 2, min(c + 2 + D, clast));
  }
  if (c < c1) step(Q0{}, c, clast);
  if constexpr (D > 2)
    if (c + 1 < c1) step(Q1{}, c + 1, clast);

  // ---- the segment is done: sum the waves' partial tiles through LDS (wave order)
  float* red = reinterpret_cast<float*>(lds);
  __syncthreads();   // every wave is done with both stage buffers
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < G_TN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[(wv * R + 16 * i + 4 * r4 + r) * G_RED + 16 * j + c16] = acc[i][j][r];
  __syncthreads();
  TileSource src{red, R, false, ks, nullptr};
  if (ks == 1) {
    tile_epilogue<TM, EPI>(a, src, t, pre);
    return;
  }
  // sliced tile: publish this slice's partial; the last slice to arrive sums all of them in slice order
  float* tile_part = a.part + int64_t(t - a.whole) * ks * G_MAX_M * 64;
  float* my = tile_part + int64_t(s) * G_MAX_M * 64;
#pragma unroll
  for (int it = 0; it < g_items8<TM>(); ++it) {
    const int idx = tid + it * G_WAVES * 64;
    const int m = idx >> 3, cq = idx & 7;
    if (m < a.M) {
      float v[8];
      tile_values(src, m, 8 * cq, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) publish_store(my + e * G_MAX_M * 8 + m * 8 + cq, v[e]);
    }
  }
  publish_complete();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = publish_count(a.cnt + (t - a.whole) * a.cstride);
    const unsigned last = prev == unsigned(ks - 1);
    if (last) publish_reset(a.cnt + (t - a.whole) * a.cstride);
    s_flag = last;
  }
  __syncthreads();
  if (s_flag == 0u) return;
  acquire_published();
  src.from_parts = true;
  src.part = tile_part;
  tile_epilogue<TM, EPI>(a, src, t, pre);
}

// ---------------------------------------------------------------------------------------------------
// Persistent 64-row GEMM for wide STORE projections (the tied LM head: ~2,400 tiles of 64 vocabulary rows)
// with M <= 32 and K <= 2048. Launched one workgroup per tile, every workgroup re-reads the whole activation
// block (96 KB at M = 32, K = 1536) for its 196 KB of weights. Here about two workgroups per CU stay
// resident and walk tiles blockIdx.x, blockIdx.x + G, ...: each wave loads the activation fragments of its
// k-steps (2 wv, 2 wv + 1 of every 256-k chunk) once -- normalised once for a normalised input -- and keeps
// them in registers, so the weights are the only stream. A workgroup's (tile, chunk) sequence is one
// rolling pipeline (two chunks of weight loads in flight, staged through LDS exactly as in the 64-row
// kernel), so the next tile's first chunks are in flight while a tile's partial sums are reduced and
// stored; the reduction reuses the stage buffer of the tile's last chunk. CP: chunks per tile rounded up to
// even (a padding chunk re-reads the last one and multiplies nothing).
// AM: the greedy argmax of every row is fused (the LM head of a decode step). The thread that stores
// (row m, 8 columns) of a tile keeps the row's best (stored bf16 value, index) over its tiles; at the end
// the 8 threads of a row combine, one 64-bit atomic max per (workgroup, row) folds it into the row's key
// (argmax_key: the order of torch.argmax), and the last workgroup to arrive turns the keys into tokens and
// clears them. The result is ns_argmax_rows' on the stored logits.
template <int TM, bool NX, int CP, bool AM>
__global__ __launch_bounds__(G_WAVES * 64) __attribute__((amdgpu_waves_per_eu(2, 2))) void persist_gemm_kernel(GemmArgs a) {
  static_assert(TM <= 2 && CP % 2 == 0 && CP <= 8, "reduction in one stage buffer; K <= 2048");
  static_assert(g_items8<TM>() == 1, "one (row, 8 columns) item per thread");
  __shared__ __align__(16) unsigned char lds[2 * G_STAGE];
  constexpr int R = 16 * TM;
  const int G = gridDim.x, K = a.K, N = a.N;
  const int n_my = (a.tiles - int(blockIdx.x) + G - 1) / G;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int c16 = lane & 15, r4 = lane >> 4;
  const int half_sel = lane >> 5, col16 = lane & 31;
  const int st_off = wv * G_NTB + half_sel * 512 + col16 * 16;        // + p * G_PAIR
  const int fr_off = (c16 & 7) * G_PAIR + (c16 >> 3) * 512 + r4 * 16;   // + j * G_NTB + kstep * 64

  // (normalised input) statistics and norm weight first, so waiting for them waits for nothing else
  const bool stat_wave = wv < TM;
  const int ptiles = (K + G_NORM_COLS - 1) / G_NORM_COLS;
  float rs[RS_PRE];
  constexpr int NWT = 2048 / 2 / (G_WAVES * 64);   // norm-weight words per thread (K <= 2048)
  uint32_t nw_word[NWT];
  if constexpr (NX) {
    if (stat_wave) row_stats_issue(a.xsq, ptiles, a.M, rs);
#pragma unroll
    for (int j = 0; j < NWT; ++j)
      nw_word[j] = reinterpret_cast<const uint32_t*>(a.xnw)[min(tid + j * G_WAVES * 64, (K >> 1) - 1)];
  }
  // this wave's activation fragments of every chunk
  g_u32x4_t xa[CP][2][TM];
#pragma unroll
  for (int c = 0; c < CP; ++c)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int k = min(c * G_KC + 32 * (2 * wv + h), K - 32) + 8 * r4;
#pragma unroll
      for (int i = 0; i < TM; ++i)
        xa[c][h][i] = *reinterpret_cast<const g_u32x4_t*>(a.x + int64_t(min(16 * i + c16, a.M - 1)) * K + k);
    }
  // weights: stream position (tile i of this workgroup, chunk c); past the end it re-reads the last one
  g_u32x4_t wr[2][8];
  auto load_w = [&](auto qc, int i, int c) __attribute__((always_inline)) {
    constexpr int q = decltype(qc)::value;
    if (c >= CP) {
      c -= CP;
      ++i;
    }
    if (i >= n_my) {
      i = n_my - 1;
      c = CP - 1;
    }
    const int t = int(blockIdx.x) + i * G;
    const int kc = min(c * G_KC, K - 8 * col16 - 8);   // k beyond K: a clamped in-bounds address, not multiplied
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const int row = min(t * 64 + 16 * wv + p + 8 * half_sel, N - 1);
      wr[q][p] = *reinterpret_cast<const g_u32x4_t*>(a.w + int64_t(row) * K + 8 * col16 + kc);
    }
  };
  using Q0 = std::integral_constant<int, 0>;
  using Q1 = std::integral_constant<int, 1>;
  load_w(Q0{}, 0, 0);
  load_w(Q1{}, 0, 1);
  if constexpr (NX) {
    __shared__ float s_inv[G_MAX_M];
    __shared__ __align__(16) uint32_t s_nw[1024];
    if (stat_wave) row_stats_finish(a.xsq, ptiles, a.M, K, a.xeps, rs, s_inv);
#pragma unroll
    for (int j = 0; j < NWT; ++j)
      if (tid + j * G_WAVES * 64 < (K >> 1)) s_nw[tid + j * G_WAVES * 64] = nw_word[j];
    __syncthreads();
    float xinv[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) xinv[i] = s_inv[min(16 * i + c16, a.M - 1)];
#pragma unroll
    for (int c = 0; c < CP; ++c)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k0 = c * G_KC + 32 * (2 * wv + h);
        if (k0 < K) {
          const g_u32x4_t w8 = *reinterpret_cast<const g_u32x4_t*>(s_nw + ((k0 + 8 * r4) >> 1));
#pragma unroll
          for (int i = 0; i < TM; ++i) xa[c][h][i] = norm_fragment(xa[c][h][i], w8, xinv[i]);
        }
      }
  }
  g_float4_t acc[TM][G_TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < G_TN; ++j) acc[i][j] = g_float4_t{0.f, 0.f, 0.f, 0.f};
  int buf = 0;
  auto step = [&](auto qc, auto cc, int i) __attribute__((always_inline)) {
    constexpr int q = decltype(qc)::value, c = decltype(cc)::value;
    unsigned char* stage = lds + buf * G_STAGE;
#pragma unroll
    for (int p = 0; p < 8; ++p) *reinterpret_cast<g_u32x4_t*>(stage + st_off + p * G_PAIR) = wr[q][p];
    load_w(qc, i, c + 2);
    __syncthreads();   // the chunk's 64 rows are in this buffer; every wave is done with the other one
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int kstep = 2 * wv + h;
      if (c * G_KC + 32 * kstep < K) {   // uniform
        g_bf16x8_t bfr[G_TN];
#pragma unroll
        for (int j = 0; j < G_TN; ++j)
          bfr[j] = __builtin_bit_cast(g_bf16x8_t, *reinterpret_cast<const g_u32x4_t*>(stage + j * G_NTB + kstep * 64 + fr_off));
#pragma unroll
        for (int ii = 0; ii < TM; ++ii)
#pragma unroll
          for (int j = 0; j < G_TN; ++j)
            acc[ii][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(g_bf16x8_t, xa[c][h][ii]), bfr[j],
                                                                 acc[ii][j], 0, 0, 0);
      }
    }
    buf ^= 1;
  };
  const g_u32x4_t none[g_items8<4>()] = {};
  float am_v = -INFINITY;   // AM: this thread's row best so far (row tid / 8, its 8 columns of every tile)
  int am_i = 0x7fffffff;
  for (int i = 0; i < n_my; ++i) {
    step(Q0{}, std::integral_constant<int, 0>{}, i);
    step(Q1{}, std::integral_constant<int, 1>{}, i);
    if constexpr (CP > 2) {
      step(Q0{}, std::integral_constant<int, 2>{}, i);
      step(Q1{}, std::integral_constant<int, 3>{}, i);
    }
    if constexpr (CP > 4) {
      step(Q0{}, std::integral_constant<int, 4>{}, i);
      step(Q1{}, std::integral_constant<int, 5>{}, i);
    }
    if constexpr (CP > 6) {
      step(Q0{}, std::integral_constant<int, 6>{}, i);
      step(Q1{}, std::integral_constant<int, 7>{}, i);
    }
    // tile done: the waves' partial tiles are summed through the buffer of the last chunk (wave order)
    float* red = reinterpret_cast<float*>(lds + (buf ^ 1) * G_STAGE);
    __syncthreads();   // every wave is done multiplying out of that buffer
#pragma unroll
    for (int ii = 0; ii < TM; ++ii)
#pragma unroll
      for (int j = 0; j < G_TN; ++j) {
#pragma unroll
        for (int r = 0; r < 4; ++r) red[(wv * R + 16 * ii + 4 * r4 + r) * G_RED + 16 * j + c16] = acc[ii][j][r];
        acc[ii][j] = g_float4_t{0.f, 0.f, 0.f, 0.f};
      }
    __syncthreads();
    TileSource src{red, R, false, 1, nullptr};
    if constexpr (!AM) {
      tile_epilogue<TM, EPI_STORE>(a, src, int(blockIdx.x) + i * G, none);
    } else {   // the STORE epilogue (no bias), keeping the stored values' best per row
      const int m = tid >> 3, cq = tid & 7, n0 = (int(blockIdx.x) + i * G) * 64 + 8 * cq;
      if (m < a.M && n0 < N) {
        float v[8];
        tile_values(src, m, 8 * cq, v);
        bf16_t* dst = a.y + int64_t(m) * N + n0;
        if ((N & 7) == 0) {
          store_bf16x8(dst, v);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float f = __uint_as_float(pack_bf16x2(v[e], 0.f) << 16);
            if (better(f, n0 + e, am_v, am_i)) { am_v = f; am_i = n0 + e; }
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (n0 + e < N) {
              const bf16_t b = f32_to_bf16(v[e]);
              dst[e] = b;
              const float f = bf16_to_f32(b);
              if (better(f, n0 + e, am_v, am_i)) { am_v = f; am_i = n0 + e; }
            }
        }
      }
    }
  }
  if constexpr (AM) {
    __shared__ unsigned s_am_last;
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) {   // the 8 threads of a row are 8 consecutive lanes
      const float ov = __shfl_xor(am_v, o, 64);
      const int oi = __shfl_xor(am_i, o, 64);
      if (better(ov, oi, am_v, am_i)) { am_v = ov; am_i = oi; }
    }
    const int m = tid >> 3;
    if ((tid & 7) == 0 && m < a.M && am_i != 0x7fffffff)
      __hip_atomic_fetch_max(a.am_key + m, argmax_key(am_v, am_i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    publish_complete();
    __syncthreads();
    if (tid == 0) {
      const unsigned prev = publish_count(a.am_cnt);
      const unsigned last = prev == unsigned(G - 1);
      if (last) publish_reset(a.am_cnt);
      s_am_last = last;
    }
    __syncthreads();
    if (s_am_last == 0u) return;
    acquire_published();
    if (tid < a.M) {
      const unsigned long long key = __hip_atomic_load(a.am_key + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.am_key + tid, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      a.am_out[tid] = key == 0ull ? 0 : int64_t(~uint32_t(key));
    }
  }
}

// ---------------------------------------------------------------------------------------------------
// Tile-16 GEMM for projections with few weight rows (QKV, O: N in the low thousands, K <= 2048). A split-K
// plan would need a cross-workgroup merge whose round trips (publish, counter, reload) cost more than the
// few microseconds these projections stream for, so here one workgroup owns 16 weight rows over the whole
// of K and nothing crosses workgroups:
//   * 16 waves; wave w reads weight row w of the tile row-contiguously (16 bytes per lane, 1 KB per
//     instruction) and stores it to LDS with its 16-byte chunks XOR-swizzled by the row inside each
//     256-byte group, so the 16 rows one B-fragment read touches sit in 16 different bank groups.
//   * wave w multiplies k-steps [w nks / 16, (w + 1) nks / 16): X fragments straight from L2 (normalised
//     on load when the input is a NormedRows), B fragments from LDS; the 16 partial tiles are summed
//     through LDS in wave order (deterministic).
//   * everything the epilogue reads (bias, residual, cos/sin, slots, row statistics) is loaded at kernel
//     start together with the weights, so the only dependent steps are the one weight round trip, the
//     barrier and the stores.
// Tiles: STORE / RESNORM 16 consecutive rows; SILU 8 gate rows + the matching 8 up rows (8 output
// columns); ROPE 8 dims of a head + the 8 dims half a head further (the rotate-half partners).
constexpr int T16_WAVES = 16;
constexpr int T16_MAX_K = 2048;
constexpr int T16_KSW = T16_MAX_K / 32 / T16_WAVES;   // k-steps per wave at most

template <int EPI>
__device__ __forceinline__ int t16_row(const GemmArgs& a, int t, int r) {
  if constexpr (EPI == EPI_SILU) {
    const int half = a.N >> 1;
    return r < 8 ? min(8 * t + r, half - 1) : half + min(8 * t + r - 8, half - 1);
  } else if constexpr (EPI == EPI_ROPE) {
    const int tph = a.hd >> 4, head = t / tph, f = t - head * tph;
    return head * a.hd + 8 * f + (r < 8 ? r : (a.hd >> 1) + r - 8);
  } else {
    return min(16 * t + r, a.N - 1);
  }
}

template <int TM, int EPI, bool NX>
__global__ __launch_bounds__(T16_WAVES * 64) void tile16_gemm_kernel(GemmArgs a) {
  __shared__ __align__(16) unsigned char lds[16 * 2 * T16_MAX_K];   // weight tile, then the partial tiles
  // Token-split launch (TM = 1 with M > 16, gridDim.x = tiles * ceil(M / 16)): workgroup mb * tiles + t
  // computes tokens [16 mb, 16 mb + 16) of tile t over all of K. The token blocks of a tile share its weight
  // rows through L2 (same XCD when tiles % 8 == 0) and each workgroup reads half the activations.
  int t = blockIdx.x;
  if (TM == 1 && a.M > 16) {
    const int mbs = (a.M + 15) >> 4, tiles = int(gridDim.x) / mbs, mb = t / tiles, m0 = 16 * mb;
    t -= mb * tiles;
    a.M = min(16, a.M - m0);
    a.x += int64_t(m0) * a.K;
    if constexpr (NX) a.xsq += m0;
    if constexpr (EPI == EPI_STORE) {
      a.y += int64_t(m0) * a.N;
    } else if constexpr (EPI == EPI_RESNORM) {
      a.residual += int64_t(m0) * a.N;
      a.res_out += int64_t(m0) * a.N;
      if (a.sumsq_out != nullptr) a.sumsq_out += m0;
    } else if constexpr (EPI == EPI_SILU) {
      a.y += int64_t(m0) * (a.N >> 1);
    } else {
      a.cosb += int64_t(m0) * a.hd;
      a.sinb += int64_t(m0) * a.hd;
      if (a.slots != nullptr) a.slots += m0;
      a.q += int64_t(m0) * a.nh * a.hd;
      a.k += int64_t(m0) * a.nkv * a.hd;
      a.v += int64_t(m0) * a.nkv * a.hd;
    }
  }
  const int M = a.M, K = a.K;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int c16 = lane & 15, r4 = lane >> 4;
  const int rowb = 2 * K;   // bytes of a weight row = LDS pitch

  // Epilogue operands (raw bits) and the row statistics go out first, with branch-free addresses (a
  // missing operand reads a harmless in-bounds word instead): they return before the weights, waiting for
  // them never waits for the weight stream, and nothing is converted until the epilogue.
  constexpr int PAIR = (EPI == EPI_SILU || EPI == EPI_ROPE) ? 1 : 0;
  const int em = PAIR ? (tid >> 3) : (tid >> 4);
  const int en = PAIR ? (tid & 7) : (tid & 15);
  const bool elive = em < M && tid < TM * 16 * (PAIR ? 8 : 16);
  const int emc = min(em, M - 1);
  bf16_t r_b0 = 0, r_b1 = 0, r_cl = 0, r_ch = 0, r_sl = 0, r_sh = 0, r_res = 0;
  int64_t e_slot = 0;
  const bf16_t* bias_src = a.bias != nullptr ? a.bias : a.w;
  if constexpr (EPI == EPI_STORE) {
    r_b0 = bias_src[min(16 * t + en, a.N - 1)];
  } else if constexpr (EPI == EPI_RESNORM) {
    r_res = a.residual[int64_t(emc) * a.N + min(16 * t + en, a.N - 1)];
  } else if constexpr (EPI == EPI_ROPE) {
    const int tph = a.hd >> 4, head = t / tph, f = t - head * tph, hh = a.hd >> 1;
    const int d = 8 * f + en;
    r_b0 = bias_src[head * a.hd + d];
    r_b1 = bias_src[head * a.hd + hh + d];
    r_cl = a.cosb[int64_t(emc) * a.hd + d];
    r_ch = a.cosb[int64_t(emc) * a.hd + hh + d];
    r_sl = a.sinb[int64_t(emc) * a.hd + d];
    r_sh = a.sinb[int64_t(emc) * a.hd + hh + d];
    e_slot = (a.slots != nullptr ? a.slots : reinterpret_cast<const int64_t*>(a.w))[emc];
  }
  const bool stat_wave = wv < TM;   // threads 0 .. 64 TM - 1 hold the (row, group) pairs
  const int ptiles = (K + G_NORM_COLS - 1) / G_NORM_COLS;
  float rs[RS_PRE];
  uint32_t nw_word = 0;
  if constexpr (NX) {
    if (stat_wave) row_stats_issue(a.xsq, ptiles, M, rs);
    // the norm weight, one 4-byte word per thread (K <= 2048), staged through LDS: a per-fragment load would
    // cost a 1 KB wave access for 64 distinct bytes
    nw_word = reinterpret_cast<const uint32_t*>(a.xnw)[min(tid, (K >> 1) - 1)];
  }
  // X fragments of this wave's k-steps and weight row wv of the tile (16 bytes per lane per 1 KB piece). A
  // normalised input's fragments go out first: they arrive first and are normalised while the weight rows
  // are still in flight; a plain input's go out after the weights, which the workgroup waits for first.
  const int nks = K >> 5;
  const int ks0 = wv * nks / T16_WAVES, ks1 = (wv + 1) * nks / T16_WAVES;
  g_u32x4_t xr[T16_KSW][TM];
  g_u32x4_t wr[T16_MAX_K * 2 / 1024];
  auto load_x = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < T16_KSW; ++s) {
      const int k = 32 * max(min(ks0 + s, ks1 - 1), 0) + 8 * r4;   // past the wave's range: an in-bounds re-read
#pragma unroll
      for (int i = 0; i < TM; ++i)
        xr[s][i] = *reinterpret_cast<const g_u32x4_t*>(a.x + int64_t(min(16 * i + c16, M - 1)) * K + k);
    }
  };
  auto load_w = [&]() __attribute__((always_inline)) {
    const unsigned char* src = reinterpret_cast<const unsigned char*>(a.w + int64_t(t16_row<EPI>(a, t, wv)) * K);
#pragma unroll
    for (int j = 0; j < T16_MAX_K * 2 / 1024; ++j)
      if (j * 1024 + lane * 16 < rowb) wr[j] = *reinterpret_cast<const g_u32x4_t*>(src + j * 1024 + lane * 16);
  };
  if constexpr (NX) {
    load_x();
    load_w();
  } else {
    load_w();
    load_x();
  }
  if constexpr (NX) {
    __shared__ float s_inv[G_MAX_M];
    __shared__ __align__(16) uint32_t s_nw[T16_MAX_K / 2];
    if (stat_wave) row_stats_finish(a.xsq, ptiles, M, K, a.xeps, rs, s_inv);
    if (tid < (K >> 1)) s_nw[tid] = nw_word;
    __syncthreads();   // every row's inv and the norm weight are in LDS
    float xinv[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) xinv[i] = s_inv[min(16 * i + c16, M - 1)];
#pragma unroll
    for (int s = 0; s < T16_KSW; ++s)
      if (ks0 + s < ks1) {
        const g_u32x4_t w8 = *reinterpret_cast<const g_u32x4_t*>(s_nw + 16 * (ks0 + s) + 4 * r4);
#pragma unroll
        for (int i = 0; i < TM; ++i) xr[s][i] = norm_fragment(xr[s][i], w8, xinv[i]);
      }
  }

  // weight row -> LDS: chunk q of row wv at (q & ~15) | ((q ^ wv) & 15)
#pragma unroll
  for (int j = 0; j < T16_MAX_K * 2 / 1024; ++j) {
    const int q = j * 64 + lane;
    if (q * 16 < rowb) *reinterpret_cast<g_u32x4_t*>(lds + wv * rowb + (((q & ~15) | ((q ^ wv) & 15)) << 4)) = wr[j];
  }
  __syncthreads();
  g_float4_t acc[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) acc[i] = g_float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < T16_KSW; ++s) {
    const int ks = ks0 + s;
    if (ks < ks1) {
      const int q = 4 * ks + r4;   // chunk of row c16 this lane's B fragment is
      const g_bf16x8_t b = __builtin_bit_cast(
          g_bf16x8_t, *reinterpret_cast<const g_u32x4_t*>(lds + c16 * rowb + (((q & ~15) | ((q ^ c16) & 15)) << 4)));
#pragma unroll
      for (int i = 0; i < TM; ++i)
        acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(g_bf16x8_t, xr[s][i]), b, acc[i], 0, 0, 0);
    }
  }
  __syncthreads();   // every wave is done with the weight tile: the LDS now takes the partial tiles
  float* red = reinterpret_cast<float*>(lds);   // [wave][TM * 16 rows][16 columns]
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) red[(wv * TM * 16 + 16 * i + 4 * r4 + e) * 16 + c16] = acc[i][e];
  __syncthreads();
  auto value = [&](int m, int n) __attribute__((always_inline)) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < T16_WAVES; ++w) v += red[(w * TM * 16 + m) * 16 + n];
    return v;
  };
  const float e_bias0 = a.bias != nullptr ? bf16_to_f32(r_b0) : 0.f, e_bias1 = a.bias != nullptr ? bf16_to_f32(r_b1) : 0.f;
  if constexpr (EPI == EPI_STORE) {
    if (elive && 16 * t + en < a.N) a.y[int64_t(em) * a.N + 16 * t + en] = f32_to_bf16(value(em, en) + e_bias0);
  } else if constexpr (EPI == EPI_RESNORM) {
    float ss = 0.f;
    if (tid < TM * 256) {
      const float r = round_bf16(bf16_to_f32(r_res) + round_bf16(value(em, en)));
      if (elive && 16 * t + en < a.N) a.res_out[int64_t(em) * a.N + 16 * t + en] = f32_to_bf16(r);
      ss = 16 * t + en < a.N ? r * r : 0.f;
    }
    // the row's 16 columns are lanes 16k .. 16k+15 of one wave
    ss += __shfl_xor(ss, 8, 64);
    ss += __shfl_xor(ss, 4, 64);
    ss += __shfl_xor(ss, 2, 64);
    ss += __shfl_xor(ss, 1, 64);
    if (elive && en == 0 && a.sumsq_out != nullptr) a.sumsq_out[int64_t(t) * G_NORM_ROWS + em] = ss;
  } else if constexpr (EPI == EPI_SILU) {
    const int half = a.N >> 1, oc = 8 * t + en;
    if (elive && oc < half) {
      const float gb = round_bf16(value(em, en)), ub = round_bf16(value(em, en + 8));
      a.y[int64_t(em) * half + oc] = f32_to_bf16(round_bf16(gb / (1.0f + expf(-gb))) * ub);
    }
  } else {   // EPI_ROPE
    if (elive) {
      const int tph = a.hd >> 4, head = t / tph, f = t - head * tph, hh = a.hd >> 1;
      const int d = 8 * f + en;
      const float xl = round_bf16(value(em, en) + e_bias0), xh = round_bf16(value(em, en + 8) + e_bias1);
      float lo = xl, hi = xh;
      if (head < a.nh + a.nkv) {
        const float e_cl = bf16_to_f32(r_cl), e_ch = bf16_to_f32(r_ch), e_sl = bf16_to_f32(r_sl), e_sh = bf16_to_f32(r_sh);
        lo = round_bf16(xl * e_cl) - round_bf16(xh * e_sl);
        hi = round_bf16(xh * e_ch) + round_bf16(xl * e_sh);
      }
      bf16_t* dst;
      bf16_t* cdst = nullptr;
      if (head < a.nh) {
        dst = a.q + (int64_t(em) * a.nh + head) * a.hd;
      } else if (head < a.nh + a.nkv) {
        const int kh = head - a.nh;
        dst = a.k + (int64_t(em) * a.nkv + kh) * a.hd;
        if (a.kc != nullptr) cdst = a.kc + (e_slot * a.nkv + kh) * a.hd;
      } else {
        const int vh = head - a.nh - a.nkv;
        dst = a.v + (int64_t(em) * a.nkv + vh) * a.hd;
        if (a.vc != nullptr) cdst = a.vc + (e_slot * a.nkv + vh) * a.hd;
      }
      const bf16_t blo = f32_to_bf16(lo), bhi = f32_to_bf16(hi);
      dst[d] = blo;
      dst[hh + d] = bhi;
      if (cdst != nullptr) {
        cdst[d] = blo;
        cdst[hh + d] = bhi;
      }
    }
  }
}

// h = round(w * round(r * inv)) for whole rows, inv exactly as the GEMMs compute it on load: one wave per
// row, 8 columns (16 bytes) per lane per step.
__global__ __launch_bounds__(64) void rms_norm_apply_kernel(const bf16_t* __restrict__ r, const float* __restrict__ sumsq,
                                                           const bf16_t* __restrict__ w, bf16_t* __restrict__ h, int N,
                                                           float eps) {
  const int m = blockIdx.x, lane = threadIdx.x;
  const float inv = rms_norm_row_inv(sumsq, (N + G_NORM_COLS - 1) / G_NORM_COLS, m, lane >> 4, N, eps);
  for (int c = 8 * lane; c < N; c += 8 * 64) {
    const g_u32x4_t rv = *reinterpret_cast<const g_u32x4_t*>(r + int64_t(m) * N + c);
    const g_u32x4_t wv = *reinterpret_cast<const g_u32x4_t*>(w + c);
    *reinterpret_cast<g_u32x4_t*>(h + int64_t(m) * N + c) = norm_fragment(rv, wv, inv);
  }
}

// ------------------------------------------------------------------------------------- tiled GEMM (M > 64)
// Prefill chunks, mixed steps and speculative verify batches: Y[M, N] = X[M, K] . W[N, K]^T for any M, bf16
// in, fp32 accumulate, with the STORE (+ bias), SILU, residual-add (RESNORM) and RoPE + K/V-write (ROPE)
// epilogues of the skinny kernels.
//   * BM x BN output tiles, NW waves in a WM x (NW / WM) grid, each a (16 FM) x (16 FN) block of
//     mfma_f32_16x16x32_bf16 tiles. Shapes: 256 x 256 (8 waves of 128 x 64, one workgroup per CU), 256 x 128
//     (8 of 64 x 64), 128 x 128 (8 of 64 x 32, or 4 of 64 x 64 two per CU) and 128 x 96 (8 of 32 x 48, the
//     tile plan below). A CU's vector memory path moves about 64 bytes per clock
//     (L2-resident loads into LDS or VGPRs alike); a 256 x 256 tile asks 7.8 bytes per kFLOP of it, half of
//     what the MFMA rate allows, a 128 x 128 tile 15.6 -- all of it -- so the plan takes the larger tile
//     whenever it alone fills the GPU.
//   * SILU: each wave's FN W-row tiles are FN / 2 gate tiles and the FN / 2 matching up tiles, so a lane
//     holds gate and up of the same outputs and finishes them in registers.
//   * K in 32-wide steps through a ring of S LDS stages (BM x 64 bytes of X rows + BN x 64 bytes of W rows
//     each), filled by buffer DMA (16 bytes per lane, each instruction 16 rows x 64 bytes; rows past M or N
//     and the empty stages past the slice read zeros through the buffer bounds, with no memory access). Each
//     64-byte row keeps its four 16-byte chunks XOR-swizzled by (row / 2) & 3, so the 16-lane fragment reads
//     are free of bank conflicts.
//   * Software pipeline, one barrier per step: step q waits for the wave's own DMA of stage q + 1 (vmcnt)
//     and meets the other waves at the barrier (which also retires the fragment reads of step q, freeing
//     stage q's slot), then issues the MFMAs of step q row by row with, between them, the DMA of stage
//     q + S into the freed slot and the fragment reads of step q + 1: A fragment i right after row i is
//     issued (an MFMA reads its sources at issue), the W fragments into the second of two sets. Fragment
//     reads are inline asm, so the compiler does not drain the DMA ring before them; the barrier's
//     lgkmcnt(0) is their wait.
//   * Workgroups map XCD-contiguously: XCD x runs a contiguous run of tiles (same W rows, successive X
//     rows), which share its L2.
//   * Few tiles, or long K with fewer tiles than CUs: K is cut into `splits` slices; each publishes its fp32
//     tile to the workspace (agent-scope stores, a per-tile arrival counter in the fixed counter region) and
//     the last to arrive sums the slices in slice order -- deterministic -- and runs the epilogue.
//   * Epilogues: STORE passes the fp32 tile through LDS in 64-row passes (RESNORM adds the residual's
//     pieces, ROPE rotates a head's low and high dims together); SILU stages only the bf16 outputs (one
//     pass). All threads then write row-contiguous 16-byte pieces. Roundings to bf16 use the hardware
//     conversion (round to nearest even); the SiLU is g * rcp(1 + exp2(-g log2 e)) on the transcendental
//     unit (within 2 ulp of fp32 division before the bf16 rounding).
constexpr int TG_BK = 32;
constexpr int TG_CROWS = 64;                  // output rows per STORE epilogue pass
constexpr int TG_MAX_SPLITS = 16;            // K slices at most
constexpr int TG_PLAN_SPLITS = 6;             // K slices the plan chooses at most
constexpr int TG_RSRC3 = 0x00020000;          // buffer resource word 3: raw (untyped) 32-bit accesses

// NW waves in a WM x (NW / WM) grid (wave w at m-block w % WM, n-block w / WM), each a (16 FM) x (16 FN) block.
template <int FM, int FN, int NW_, int WM_ = 2>
struct TgShape {
  static constexpr int NW = NW_, NT = 64 * NW, WM = WM_, WNW = NW / WM;   // waves, threads, waves along M / N
  static constexpr int BM = 16 * FM * WM, BN = 16 * FN * WNW;            // X rows, W rows of a tile
  static constexpr int WG_PER_CU = NW == 8 ? 1 : 2;
  static constexpr int S = 4;                                 // ring stages
  static constexpr int AROWS = BM * TG_BK * 2;                // bytes of the X rows of a stage
  static constexpr int STAGE = AROWS + BN * TG_BK * 2;
  static constexpr int CP = BN + 4;                           // floats per row of the staged STORE tile
  static constexpr int OCP = BN / 2 + 8;                      // bf16 per row of the staged SILU tile
  static constexpr int CBYTES = TG_CROWS * CP * 4 > BM * OCP * 2 ? TG_CROWS * CP * 4 : BM * OCP * 2;
  static constexpr int PART = BM * BN;                        // floats of one published slice of a tile
  // DMA instructions of a stage: 16-row groups, GA of X rows then GB of W rows. EVEN: wave w stages X groups
  // AJ w .. AJ w + AJ - 1 and W groups BJ w .. likewise. Otherwise instruction d of wave w stages group
  // d NW + w, and the waves left without one issue a no-traffic copy of zeros into a spare 1 KB (DUMMY), so
  // that every wave counts DMA copies per stage.
  static constexpr int GA = BM / 16, GB = BN / 16;
  static constexpr bool EVEN = GA % NW == 0 && GB % NW == 0;
  static constexpr int AJ = EVEN ? GA / NW : 0, BJ = EVEN ? GB / NW : 0;
  static constexpr int DMA = EVEN ? AJ + BJ : (GA + GB + NW - 1) / NW;
  static constexpr int DUMMY = S * STAGE;                     // spare bytes after the ring (not EVEN)
  static constexpr int RING = EVEN ? S * STAGE : S * STAGE + 1024;
  static constexpr int LDS0 = RING > CBYTES ? RING : CBYTES;
  // one workgroup per CU: more than half the CU's 160 KB
  static constexpr int LDS = WG_PER_CU == 1 && LDS0 <= 80 * 1024 ? 80 * 1024 + 16 : LDS0;
  static constexpr int MF = FM * FN;                          // MFMAs per wave per step
  static constexpr int RW = 16 * FM;                          // rows of a wave's block
  static_assert((RW % TG_CROWS == 0 || TG_CROWS % RW == 0) && (!EVEN || (AJ >= 1 && BJ >= 1)) && DMA <= MF &&
                    WG_PER_CU * LDS <= 160 * 1024,
                "tile shape");
};

struct TgArgs {
  const bf16_t* x;
  const bf16_t* w;
  const bf16_t* bias;
  bf16_t* y;
  int M, N, K;         // N: rows of w (SILU: gate rows then up rows)
  int tiles_m, tiles_n, splits, kps;   // kps: 32-wide k-steps per slice
  unsigned* cnt;
  float* part;
  const bf16_t* res;   // RESNORM epilogue: y = round(res + round(X W^T)) (the residual sum, no statistics)
  // ROPE epilogue (the ns_rope_qkv contract): per-row cos/sin tables [M, hd], outputs q [M, nh, hd],
  // k / v [M, nkv, hd], optional caches at slots[m]
  const bf16_t* cosb;
  const bf16_t* sinb;
  bf16_t *q, *k, *v, *kc, *vc;
  const int64_t* slots;
  int nh, nkv, hd;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tg_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, int(bytes), TG_RSRC3);
}
__device__ __forceinline__ uint32_t tg_lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}
// One 16-byte fragment read, no wait: the data is used only after the next barrier, whose lgkmcnt(0)
// covers it.
__device__ __forceinline__ void tg_read(uint32_t addr, g_u32x4_t& v) {
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr) : "memory");
}
// Workgroup barrier for LDS data (no wait for the wave's outstanding DMA, unlike __syncthreads)
__device__ __forceinline__ void tg_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// waitcnt immediate: at most n vector memory operations of this wave still outstanding
constexpr int tg_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | 0x70 | 0xF00; }
// Workgroup i of a grid of n -> position in the XCD-contiguous order (a bijection on [0, n)): XCD i % 8
// takes runs of n / 8 positions, the first n % 8 XCDs one more.
__host__ __device__ __forceinline__ int tg_xcd_order(int i, int n) {
  const int x = i & 7, j = i >> 3, q = n >> 3, r = n & 7;
  return x * q + (x < r ? x : r) + j;
}
// fp32 rounded to bf16 (nearest even, hardware conversion), kept in fp32
__device__ __forceinline__ float tg_round(float f) { return __uint_as_float(pack_bf16x2(f, 0.f) << 16); }
// W row staged at row r of a tile's W rows. STORE: BN tn + r. SILU: tile tn covers output columns
// (BN / 2) tn + [0, BN / 2); wave block c = r / (16 FN) stages its FN / 2 gate tiles, then the matching up tiles.
template <int EPI, int FN, int BN>
__device__ __forceinline__ int tg_wrow(int r, int tn, int half) {
  if constexpr (EPI == EPI_SILU) {
    const int c = r / (16 * FN), jj = (r / 16) % FN, rr = r % 16;
    const int oc = (BN / 2) * tn + 8 * FN * c + 16 * (jj % (FN / 2)) + rr;
    return jj < FN / 2 ? oc : half + oc;
  } else {
    return BN * tn + r;
  }
}

// ROPE epilogue item c of a staged output row (fp32 products, columns n0 .. of the tile): dims d0 .. d0+7 and
// d0 + hd/2 .. of one head of row gm. The values are rounded as the STORE epilogue stores them (bias added,
// then bf16), then rotated with the roundings of rope_qkv: lo = round(xl cl) - round(xh sl), hi = round(xh ch)
// + round(xl sh); value heads pass through. A tile holds whole heads (its width is a multiple of hd).
__device__ __forceinline__ void tg_rope_item(const TgArgs& a, const float* crow, int gm, int n0, int c) {
  const int gph = a.hd >> 4, hh = a.hd >> 1;   // 8-dim groups per half head
  const int ht = c / gph, d0 = 8 * (c - ht * gph), col = ht * a.hd + d0, gn = n0 + col;
  if (gm >= a.M || gn >= a.N) return;
  const int head = gn / a.hd;
  float xl[8], xh[8], lo[8], hi[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    xl[e] = crow[col + e];
    xh[e] = crow[col + hh + e];
  }
  if (a.bias != nullptr) {
    float bl[8], bh[8];
    load_bf16x8(a.bias + gn, bl);
    load_bf16x8(a.bias + gn + hh, bh);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xl[e] += bl[e];
      xh[e] += bh[e];
    }
  }
  if (head < a.nh + a.nkv) {
    float cl[8], ch[8], sl[8], sh[8];
    const bf16_t* cr = a.cosb + int64_t(gm) * a.hd + d0;
    const bf16_t* sr = a.sinb + int64_t(gm) * a.hd + d0;
    load_bf16x8(cr, cl);
    load_bf16x8(cr + hh, ch);
    load_bf16x8(sr, sl);
    load_bf16x8(sr + hh, sh);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float l = tg_round(xl[e]), h = tg_round(xh[e]);
      lo[e] = tg_round(l * cl[e]) - tg_round(h * sl[e]);
      hi[e] = tg_round(h * ch[e]) + tg_round(l * sh[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      lo[e] = xl[e];
      hi[e] = xh[e];
    }
  }
  bf16_t* dst;
  bf16_t* cdst = nullptr;
  if (head < a.nh) {
    dst = a.q + (int64_t(gm) * a.nh + head) * a.hd;
  } else if (head < a.nh + a.nkv) {
    const int kh = head - a.nh;
    dst = a.k + (int64_t(gm) * a.nkv + kh) * a.hd;
    if (a.kc != nullptr) cdst = a.kc + (a.slots[gm] * a.nkv + kh) * a.hd;
  } else {
    const int vh = head - a.nh - a.nkv;
    dst = a.v + (int64_t(gm) * a.nkv + vh) * a.hd;
    if (a.vc != nullptr) cdst = a.vc + (a.slots[gm] * a.nkv + vh) * a.hd;
  }
  store_bf16x8(dst + d0, lo);
  store_bf16x8(dst + d0 + hh, hi);
  if (cdst != nullptr) {
    store_bf16x8(cdst + d0, lo);
    store_bf16x8(cdst + d0 + hh, hi);
  }
}

template <int EPI, int FM, int FN, int NW, int WM>
__global__ __launch_bounds__((TgShape<FM, FN, NW, WM>::NT), (TgShape<FM, FN, NW, WM>::WG_PER_CU)) void tiled_gemm_kernel(
    TgArgs a) {
  using SH = TgShape<FM, FN, NW, WM>;
  static_assert(EPI != EPI_SILU || (WM == 2 && FN % 4 == 0), "the SiLU epilogue pairs gate and up tiles of a 2-row wave grid");
  constexpr int BM = SH::BM, BN = SH::BN, NT = SH::NT, S = SH::S;
  __shared__ __align__(16) unsigned char lds[SH::LDS];
  __shared__ unsigned s_last;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int tiles = a.tiles_m * a.tiles_n, grid = tiles * a.splits;
  const int bid = tg_xcd_order(int(blockIdx.x), grid);
  const int split = bid / tiles, t = bid - split * tiles;
  const int tm = t % a.tiles_m, tn = t / a.tiles_m;
  const int m0 = tm * BM;
  const int K = a.K, M = a.M, N = a.N, half = N >> 1;
  const int kb = split * a.kps, nk = min(a.kps, K / TG_BK - kb);

  // DMA lanes: X instruction j of wave w stages rows 16 (AJ w + j) + l / 4, W instruction j rows
  // 16 (BJ w + j) + l / 4; slot l % 4 of a row holds chunk (l % 4) ^ ((row / 2) & 3). Row offsets go in the
  // per-lane offset, so rows past M / N fail the bounds.
  constexpr int AJ = SH::AJ, BJ = SH::BJ, GA = SH::GA, GB = SH::GB;
  uint32_t voa[AJ > 0 ? AJ : 1], vob[BJ > 0 ? BJ : 1], vo[SH::DMA];
  const int wu = __builtin_amdgcn_readfirstlane(w);   // the wave index as a scalar (uniform branches)
  if constexpr (SH::EVEN) {
#pragma unroll
    for (int j = 0; j < AJ; ++j) {
      const int r = 16 * (AJ * w + j) + (l >> 2), c = (l & 3) ^ ((r >> 1) & 3);
      voa[j] = (uint32_t(m0 + r) * uint32_t(K) + uint32_t(8 * c)) * 2u;
    }
#pragma unroll
    for (int j = 0; j < BJ; ++j) {
      const int r = 16 * (BJ * w + j) + (l >> 2), c = (l & 3) ^ ((r >> 1) & 3);
      vob[j] = (uint32_t(tg_wrow<EPI, FN, BN>(r, tn, half)) * uint32_t(K) + uint32_t(8 * c)) * 2u;
    }
  } else {
#pragma unroll
    for (int d = 0; d < SH::DMA; ++d) {
      const int gx = d * NW + wu, gw = gx - GA;
      const int r = 16 * (gx < GA ? gx : gw) + (l >> 2), c = (l & 3) ^ ((r >> 1) & 3);
      const uint32_t row = gx < GA ? uint32_t(m0 + r) : gw < GB ? uint32_t(tg_wrow<EPI, FN, BN>(r, tn, half)) : 0u;
      vo[d] = (row * uint32_t(K) + uint32_t(8 * c)) * 2u;
    }
  }
  const __amdgpu_buffer_rsrc_t xr = tg_rsrc(a.x, uint32_t(M) * uint32_t(K) * 2u), xnone = tg_rsrc(a.x, 0u);
  const __amdgpu_buffer_rsrc_t wr = tg_rsrc(a.w, uint32_t(N) * uint32_t(K) * 2u), wnone = tg_rsrc(a.w, 0u);
  // DMA instruction d (X rows for d < AJ, then W rows) of stage q of the slice (past nk: zeros, no traffic)
  auto dma = [&](int q, int d) __attribute__((always_inline)) {
    const bool live = q < nk;
    const int soff = __builtin_amdgcn_readfirstlane(live ? (kb + q) * TG_BK * 2 : 0);   // uniform: an SGPR
    unsigned char* st = lds + (q % S) * SH::STAGE;
    if constexpr (!SH::EVEN) {
      const int gx = d * NW + wu, gw = gx - GA;
      if (gx < GA)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? xr : xnone,
                                                 (__attribute__((address_space(3))) void*)(st + 16 * gx * 64), 16,
                                                 int(vo[d]), soff, 0, 0);
      else if (gw < GB)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            live ? wr : wnone, (__attribute__((address_space(3))) void*)(st + SH::AROWS + 16 * gw * 64), 16,
            int(vo[d]), soff, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xnone, (__attribute__((address_space(3))) void*)(lds + SH::DUMMY),
                                                 16, 0, 0, 0, 0);
    } else if (d < AJ) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? xr : xnone,
                                               (__attribute__((address_space(3))) void*)(st + 16 * (AJ * w + d) * 64),
                                               16, int(voa[d]), soff, 0, 0);
    } else {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          live ? wr : wnone, (__attribute__((address_space(3))) void*)(st + SH::AROWS + 16 * (BJ * w + d - AJ) * 64), 16,
          int(vob[d - AJ]), soff, 0, 0);
    }
  };

  // fragment offsets within a stage: lane -> row l % 16 of the 16-row tile, 16-byte chunk l / 16; the swizzle
  // of rows 16 i + l % 16 does not depend on i, so fragment i sits 1024 i bytes further
  const int wm = w % WM, wn = w / WM;
  const int ra = 16 * FM * wm + (l & 15), rb = 16 * FN * wn + (l & 15);
  const uint32_t foa = uint32_t(ra * 64 + 16 * ((l >> 4) ^ ((ra >> 1) & 3)));
  const uint32_t fob = uint32_t(SH::AROWS + rb * 64 + 16 * ((l >> 4) ^ ((rb >> 1) & 3)));
  g_float4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = g_float4_t{0.f, 0.f, 0.f, 0.f};
  const uint32_t lds0 = tg_lds_addr(lds);

  // RESNORM: the thread's residual pieces for the epilogue's items (item k of 64-row pass p: it = tid + k NT,
  // row it / (BN / 8), 8 columns it % (BN / 8)), loaded before the K loop so their latency hides under it,
  // when they fit in 8 registers of 16 bytes (else each item loads its own). Addresses are clamped into the
  // residual, so the loads are unconditional; pieces past M or N are never used.
  constexpr int RIPR = BN / 8, RIPT = (TG_CROWS * RIPR + NT - 1) / NT;   // items per thread and pass, at most
  static_assert(TG_CROWS * RIPR % 64 == 0 && TG_CROWS * (BN / 16) % 64 == 0, "epilogue items: whole waves");
  constexpr int RPRE = EPI == EPI_RESNORM && BM / TG_CROWS * RIPT <= 8 ? BM / TG_CROWS * RIPT : 0;
  g_u32x4_t rres[RPRE > 0 ? RPRE : 1];
  if constexpr (RPRE > 0) {
#pragma unroll
    for (int u = 0; u < RPRE; ++u) {
      const int it = tid + (u % RIPT) * NT;
      const int gm = min(m0 + TG_CROWS * (u / RIPT) + it / RIPR, M - 1), gn = min(BN * tn + 8 * (it % RIPR), N - 8);
      rres[u] = *reinterpret_cast<const g_u32x4_t*>(a.res + int64_t(gm) * N + gn);
    }
  }

  // Step q: the MFMAs of step q, row by row, from A and Bc; between them the DMA of stage q + S, and the
  // reads of step q + 1: A[i] as soon as row i is issued, Bn spread over the step.
  g_u32x4_t A[FM], B0[FN], B1[FN];
  auto step = [&](int q, g_u32x4_t (&Bc)[FN], g_u32x4_t (&Bn)[FN]) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(tg_vmcnt(SH::DMA * (S - 2)));   // this wave's loads of stage q + 1 are done
    tg_barrier();   // ... and every wave's; every read of step q has landed, so stage q's slot is free
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t sn = lds0 + uint32_t(((q + 1) % S) * SH::STAGE);
    constexpr int EVERY = SH::MF / FN;
#pragma unroll
    for (int u = 0; u < SH::MF; ++u) {
      const int i = u / FN, j = u % FN;
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(g_bf16x8_t, A[i]),
                                                         __builtin_bit_cast(g_bf16x8_t, Bc[j]), acc[i][j], 0, 0, 0);
      if (u < SH::DMA) dma(q + S, u);
      if (j == FN - 1) tg_read(sn + foa + 1024u * i, A[i]);
      if (u % EVERY == EVERY / 2) tg_read(sn + fob + 1024u * (u / EVERY), Bn[u / EVERY]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

#pragma unroll
  for (int q = 0; q < S; ++q)
#pragma unroll
    for (int d = 0; d < SH::DMA; ++d) dma(q, d);
  __builtin_amdgcn_s_waitcnt(tg_vmcnt(SH::DMA * (S - 1)));   // stage 0
  tg_barrier();
#pragma unroll
  for (int i = 0; i < FM; ++i) tg_read(lds0 + foa + 1024u * i, A[i]);
#pragma unroll
  for (int j = 0; j < FN; ++j) tg_read(lds0 + fob + 1024u * j, B0[j]);
  for (int q = 0;; q += 2) {
    step(q, B0, B1);
    if (q + 1 >= nk) break;
    step(q + 1, B1, B0);
    if (q + 2 >= nk) break;
  }
  __builtin_amdgcn_s_waitcnt(tg_vmcnt(0));
  tg_barrier();

  // ---- K slices: publish, count, and the last slice sums them in slice order
  if (a.splits > 1) {
    float* mine = a.part + (int64_t(t) * a.splits + split) * SH::PART;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const g_float4_t v = acc[i][j];
        publish_store16(mine + (int64_t(i * FN + j) * NT + tid) * 4,
                        pub_u32x4_t{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                                    __float_as_uint(v[3])});
      }
    publish_complete();
    __syncthreads();
    if (tid == 0) {
      const unsigned prev = publish_count(a.cnt + t);
      const bool last = prev == unsigned(a.splits - 1);
      if (last) publish_reset(a.cnt + t);
      s_last = last;
    }
    __syncthreads();
    if (s_last == 0u) return;
    acquire_published();
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = g_float4_t{0.f, 0.f, 0.f, 0.f};
    const float* base = a.part + int64_t(t) * a.splits * SH::PART;
    constexpr int FB = SH::MF < 16 ? SH::MF : 16;   // partial fragments per round trip
    for (int s = 0; s < a.splits; ++s) {
#pragma unroll
      for (int f0 = 0; f0 < SH::MF; f0 += FB) {
        pub_u32x4_t v[FB];
#pragma unroll
        for (int e = 0; e < FB; ++e)
          v[e] = publish_load16(base + int64_t(s) * SH::PART + (int64_t(f0 + e) * NT + tid) * 4);
#pragma unroll
        for (int e = 0; e < FB; ++e)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[(f0 + e) / FN][(f0 + e) % FN][r] += __uint_as_float(v[e][r]);
      }
    }
  }

  // Lane layout of acc[i][j]: column 16 FN wn + 16 j + l % 16 of the tile, rows 16 FM wm + 16 i + 4 (l / 16) + r.
  if constexpr (EPI != EPI_SILU) {
    // the fp32 tile through LDS in passes of 64 rows (pass p: the waves with wm == p / (FM / 4), their
    // m-tiles 4 (p % (FM / 4)) .. + 3), then items (row m, 8 columns) of 16 bytes (RESNORM: plus the
    // residual's 8); ROPE: items (row m, 8 dims of a head's low half and the matching 8 of its high half)
    float* C = reinterpret_cast<float*>(lds);
    constexpr int CP = SH::CP, PASSES = BM / TG_CROWS, IPR = EPI == EPI_ROPE ? BN / 16 : BN / 8;
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      if constexpr (SH::RW >= TG_CROWS) {   // a wave block spans PW passes
        constexpr int PW = SH::RW / TG_CROWS;
        if (wm == p / PW) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
              for (int r = 0; r < 4; ++r)
                C[(16 * i + 4 * (l >> 4) + r) * CP + 16 * FN * wn + 16 * j + (l & 15)] = acc[4 * (p % PW) + i][j][r];
        }
      } else {   // a pass holds WPP wave blocks
        constexpr int WPP = TG_CROWS / SH::RW;
        if (wm / WPP == p) {
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
              for (int r = 0; r < 4; ++r)
                C[(SH::RW * (wm % WPP) + 16 * i + 4 * (l >> 4) + r) * CP + 16 * FN * wn + 16 * j + (l & 15)] =
                    acc[i][j][r];
        }
      }
      tg_barrier();   // LDS only: the global stores of the previous pass need not land first
      const int mb = m0 + TG_CROWS * p;
      constexpr int IPT = (TG_CROWS * IPR + NT - 1) / NT;   // items per thread and pass, at most
#pragma unroll
      for (int k = 0; k < IPT; ++k) {
        const int it = tid + k * NT, m = it / IPR, c8 = it % IPR, gm = mb + m, gn = BN * tn + 8 * c8;
        if (TG_CROWS * IPR % NT != 0 && it >= TG_CROWS * IPR) continue;   // whole waves (checked above)
        if constexpr (EPI == EPI_ROPE) {
          tg_rope_item(a, C + m * CP, gm, BN * tn, c8);
          continue;
        }
        if (gm >= M || gn >= N) continue;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = C[m * CP + 8 * c8 + e];
        if (a.bias != nullptr) {
          if ((N & 7) == 0) {
            float b[8];
            load_bf16x8(a.bias + gn, b);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] += b[e];
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] += gn + e < N ? bf16_to_f32(a.bias[gn + e]) : 0.f;
          }
        }
        if constexpr (EPI == EPI_RESNORM) {   // N % 8 == 0 (checked by the entry point)
          g_u32x4_t u;
          if constexpr (RPRE > 0)
            u = rres[p * IPT + k];
          else
            u = *reinterpret_cast<const g_u32x4_t*>(a.res + int64_t(gm) * N + gn);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[2 * e] = __uint_as_float(u[e] << 16) + tg_round(v[2 * e]);
            v[2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u) + tg_round(v[2 * e + 1]);
          }
        }
        bf16_t* dst = a.y + int64_t(gm) * N + gn;
        if ((N & 7) == 0) {
          store_bf16x8(dst, v);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (gn + e < N) dst[e] = f32_to_bf16(v[e]);
        }
      }
      if (p + 1 < PASSES) tg_barrier();
    }
  } else {
    // SILU: gate acc[i][j], up acc[i][j + FN / 2] -> output column 8 FN wn + 16 j + l % 16 of the tile's
    // BN / 2; the bf16 outputs go through LDS ([BM][OCP]) in one pass, then items (row m, 8 columns)
    bf16_t* O = reinterpret_cast<bf16_t*>(lds);
    constexpr int OCP = SH::OCP, IPR = BN / 16;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN / 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float gb = tg_round(acc[i][j][r]), ub = tg_round(acc[i][j + FN / 2][r]);
          const float sg = gb * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(gb * -1.44269504088896341f));
          O[(16 * FM * wm + 16 * i + 4 * (l >> 4) + r) * OCP + 8 * FN * wn + 16 * j + (l & 15)] =
              bf16_t(pack_bf16x2(tg_round(sg) * ub, 0.f));
        }
    tg_barrier();
#pragma unroll 2
    for (int it = tid; it < BM * IPR; it += NT) {
      const int m = it / IPR, c8 = it % IPR, gm = m0 + m, gn = (BN / 2) * tn + 8 * c8;
      if (gm >= M || gn >= half) continue;
      const g_u32x4_t v = *reinterpret_cast<const g_u32x4_t*>(O + m * OCP + 8 * c8);
      bf16_t* dst = a.y + int64_t(gm) * half + gn;
      if ((half & 7) == 0) {
        *reinterpret_cast<g_u32x4_t*>(dst) = v;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (gn + e < half) dst[e] = bf16_t(v[e >> 1] >> (16 * (e & 1)));
      }
    }
  }
}

// ------------------------------------------------------------------------------------------- host side
// Workgroups that stream at once: one per CU of the MI355X. The plans depend on the shape alone (no
// environment or device query), so a given call always sums in the same order and gives the same bits.
constexpr int target_workgroups() { return 256; }

struct Plan {
  int tiles, chunks, whole, ks, grid;
  size_t cnt_off, part_off, bytes;
};

static size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// tiles: 64-row tiles of the weight (SILU: 32 gate + 32 up rows, i.e. 32 output columns).
// Many tiles: one workgroup per tile. Fewer than twice the target: the target's worth of whole tiles,
// and the rest cut into K slices so that the last round is spread over the GPU too. Fewer tiles than
// the target: every tile cut into up to `chunks` slices. At most G_MAXC slices per tile, so the last
// slice loads all partials in one round trip (the down projection: 8 slices of 24 tiles, 12.5 us, against
// 13.4 us with 10 slices and 14.2 with 6).
static Plan make_plan(int tiles, int K) {
  Plan p;
  const int T = target_workgroups();
  p.tiles = tiles;
  p.chunks = (K + G_KC - 1) / G_KC;
  if (tiles >= 2 * T) {
    p.whole = tiles;
    p.ks = 1;
  } else {
    p.whole = tiles >= T ? T : 0;
    const int rest = tiles - p.whole;
    const int ks = rest > 0 ? T / rest : 1;   // the sliced round fits the target (never a partial extra wave)
    p.ks = ks < 1 ? 1 : (ks > p.chunks ? p.chunks : ks);
    if (p.ks > G_MAXC) p.ks = G_MAXC;   // the last slice loads every partial in one round trip
  }
  if (p.ks == 1) p.whole = tiles;
  p.grid = p.whole + (tiles - p.whole) * p.ks;
  p.cnt_off = 0;
  p.part_off = G_CNT_BYTES;   // fixed: every plan finds the counters at the same, otherwise unused bytes
  p.bytes = p.part_off + align256(sizeof(float) * size_t(tiles - p.whole) * p.ks * G_MAX_M * 64);
  return p;
}

// max_m: G_MAX_M for the entry points that only have skinny kernels, INT_MAX where M > 64 goes tiled
static int check_common(const void* x, const void* w, int M, int N, int K, int dtype, int max_m = G_MAX_M) {
  NS_REQUIRE(dtype == NS_DTYPE_BF16, "skinny gemm: bf16 only (dtype %d)", dtype);
  NS_REQUIRE(M >= 1 && M <= max_m, "skinny gemm: M=%d outside [1, %d]", M, max_m);
  NS_REQUIRE(N >= 1 && K >= 32 && K % 32 == 0, "skinny gemm: N=%d K=%d (K must be a positive multiple of 32)", N, K);
  NS_REQUIRE(x != nullptr && w != nullptr, "skinny gemm: null operand");
  NS_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0,
             "skinny gemm: operands must be 16-byte aligned");
  return NS_OK;
}

static int bind_workspace(GemmArgs& a, const Plan& p, void* ws, size_t ws_bytes) {
  NS_REQUIRE(p.tiles <= G_MAX_TILES, "skinny gemm: %d tiles exceed the %d the workspace counters cover", p.tiles,
             G_MAX_TILES);
  if (ws == nullptr || ws_bytes < p.bytes || reinterpret_cast<uintptr_t>(ws) % 256 != 0) {
    set_error("skinny gemm: a zero-initialised, 256-byte aligned workspace of %zu bytes is needed, got %zu", p.bytes,
              ws == nullptr ? size_t(0) : ws_bytes);
    return NS_E_WORKSPACE;
  }
  unsigned char* b = static_cast<unsigned char*>(ws);
  a.cnt = reinterpret_cast<unsigned*>(b + p.cnt_off);
  const size_t n_ctr = size_t(p.tiles - p.whole) * size_t(a.mblocks > 1 ? a.mblocks : 1);
  a.cstride = ws_counter_stride(n_ctr, size_t(G_MAX_TILES + 1));
  NS_REQUIRE(n_ctr * a.cstride <= size_t(G_MAX_TILES + 1), "skinny gemm: %zu split tiles exceed the %d counters", n_ctr,
             G_MAX_TILES + 1);
  a.part = reinterpret_cast<float*>(b + p.part_off);
  a.tiles = p.tiles;
  a.chunks = p.chunks;
  a.whole = p.whole;
  a.ks = p.ks;
  return NS_OK;
}

template <int EPI, bool NX>
static void launch_nx(const GemmArgs& a, hipStream_t st) {
  const dim3 grid(unsigned((a.whole + (a.tiles - a.whole) * a.ks) * (a.mblocks > 1 ? a.mblocks : 1))),
      block(G_WAVES * 64);
  if (a.M <= 16)
    hipLaunchKernelGGL((skinny_gemm_kernel<1, EPI, NX>), grid, block, 0, st, a);
  else if (a.M <= 32)
    hipLaunchKernelGGL((skinny_gemm_kernel<2, EPI, NX>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((skinny_gemm_kernel<4, EPI, NX>), grid, block, 0, st, a);
}
// The tile-16 kernel takes projections with K <= 2048 and at most T16_MAX_TILES tiles (two per CU); wider
// ones stream better through the 64-row tiles above.
constexpr int T16_MAX_TILES = 512;
static bool tile16_fits(int K, int tiles) { return K <= T16_MAX_K && tiles <= T16_MAX_TILES; }

// Token split: with at most T16_MAX_TILES workgroups in all, each tile's tokens are cut into blocks of 16,
// one workgroup each.
static bool t16_token_split(int M, int tiles) {
  return M > 16 && tiles * ((M + 15) / 16) <= T16_MAX_TILES;
}
// Above 64 rows a plain input on a projection the tile-16 kernel takes (K <= 2048, at most T16_MAX_TILES
// tiles) runs it token-split (16-token blocks, the blocks of a tile re-reading its weights from L2), in as
// many rounds as it needs, up to T16_LARGE_M rows (speculative verify batches); larger chunks go to the
// tiled kernel.
constexpr int T16_LARGE_M = 192;
constexpr int t16_max_m() { return T16_LARGE_M; }
static bool t16_large_m(int M, int K, int tiles, bool normed) {
  return M > G_MAX_M && M <= (normed ? G_NORM_ROWS : t16_max_m()) && tile16_fits(K, tiles);
}
template <int EPI, bool NX>
static void launch_t16_nx(const GemmArgs& a, int tiles, hipStream_t st) {
  const dim3 block{unsigned(T16_WAVES * 64)};
  if (a.M > G_MAX_M || t16_token_split(a.M, tiles)) {
    hipLaunchKernelGGL((tile16_gemm_kernel<1, EPI, NX>), dim3(unsigned(tiles * ((a.M + 15) / 16))), block, 0, st, a);
    return;
  }
  const dim3 grid{unsigned(tiles)};
  if (a.M <= 16)
    hipLaunchKernelGGL((tile16_gemm_kernel<1, EPI, NX>), grid, block, 0, st, a);
  else if (a.M <= 32)
    hipLaunchKernelGGL((tile16_gemm_kernel<2, EPI, NX>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((tile16_gemm_kernel<4, EPI, NX>), grid, block, 0, st, a);
}
template <int EPI>
static int launch_t16(const GemmArgs& a, int tiles, hipStream_t st) {
  if constexpr (EPI == EPI_RESNORM) {
    launch_t16_nx<EPI, false>(a, tiles, st);
  } else {
    if (a.xsq != nullptr)
      launch_t16_nx<EPI, true>(a, tiles, st);
    else
      launch_t16_nx<EPI, false>(a, tiles, st);
  }
  return check_launch("skinny_gemm(tile16)");
}

// The persistent kernel takes wide STORE projections without bias: M <= 32, K <= 2048, at least four tiles
// per CU (the LM head).
static bool persist_fits(int M, int K, int tiles, const void* bias) {
  return M <= 32 && K <= 2048 && tiles >= 4 * target_workgroups() && bias == nullptr;
}
template <bool NX, int CP, bool AM>
static void launch_persist_cp(const GemmArgs& a, int grid, hipStream_t st) {
  if (a.M <= 16)
    hipLaunchKernelGGL((persist_gemm_kernel<1, NX, CP, AM>), dim3(unsigned(grid)), dim3(G_WAVES * 64), 0, st, a);
  else
    hipLaunchKernelGGL((persist_gemm_kernel<2, NX, CP, AM>), dim3(unsigned(grid)), dim3(G_WAVES * 64), 0, st, a);
}
template <bool NX, bool AM>
static void launch_persist_nx(const GemmArgs& a, int grid, hipStream_t st) {
  switch ((a.chunks + 1) & ~1) {
    case 2: launch_persist_cp<NX, 2, AM>(a, grid, st); break;
    case 4: launch_persist_cp<NX, 4, AM>(a, grid, st); break;
    case 6: launch_persist_cp<NX, 6, AM>(a, grid, st); break;
    default: launch_persist_cp<NX, 8, AM>(a, grid, st); break;
  }
}
// Two resident workgroups per CU, each with the same number of tiles (the last one fewer). a.am_out set:
// the argmax fused.
static int launch_persist(GemmArgs a, int tiles, hipStream_t st) {
  a.tiles = tiles;
  a.chunks = (a.K + G_KC - 1) / G_KC;
  const int T = 2 * target_workgroups();
  const int per = (tiles + T - 1) / T;
  const int grid = (tiles + per - 1) / per;
  if (a.am_out != nullptr) {
    if (a.xsq != nullptr)
      launch_persist_nx<true, true>(a, grid, st);
    else
      launch_persist_nx<false, true>(a, grid, st);
  } else {
    if (a.xsq != nullptr)
      launch_persist_nx<true, false>(a, grid, st);
    else
      launch_persist_nx<false, false>(a, grid, st);
  }
  return check_launch("gemm(persistent)");
}

template <int EPI>
static int launch(const GemmArgs& a, hipStream_t st) {
  if constexpr (EPI == EPI_RESNORM) {
    launch_nx<EPI, false>(a, st);
  } else {
    if (a.xsq != nullptr)
      launch_nx<EPI, true>(a, st);
    else
      launch_nx<EPI, false>(a, st);
  }
  return check_launch("skinny_gemm");
}

// Optional normalised input (x holds r; see the file comment): sumsq NULL = plain x.
static int bind_xnorm(GemmArgs& a, const float* x_sumsq, const void* x_norm_w, float x_eps) {
  NS_REQUIRE(x_sumsq == nullptr || (x_norm_w != nullptr && reinterpret_cast<uintptr_t>(x_norm_w) % 16 == 0 &&
                                     a.K % 8 == 0 && a.K <= G_NX_MAX_K),
             "skinny gemm: a normalised input needs a 16-byte aligned norm weight, K %% 8 == 0 and K <= %d (K=%d)",
             G_NX_MAX_K, a.K);
  a.xsq = x_sumsq;
  a.xnw = static_cast<const bf16_t*>(x_norm_w);
  a.xeps = x_eps;
  return NS_OK;
}

// ---- tiled GEMM plan and launch (M > 64)
enum TgTile { TG_SMALL = 0, TG_BIG = 1, TG_TALL = 2, TG_SMALL8 = 3, TG_N96 = 4 };
struct TgPlan {
  int shape;   // TgTile: 128 x 128 (4 waves, two per CU), 256 x 256 or 256 x 128 (8 waves, one per CU)
  int tiles_m, tiles_n, splits, kps;
  size_t bytes;   // workspace (0: no K slices)
};
using TgBig = TgShape<8, 4, 8>;
using TgSmall = TgShape<4, 4, 4>;
using TgTall = TgShape<4, 4, 8, 4>;   // 256 X rows x 128 W rows: waves in a 4 x 2 grid of 64 x 64 blocks
using TgSmall8 = TgShape<4, 2, 8, 2>; // 128 x 128 with 8 waves in a 2 x 4 grid of 64 x 32 blocks
using TgN96 = TgShape<2, 3, 8, 4>;    // 128 x 96 with 8 waves in a 4 x 2 grid of 32 x 48 blocks
static_assert(TgSmall8::BM == TgSmall::BM && TgSmall8::BN == TgSmall::BN, "same tile, twice the waves");
static int tg_bm(int shape) { return shape == TG_BIG ? TgBig::BM : shape == TG_TALL ? TgTall::BM : TgSmall::BM; }
static int tg_bn(int shape) {
  return shape == TG_BIG ? TgBig::BN : shape == TG_TALL ? TgTall::BN : shape == TG_N96 ? TgN96::BN : TgSmall::BN;
}
static void tg_tiles(TgPlan& p, int M, int N, bool silu) {
  const int bm = tg_bm(p.shape), bn = tg_bn(p.shape);
  p.tiles_m = (M + bm - 1) / bm;
  p.tiles_n = silu ? (N / 2 + bn / 2 - 1) / (bn / 2) : (N + bn - 1) / bn;
}
// 256 x 256 tiles (one workgroup per CU) when there is one for every CU; otherwise 128 x 128 tiles (two per
// CU), unsliced: K = 1536 shapes were never faster sliced. Long K (at least 128 steps, a STORE epilogue) with
// fewer tiles than CUs: one round of at most one workgroup per CU -- a CU that runs two workgroups of a
// launch finishes last, at about twice the time of the others -- either 128 x 128 tiles in at most
// TG_PLAN_SPLITS K slices or 256 x 128 tiles in at most 4 (the last slice's merge reads every partial tile),
// whichever fills more CUs, the 256 x 128 tiles on a tie (they move 25 % fewer bytes per flop through the
// CU's load path). Each slice holds at least eight 32-wide steps. Measured, 1536 x 8960 weights (us):
//   rows                    256   512   768  1024  1280  1552  2048
//   128^2, slices to fill   36.0  40.6  50.0  65.2  68.8  83.5 109.6   (6, 5, 3, 2, 2, 1 (3 at 1552), 1)
//   256 x 128, to fill        -     -     -   63.7  69.9  76.7  96.0   (4, 4, 3, 2 slices)
//   the earlier plan (128^2 slices for two per CU)  36.0  60.6  57.6  63.9  73.0  83.0 116.8
static inline void tg_plan_override(TgPlan&, int, int, bool, int&) {}
static int tg_fill_splits(int tiles, int max_splits, int steps) {
  int s = target_workgroups() / tiles;
  if (s > max_splits) s = max_splits;
  if (s > steps / 8) s = steps / 8;
  return s < 1 ? 1 : s;
}
static TgPlan tg_plan(int M, int N, int K, int epi) {
  const bool silu = epi == EPI_SILU;
  TgPlan p;
  const int T = target_workgroups(), steps = K / TG_BK;
  p.shape = TG_BIG;
  tg_tiles(p, M, N, silu);
  if (int64_t(p.tiles_m) * p.tiles_n < T) {
    p.shape = TG_SMALL;
    tg_tiles(p, M, N, silu);
  }
  int tiles = p.tiles_m * p.tiles_n;
  int splits = 1;
  if (steps >= 128 && !silu && p.shape == TG_SMALL && tiles < T) {
    const int s_small = tg_fill_splits(tiles, TG_PLAN_SPLITS, steps);
    TgPlan t = p;
    t.shape = TG_TALL;
    tg_tiles(t, M, N, silu);
    const int tt = t.tiles_m * t.tiles_n, s_tall = tt < T ? tg_fill_splits(tt, 4, steps) : 1;
    if (tt < T && tt * s_tall >= tiles * s_small) {
      p = t;
      splits = s_tall;
    } else {
      splits = s_small;
    }
  }
  // a 128 x 128 STORE plan that fits one workgroup per CU runs the 8-wave tile: two waves per SIMD instead of
  // one, so one wave's LDS reads and barrier overlap the other's products (1552 x 1536 x 1536: 18.8 -> 17.4 us;
  // 512 x 1536 x 8960 in 5 slices: 40.4 -> 38.0)
  if (!silu && p.shape == TG_SMALL && tiles * splits <= T) p.shape = TG_SMALL8;
  // ... and an unsliced one (no RoPE: its heads are 64 or 128 wide) that leaves CUs idle takes 128 x 96 tiles
  // (8 waves of 32 x 48) when they too fit one round and cover N exactly: more CUs, each SIMD with three
  // quarters of the work (1552 x 1536 x 1536: 19.1 -> 18.7 us, 20.0 -> 19.3 with the residual add; 300 rows
  // 18.8 -> 17.2; 1552 x 1003 x 896, a partial last column tile: 14.3 -> 14.6, hence N % 96 == 0)
  if ((epi == EPI_STORE || epi == EPI_RESNORM) && p.shape == TG_SMALL8 && splits == 1 && N % TgN96::BN == 0) {
    TgPlan t = p;
    t.shape = TG_N96;
    tg_tiles(t, M, N, false);
    if (t.tiles_m * t.tiles_n <= T) p = t;
  }
  tg_plan_override(p, M, N, silu, splits);
  tiles = p.tiles_m * p.tiles_n;
  if (splits > TG_MAX_SPLITS) splits = TG_MAX_SPLITS;
  if (splits > steps) splits = steps;
  if (splits < 1) splits = 1;
  p.kps = (steps + splits - 1) / splits;
  p.splits = (steps + p.kps - 1) / p.kps;   // every slice non-empty
  const int part = tg_bm(p.shape) * tg_bn(p.shape);
  p.bytes = p.splits > 1 ? G_CNT_BYTES + align256(sizeof(float) * size_t(tiles) * p.splits * part) : 0;
  return p;
}
static TgArgs tg_args(const void* x, const void* w, const void* bias, void* y, int M, int N, int K) {
  TgArgs a{};
  a.x = static_cast<const bf16_t*>(x);
  a.w = static_cast<const bf16_t*>(w);
  a.bias = static_cast<const bf16_t*>(bias);
  a.y = static_cast<bf16_t*>(y);
  a.M = M;
  a.N = N;
  a.K = K;
  return a;
}
// a: operands, shape and (ROPE) the epilogue's fields; the plan fills the rest
template <int EPI>
static int launch_tiled(TgArgs a, void* ws, size_t ws_bytes, hipStream_t st) {
  const int M = a.M, N = a.N, K = a.K;
  // 32-bit buffer offsets: every row offset of X and W (plus a tile's overhang) must fit
  NS_REQUIRE((int64_t(M) + 256) * K * 2 < (int64_t(1) << 31) && (int64_t(N) + 256) * K * 2 < (int64_t(1) << 31),
             "gemm: X [%d, %d] or W [%d, %d] too large for 32-bit buffer offsets", M, K, N, K);
  const TgPlan p = tg_plan(M, N, K, EPI);
  NS_REQUIRE(EPI != EPI_ROPE || (tg_bn(p.shape) % a.hd == 0), "gemm(tiled): head_dim %d does not divide the tile", a.hd);
  a.tiles_m = p.tiles_m;
  a.tiles_n = p.tiles_n;
  a.splits = p.splits;
  a.kps = p.kps;
  if (p.splits > 1) {
    NS_REQUIRE(p.tiles_m * p.tiles_n <= G_MAX_TILES, "gemm: %d tiles exceed the counter region", p.tiles_m * p.tiles_n);
    if (ws == nullptr || ws_bytes < p.bytes || reinterpret_cast<uintptr_t>(ws) % 256 != 0) {
      set_error("gemm: a zero-initialised, 256-byte aligned workspace of %zu bytes is needed, got %zu", p.bytes,
                ws == nullptr ? size_t(0) : ws_bytes);
      return NS_E_WORKSPACE;
    }
    a.cnt = static_cast<unsigned*>(ws);
    a.part = reinterpret_cast<float*>(static_cast<unsigned char*>(ws) + G_CNT_BYTES);
  }
  const dim3 grid(unsigned(p.tiles_m * p.tiles_n * p.splits));
  constexpr int EPIT = EPI == EPI_SILU ? EPI_STORE : EPI;   // the 256 x 128 and 8-wave 128^2 tiles: no SiLU
  if (p.shape == TG_BIG)
    hipLaunchKernelGGL((tiled_gemm_kernel<EPI, 8, 4, 8, 2>), grid, dim3(TgBig::NT), 0, st, a);
  else if (EPI != EPI_SILU && p.shape == TG_TALL)
    hipLaunchKernelGGL((tiled_gemm_kernel<EPIT, 4, 4, 8, 4>), grid, dim3(TgTall::NT), 0, st, a);
  else if (EPI != EPI_SILU && p.shape == TG_SMALL8)
    hipLaunchKernelGGL((tiled_gemm_kernel<EPIT, 4, 2, 8, 2>), grid, dim3(TgSmall8::NT), 0, st, a);
  else if (p.shape == TG_N96) {
    if constexpr (EPI == EPI_STORE || EPI == EPI_RESNORM)
      hipLaunchKernelGGL((tiled_gemm_kernel<EPI, 2, 3, 8, 4>), grid, dim3(TgN96::NT), 0, st, a);
  }
  else
    hipLaunchKernelGGL((tiled_gemm_kernel<EPI, 4, 4, 4, 2>), grid, dim3(TgSmall::NT), 0, st, a);
  return check_launch("gemm(tiled)");
}

static GemmArgs base_args(const void* x, const void* w, int M, int N, int K) {
  GemmArgs a{};
  a.x = static_cast<const bf16_t*>(x);
  a.w = static_cast<const bf16_t*>(w);
  a.M = M;
  a.N = N;
  a.K = K;
  return a;
}

static bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace ns

using namespace ns;

// Largest workspace any entry point needs for this shape (the SILU plan has at most as many tiles).
// Above 64 rows a plain STORE projection too long for the tile-16 kernel (K > 2048: the down projection of a
// verify batch) runs the skinny kernel in 64-row token blocks, up to T16_LARGE_M rows: every block a whole
// plan with its own counters and partials, all in one launch (the later blocks find the weights in L2).
static bool skinny_large_m(int M, int K, int N) {
  return M > G_MAX_M && M <= t16_max_m() && K > T16_MAX_K && (M + G_MAX_M - 1) / G_MAX_M * ((N + 63) / 64) <= G_MAX_TILES;
}
static size_t skinny_large_m_bytes(const Plan& p, int mblocks) {
  return p.part_off + size_t(mblocks) * (p.bytes - p.part_off);
}

extern "C" size_t ns_gemm_workspace_bytes(int M, int N, int K) {
  if (M < 1 || N < 1 || K < 32) return 0;
  if (M > G_MAX_M) {
    size_t a = tg_plan(M, N, K, EPI_STORE).bytes, b = tg_plan(M, N, K, EPI_SILU).bytes;
    // the 64-row token blocks of the skinny kernel (STORE with long K; residual + statistics at any K)
    if (M <= t16_max_m() && (M + G_MAX_M - 1) / G_MAX_M * ((N + 63) / 64) <= G_MAX_TILES) {
      const size_t c = skinny_large_m_bytes(make_plan((N + 63) / 64, K), (M + G_MAX_M - 1) / G_MAX_M);
      a = a > c ? a : c;
    }
    return a > b ? a : b;
  }
  return make_plan((N + 63) / 64, K).bytes;
}

extern "C" int ns_gemm(const void* x, const void* w, const void* bias, void* y, int M, int N, int K, int dtype,
                       const float* x_sumsq, const void* x_norm_w, float x_eps, void* ws, size_t ws_bytes,
                       void* stream) {
  int st = check_common(x, w, M, N, K, dtype, INT_MAX);
  if (st != NS_OK) return st;
  NS_REQUIRE(y != nullptr && aligned16(y), "gemm: output must be 16-byte aligned");
  if (M > G_MAX_M) {
    if (t16_large_m(M, K, (N + 15) / 16, x_sumsq != nullptr)) {
      GemmArgs a = base_args(x, w, M, N, K);
      a.bias = static_cast<const bf16_t*>(bias);
      a.y = static_cast<bf16_t*>(y);
      if ((st = bind_xnorm(a, x_sumsq, x_norm_w, x_eps)) != NS_OK) return st;
      return launch_t16<EPI_STORE>(a, (N + 15) / 16, reinterpret_cast<hipStream_t>(stream));
    }
    NS_REQUIRE(x_sumsq == nullptr, "gemm: a normalised input (x_sumsq) above %d rows needs K <= %d and at most %d "
                                   "rows", G_MAX_M, T16_MAX_K, G_NORM_ROWS);
    if (skinny_large_m(M, K, N)) {
      GemmArgs a = base_args(x, w, M, N, K);
      a.bias = static_cast<const bf16_t*>(bias);
      a.y = static_cast<bf16_t*>(y);
      a.mblocks = (M + G_MAX_M - 1) / G_MAX_M;
      const Plan p = make_plan((N + 63) / 64, K);
      Plan pm = p;
      pm.bytes = skinny_large_m_bytes(p, a.mblocks);
      if ((st = bind_workspace(a, pm, ws, ws_bytes)) != NS_OK) return st;
      return launch<EPI_STORE>(a, reinterpret_cast<hipStream_t>(stream));
    }
    return launch_tiled<EPI_STORE>(tg_args(x, w, bias, y, M, N, K), ws, ws_bytes, reinterpret_cast<hipStream_t>(stream));
  }
  GemmArgs a = base_args(x, w, M, N, K);
  a.bias = static_cast<const bf16_t*>(bias);
  a.y = static_cast<bf16_t*>(y);
  if ((st = bind_xnorm(a, x_sumsq, x_norm_w, x_eps)) != NS_OK) return st;
  if (tile16_fits(K, (N + 15) / 16)) return launch_t16<EPI_STORE>(a, (N + 15) / 16, reinterpret_cast<hipStream_t>(stream));
  if (persist_fits(M, K, (N + 63) / 64, bias)) return launch_persist(a, (N + 63) / 64, reinterpret_cast<hipStream_t>(stream));
  if ((st = bind_workspace(a, make_plan((N + 63) / 64, K), ws, ws_bytes)) != NS_OK) return st;
  return launch<EPI_STORE>(a, reinterpret_cast<hipStream_t>(stream));
}

static_assert(WS_AM_FUSED_OFF % 2 == 0 && 2 + 2 * G_MAX_M <= WS_AM_FUSED_WORDS, "fused argmax words");
extern "C" int ns_gemm_argmax_fused(int M, int N, int K) {
  return M >= 1 && M <= G_MAX_M && N >= 1 && K >= 32 && K % 32 == 0 && persist_fits(M, K, (N + 63) / 64, nullptr) ? 1 : 0;
}

extern "C" int ns_gemm_argmax(const void* x, const void* w, void* y, int M, int N, int K, int dtype,
                              const float* x_sumsq, const void* x_norm_w, float x_eps, int64_t* tokens,
                              void* argmax_ws, size_t argmax_ws_bytes, void* stream) {
  int st = check_common(x, w, M, N, K, dtype);
  if (st != NS_OK) return st;
  NS_REQUIRE(ns_gemm_argmax_fused(M, N, K) == 1,
             "gemm_argmax: M=%d N=%d K=%d is not a persistent LM-head shape (ns_gemm_argmax_fused)", M, N, K);
  NS_REQUIRE(y != nullptr && aligned16(y) && tokens != nullptr, "gemm_argmax: 16-byte aligned y and tokens needed");
  if (argmax_ws == nullptr || argmax_ws_bytes < WS_COUNTER_BYTES || reinterpret_cast<uintptr_t>(argmax_ws) % 256 != 0) {
    set_error("gemm_argmax: a zero-initialised, 256-byte aligned argmax workspace of at least %zu bytes is needed, got %zu",
              WS_COUNTER_BYTES, argmax_ws == nullptr ? size_t(0) : argmax_ws_bytes);
    return NS_E_WORKSPACE;
  }
  GemmArgs a = base_args(x, w, M, N, K);
  a.y = static_cast<bf16_t*>(y);
  if ((st = bind_xnorm(a, x_sumsq, x_norm_w, x_eps)) != NS_OK) return st;
  unsigned* words = static_cast<unsigned*>(argmax_ws);
  a.am_out = tokens;
  a.am_cnt = words + WS_AM_FUSED_OFF;
  a.am_key = reinterpret_cast<unsigned long long*>(words + WS_AM_FUSED_OFF + 2);
  return launch_persist(a, (N + 63) / 64, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int ns_gemm_silu_mul(const void* x, const void* w_gate_up, void* out, int M, int N2, int K, int dtype,
                                const float* x_sumsq, const void* x_norm_w, float x_eps, void* ws, size_t ws_bytes,
                                void* stream) {
  int st = check_common(x, w_gate_up, M, N2, K, dtype, INT_MAX);
  if (st != NS_OK) return st;
  NS_REQUIRE(N2 % 2 == 0, "gemm_silu_mul: merged gate/up rows %d must be even", N2);
  NS_REQUIRE(out != nullptr && aligned16(out), "gemm_silu_mul: output must be 16-byte aligned");
  if (M > G_MAX_M) {
    NS_REQUIRE(x_sumsq == nullptr, "gemm_silu_mul: a normalised input (x_sumsq) needs M <= %d", G_MAX_M);
    return launch_tiled<EPI_SILU>(tg_args(x, w_gate_up, nullptr, out, M, N2, K), ws, ws_bytes,
                                  reinterpret_cast<hipStream_t>(stream));
  }
  GemmArgs a = base_args(x, w_gate_up, M, N2, K);
  a.y = static_cast<bf16_t*>(out);
  if ((st = bind_xnorm(a, x_sumsq, x_norm_w, x_eps)) != NS_OK) return st;
  if (tile16_fits(K, (N2 / 2 + 7) / 8)) return launch_t16<EPI_SILU>(a, (N2 / 2 + 7) / 8, reinterpret_cast<hipStream_t>(stream));
  if ((st = bind_workspace(a, make_plan((N2 / 2 + 31) / 32, K), ws, ws_bytes)) != NS_OK) return st;
  return launch<EPI_SILU>(a, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int ns_gemm_residual_norm_stats(const void* x, const void* w, const void* residual, void* res_out,
                                           float* row_sumsq, int M, int N, int K, int dtype, void* ws,
                                           size_t ws_bytes, void* stream) {
  const bool tiled = row_sumsq == nullptr && M > t16_max_m();   // prefill chunks and mixed steps: the sum only
  int st = check_common(x, w, M, N, K, dtype, tiled ? INT_MAX : G_NORM_ROWS);
  if (st != NS_OK) return st;
  NS_REQUIRE(N % 8 == 0, "gemm_residual_norm_stats: row length %d must be a multiple of 8", N);
  NS_REQUIRE(residual != nullptr && res_out != nullptr, "gemm_residual_norm_stats: residual and res_out required");
  NS_REQUIRE(aligned16(residual) && aligned16(res_out), "gemm_residual_norm_stats: operands must be 16-byte aligned");
  if (tiled) {
    TgArgs t = tg_args(x, w, nullptr, res_out, M, N, K);
    t.res = static_cast<const bf16_t*>(residual);
    return launch_tiled<EPI_RESNORM>(t, ws, ws_bytes, reinterpret_cast<hipStream_t>(stream));
  }
  GemmArgs a = base_args(x, w, M, N, K);
  a.residual = static_cast<const bf16_t*>(residual);
  a.res_out = static_cast<bf16_t*>(res_out);
  a.sumsq_out = row_sumsq;
  if (M > G_MAX_M) {   // verify batches: 16-row blocks of the tile-16 kernel, or 64-row blocks of the skinny one
    if (t16_large_m(M, K, (N + 15) / 16, false))
      return launch_t16<EPI_RESNORM>(a, (N + 15) / 16, reinterpret_cast<hipStream_t>(stream));
    NS_REQUIRE((M + G_MAX_M - 1) / G_MAX_M * ((N + 63) / 64) <= G_MAX_TILES,
               "gemm_residual_norm_stats: M=%d N=%d: too many 64-row token blocks x tiles", M, N);
    a.mblocks = (M + G_MAX_M - 1) / G_MAX_M;
    const Plan p = make_plan((N + 63) / 64, K);
    Plan pm = p;
    pm.bytes = skinny_large_m_bytes(p, a.mblocks);
    if ((st = bind_workspace(a, pm, ws, ws_bytes)) != NS_OK) return st;
    return launch<EPI_RESNORM>(a, reinterpret_cast<hipStream_t>(stream));
  }
  if (tile16_fits(K, (N + 15) / 16)) return launch_t16<EPI_RESNORM>(a, (N + 15) / 16, reinterpret_cast<hipStream_t>(stream));
  if ((st = bind_workspace(a, make_plan((N + 63) / 64, K), ws, ws_bytes)) != NS_OK) return st;
  return launch<EPI_RESNORM>(a, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int ns_rms_norm_apply(const void* r, const float* row_sumsq, const void* norm_w, float eps, void* h,
                                 int64_t rows, int n, int dtype, void* stream) {
  NS_REQUIRE(dtype == NS_DTYPE_BF16, "rms_norm_apply: bf16 only (dtype %d)", dtype);
  NS_REQUIRE(rows >= 0 && rows <= G_NORM_ROWS && n >= 8 && n % 8 == 0,
             "rms_norm_apply: rows=%lld n=%d (rows <= %d, n %% 8 == 0)", (long long)rows, n, G_NORM_ROWS);
  NS_REQUIRE(r != nullptr && row_sumsq != nullptr && norm_w != nullptr && h != nullptr && aligned16(r) &&
                 aligned16(norm_w) && aligned16(h),
             "rms_norm_apply: null or misaligned operand");
  if (rows == 0) return NS_OK;
  hipLaunchKernelGGL(rms_norm_apply_kernel, dim3(unsigned(rows)), dim3(64), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<const bf16_t*>(r), row_sumsq, static_cast<const bf16_t*>(norm_w), static_cast<bf16_t*>(h),
                     n, eps);
  return check_launch("rms_norm_apply");
}

extern "C" int ns_gemm_rope_qkv_fits(int M, int K, int n_heads, int n_kv_heads, int head_dim, int normed) {
  const int N = (n_heads + 2 * n_kv_heads) * head_dim;
  if (M < 1 || K < 32 || K % 32 != 0 || n_heads < 1 || n_kv_heads < 1 || (head_dim != 64 && head_dim != 128)) return 0;
  // above 64 rows: the tile-16 kernel, else (a plain input) the tiled kernel's ROPE epilogue
  return M <= G_MAX_M || t16_large_m(M, K, N / 16, normed != 0) || normed == 0 ? 1 : 0;
}

extern "C" int ns_gemm_rope_qkv(const void* x, const void* w, const void* bias, const void* cos, const void* sin,
                                void* q, void* k, void* v, void* k_cache, void* v_cache, const int64_t* slots, int M,
                                int K, int n_heads, int n_kv_heads, int head_dim, int dtype, const float* x_sumsq,
                                const void* x_norm_w, float x_eps, void* ws, size_t ws_bytes, void* stream) {
  NS_REQUIRE(head_dim == 64 || head_dim == 128, "gemm_rope_qkv: head_dim %d (64 or 128)", head_dim);
  NS_REQUIRE(n_heads >= 1 && n_kv_heads >= 1, "gemm_rope_qkv: heads %d / %d", n_heads, n_kv_heads);
  const int N = (n_heads + 2 * n_kv_heads) * head_dim;
  int st = check_common(x, w, M, N, K, dtype, INT_MAX);
  if (st != NS_OK) return st;
  NS_REQUIRE(M <= G_MAX_M || t16_large_m(M, K, N / 16, x_sumsq != nullptr) || x_sumsq == nullptr,
             "gemm_rope_qkv: a normalised input above %d rows needs K <= %d and at most %d rows (ns_gemm_rope_qkv_fits)",
             G_MAX_M, T16_MAX_K, G_NORM_ROWS);
  NS_REQUIRE((k_cache == nullptr) == (v_cache == nullptr) && (k_cache == nullptr || slots != nullptr),
             "gemm_rope_qkv: give both caches and slots, or none");
  NS_REQUIRE(cos != nullptr && sin != nullptr && q != nullptr && k != nullptr && v != nullptr,
             "gemm_rope_qkv: null operand");
  NS_REQUIRE(aligned16(cos) && aligned16(sin) && aligned16(q) && aligned16(k) && aligned16(v) && aligned16(k_cache) &&
                 aligned16(v_cache),
             "gemm_rope_qkv: operands must be 16-byte aligned");
  if (M > G_MAX_M && !t16_large_m(M, K, N / 16, x_sumsq != nullptr)) {
    TgArgs t = tg_args(x, w, bias, nullptr, M, N, K);
    t.cosb = static_cast<const bf16_t*>(cos);
    t.sinb = static_cast<const bf16_t*>(sin);
    t.q = static_cast<bf16_t*>(q);
    t.k = static_cast<bf16_t*>(k);
    t.v = static_cast<bf16_t*>(v);
    t.kc = static_cast<bf16_t*>(k_cache);
    t.vc = static_cast<bf16_t*>(v_cache);
    t.slots = slots;
    t.nh = n_heads;
    t.nkv = n_kv_heads;
    t.hd = head_dim;
    NS_REQUIRE(bias == nullptr || aligned16(bias), "gemm_rope_qkv: bias must be 16-byte aligned");
    return launch_tiled<EPI_ROPE>(t, ws, ws_bytes, reinterpret_cast<hipStream_t>(stream));
  }
  GemmArgs a = base_args(x, w, M, N, K);
  a.bias = static_cast<const bf16_t*>(bias);
  a.cosb = static_cast<const bf16_t*>(cos);
  a.sinb = static_cast<const bf16_t*>(sin);
  a.q = static_cast<bf16_t*>(q);
  a.k = static_cast<bf16_t*>(k);
  a.v = static_cast<bf16_t*>(v);
  a.kc = static_cast<bf16_t*>(k_cache);
  a.vc = static_cast<bf16_t*>(v_cache);
  a.slots = slots;
  a.nh = n_heads;
  a.nkv = n_kv_heads;
  a.hd = head_dim;
  if ((st = bind_xnorm(a, x_sumsq, x_norm_w, x_eps)) != NS_OK) return st;
  if (tile16_fits(K, N / 16)) return launch_t16<EPI_ROPE>(a, N / 16, reinterpret_cast<hipStream_t>(stream));
  if ((st = bind_workspace(a, make_plan(N / 64, K), ws, ws_bytes)) != NS_OK) return st;
  return launch<EPI_ROPE>(a, reinterpret_cast<hipStream_t>(stream));
}
