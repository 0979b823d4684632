// Decode-sized GEMMs (M <= 64) on fragment-packed weights, gfx950: Y[M, N] = X[M, K] . W[N, K]^T with bf16
// in, fp32 accumulate, one launch per projection and the neighbouring token-wise op in the epilogue (the
// same epilogues and rounding points as the row-major kernels of gemm.hip).
//
// Why a second weight layout. At M = 32 a projection is bound by streaming W once from HBM. Measured on the
// MI355X, a wave that loads 1 KB of contiguous memory per instruction streams far faster than one whose
// instruction gathers the 16 rows x 64 bytes an MFMA operand fragment needs, and staging contiguous rows
// through LDS to re-read them as fragments costs a barrier per chunk that caps the row-major kernels at
// ~3 TB/s. So the weights are stored a second time, once at load, in the order the MFMA consumes them:
//
//   packed block (t, s) = 1 KB = the A operand of mfma_f32_16x16x32_bf16 for 16-row tile t and k-step s
//   (k = 32 s .. 32 s + 31): lane l's 16 bytes are W[row(t, l % 16)][32 s + 8 (l / 16) .. + 7];
//   blocks in (tile, step) order, so a tile's K is contiguous (16 rows x 2K bytes).
//
// Tile row orders (pk_row) put the rows an epilogue pairs into one tile: PK_ROWS 16 consecutive rows;
// PK_GATE_UP 8 gate rows + the matching 8 up rows of a merged [gate; up] weight; PK_ROPE 8 dims of a head +
// the 8 dims half a head further (the rotate-half partners). The same orders as the tile-16 kernel.
//
// Kernel (one workgroup per CU, persistent): a work unit is (tile, K slice). With K whole (sl = 1) workgroup
// g walks a contiguous block of tiles, so its outputs fill whole lines of its own XCD's L2; with sl > 1 it
// owns slice g % sl and walks the units g, g + G, g + 2G, ... (G a multiple of sl). Weights are read
// non-temporally (streamed once). Wave w of the workgroup owns steps
// [w S, w S + S) of the slice: it loads the matching X fragments once (B operand, 16 tokens x 32 k per
// fragment; normalised on load for an rms_norm input) and keeps them in registers, then for each unit
// issues its S weight blocks (S contiguous 1 KB loads), multiplies them as they arrive, and writes its
// partial 16 x 16 TM tile to LDS; after one barrier the epilogue threads add the waves' partials in wave
// order (deterministic) and run the epilogue. One unit of loads in flight per wave measured fastest (more
// queues behind itself at memory). Units of a sliced tile (sl > 1: long K, or too few tiles to fill the
// GPU) publish their fp32 partials; after its last unit a workgroup counts them in and the last slice of
// a tile to arrive adds the slices in slice order and runs the epilogue. Each unit's epilogue operands are
// loaded before the next unit's weights are requested, so waiting for them never waits for the stream
// (vector loads complete in issue order).
#include <climits>
#include <type_traits>

#include "gemm_common.h"

namespace ns {

enum PackOrder { PK_ROWS = 0, PK_GATE_UP = 1, PK_ROPE = 2 };

constexpr int PK_SMAX = 8;        // k-steps per wave per unit at most
constexpr int PK_CU = 256;        // workgroups that stream at once: one per CU
constexpr int PK_NX_MAX_K = 4 * RS_PRE * G_NORM_COLS;   // longest normalised input (its norm weight in LDS)
constexpr int PK_MAX_TILES = 8191;
constexpr int PK_MAX_UNITS_PER_WG = 256;   // sliced units one workgroup may own (merge flags in LDS)
constexpr size_t PK_CNT_BYTES = sizeof(unsigned) * (PK_MAX_TILES + 1);

__host__ __device__ inline int pk_tiles(int N, int order, int hd) {
  if (order == PK_GATE_UP) return (N / 2 + 7) / 8;
  if (order == PK_ROPE) return N / 16;
  (void)hd;
  return (N + 15) / 16;
}

// Weight row of row r (0..15) of tile t, clamped inside the matrix (or its half).
__device__ __forceinline__ int pk_row(int order, int N, int hd, int t, int r) {
  if (order == PK_GATE_UP) {
    const int half = N >> 1;
    return r < 8 ? min(8 * t + r, half - 1) : half + min(8 * t + r - 8, half - 1);
  }
  if (order == PK_ROPE) {
    const int tph = hd >> 4, head = t / tph, f = t - head * tph;
    return head * hd + 8 * f + (r < 8 ? r : (hd >> 1) + r - 8);
  }
  return min(16 * t + r, N - 1);
}

__global__ __launch_bounds__(256) void pack_weight_kernel(const g_u32x4_t* __restrict__ w, g_u32x4_t* __restrict__ p,
                                                          int N, int K, int order, int hd, int tiles) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;   // (tile, step, lane)
  const int steps = K >> 5;
  if (i >= int64_t(tiles) * steps * 64) return;
  const int lane = int(i & 63);
  const int64_t ts = i >> 6;
  const int t = int(ts / steps), s = int(ts - int64_t(t) * steps);
  const int row = pk_row(order, N, hd, t, lane & 15);
  p[i] = w[(int64_t(row) * K + 32 * s + 8 * (lane >> 4)) >> 3];
}

struct PkArgs {
  const bf16_t* x;            // [M, K] (an rms_norm input: r, normalised on load)
  const g_u32x4_t* wp;        // packed weight
  int M, N, K;                // N: rows of W
  int tiles, steps, sl, sps;  // tiles, K / 32, K slices, steps per slice
  int tb;                     // token blocks: > 1 splits M into 16-row blocks, one workgroup per (tile, block)
  const bf16_t* bias;
  bf16_t* y;
  const bf16_t* residual;
  bf16_t* res_out;
  float* sumsq_out;           // RESNORM: [tiles][64] row sums of r^2 over the tile's 16 columns
  const float* xsq;           // normalised input: [ceil(K/16)][64] row sums of r^2
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
  unsigned* cnt;              // sliced tiles' arrival counters, cstride words apart (zero between calls)
  int cstride;
  float* part;                // [tiles][sl][TM * 32 items][8] published partial tiles
  int64_t* am_out;            // fused argmax (LM head): tokens [M], row keys [M], arrival counter
  unsigned long long* am_key;
  unsigned* am_cnt;
};

// Epilogue items: every thread of the workgroup takes two adjacent values of one row. STORE / RESNORM item
// (m, j) = row m, tile columns 2j, 2j + 1 (8 items per row); SILU / ROPE item (m, j) = row m, tile rows 2j,
// 2j + 1 (gate, or the lo dims) and 8 + 2j, 8 + 2j + 1 (up, or the hi dims) (4 items per row). Short
// per-thread chains keep the epilogue of a unit off the next unit's critical path (all waves meet at the
// next barrier).
template <int EPI>
constexpr bool pk_pair() { return EPI == EPI_SILU || EPI == EPI_ROPE; }
template <int TM, int EPI>
constexpr int pk_items() { return TM * 16 * (pk_pair<EPI>() ? 4 : 8); }

// Operands an item's epilogue reads (raw bits, clamped addresses), loaded before the next unit's weights.
struct PkOps {
  uint32_t a, b, c, d, e, f;
  int64_t slot;
};

template <int EPI>
__device__ __forceinline__ void pk_load_ops(const PkArgs& p, int t, int m, int j, PkOps& o) {
  const bf16_t* bsrc = p.bias != nullptr ? p.bias : reinterpret_cast<const bf16_t*>(p.wp);
  if constexpr (EPI == EPI_STORE) {
    o.a = *reinterpret_cast<const uint32_t*>(bsrc + min(16 * t + 2 * j, p.N - 2));
  } else if constexpr (EPI == EPI_RESNORM) {
    o.a = *reinterpret_cast<const uint32_t*>(p.residual + int64_t(m) * p.N + min(16 * t + 2 * j, p.N - 2));
  } else if constexpr (EPI == EPI_ROPE) {
    const int tph = p.hd >> 4, head = t / tph, f = t - head * tph, hh = p.hd >> 1, d = 8 * f + 2 * j;
    o.a = *reinterpret_cast<const uint32_t*>(bsrc + head * p.hd + d);
    o.b = *reinterpret_cast<const uint32_t*>(bsrc + head * p.hd + hh + d);
    o.c = *reinterpret_cast<const uint32_t*>(p.cosb + int64_t(m) * p.hd + d);
    o.d = *reinterpret_cast<const uint32_t*>(p.cosb + int64_t(m) * p.hd + hh + d);
    o.e = *reinterpret_cast<const uint32_t*>(p.sinb + int64_t(m) * p.hd + d);
    o.f = *reinterpret_cast<const uint32_t*>(p.sinb + int64_t(m) * p.hd + hh + d);
    o.slot = (p.slots != nullptr ? p.slots : reinterpret_cast<const int64_t*>(p.wp))[m];
  }
}

__device__ __forceinline__ float bf_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// The epilogue of item (m, j) of tile t from its fp32 values (lo: columns 2j, 2j + 1, or rows 2j, 2j + 1;
// hi: rows 8 + 2j, 9 + 2j of a paired item). Returns RESNORM's r0^2 + r1^2 (0 otherwise). am (STORE): the
// stored values' best (value, index) of this item, updated.
template <int EPI>
__device__ __forceinline__ float pk_epilogue(const PkArgs& p, int t, int m, int j, const float (&lo)[2],
                                             const float (&hi)[2], const PkOps& o, bool am, float& am_v, int& am_i) {
  if constexpr (EPI == EPI_STORE) {
    const int n = 16 * t + 2 * j;   // N is even: the pair is whole or past the end
    if (n >= p.N) return 0.f;
    const bool bias = p.bias != nullptr;
    const uint32_t w = pack_bf16x2(lo[0] + (bias ? bf_lo(o.a) : 0.f), lo[1] + (bias ? bf_hi(o.a) : 0.f));
    *reinterpret_cast<uint32_t*>(p.y + int64_t(m) * p.N + n) = w;
    if (am) {
      if (better(bf_lo(w), n, am_v, am_i)) { am_v = bf_lo(w); am_i = n; }
      if (better(bf_hi(w), n + 1, am_v, am_i)) { am_v = bf_hi(w); am_i = n + 1; }
    }
    return 0.f;
  } else if constexpr (EPI == EPI_RESNORM) {
    const int n = 16 * t + 2 * j;
    if (n >= p.N) return 0.f;
    const float r0 = round_bf16(bf_lo(o.a) + round_bf16(lo[0])), r1 = round_bf16(bf_hi(o.a) + round_bf16(lo[1]));
    *reinterpret_cast<uint32_t*>(p.res_out + int64_t(m) * p.N + n) = pack_bf16x2(r0, r1);
    return r0 * r0 + r1 * r1;
  } else if constexpr (EPI == EPI_SILU) {
    const int half = p.N >> 1, c = 8 * t + 2 * j;
    float out[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float gb = round_bf16(lo[e]), ub = round_bf16(hi[e]);
      const float sg = gb * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(gb * -1.44269504088896341f));
      out[e] = round_bf16(sg) * ub;
    }
    bf16_t* dst = p.y + int64_t(m) * half + c;
    if ((half & 1) == 0 && c + 1 < half) {
      *reinterpret_cast<uint32_t*>(dst) = pack_bf16x2(out[0], out[1]);   // 4-byte aligned
    } else {
      if (c < half) dst[0] = bf16_t(pack_bf16x2(out[0], 0.f));
      if (c + 1 < half) dst[1] = bf16_t(pack_bf16x2(out[1], 0.f));
    }
    return 0.f;
  } else {   // EPI_ROPE
    const int tph = p.hd >> 4, head = t / tph, f = t - head * tph, hh = p.hd >> 1, d = 8 * f + 2 * j;
    const bool bias = p.bias != nullptr;
    const float xl0 = round_bf16(lo[0] + (bias ? bf_lo(o.a) : 0.f)), xl1 = round_bf16(lo[1] + (bias ? bf_hi(o.a) : 0.f));
    const float xh0 = round_bf16(hi[0] + (bias ? bf_lo(o.b) : 0.f)), xh1 = round_bf16(hi[1] + (bias ? bf_hi(o.b) : 0.f));
    float ol0 = xl0, ol1 = xl1, oh0 = xh0, oh1 = xh1;
    if (head < p.nh + p.nkv) {
      ol0 = round_bf16(xl0 * bf_lo(o.c)) - round_bf16(xh0 * bf_lo(o.e));
      ol1 = round_bf16(xl1 * bf_hi(o.c)) - round_bf16(xh1 * bf_hi(o.e));
      oh0 = round_bf16(xh0 * bf_lo(o.d)) + round_bf16(xl0 * bf_lo(o.f));
      oh1 = round_bf16(xh1 * bf_hi(o.d)) + round_bf16(xl1 * bf_hi(o.f));
    }
    const uint32_t wl = pack_bf16x2(ol0, ol1), wh = pack_bf16x2(oh0, oh1);
    bf16_t* dst;
    bf16_t* cdst = nullptr;
    if (head < p.nh) {
      dst = p.q + (int64_t(m) * p.nh + head) * p.hd;
    } else if (head < p.nh + p.nkv) {
      const int kh = head - p.nh;
      dst = p.k + (int64_t(m) * p.nkv + kh) * p.hd;
      if (p.kc != nullptr) cdst = p.kc + (o.slot * p.nkv + kh) * p.hd;
    } else {
      const int vh = head - p.nh - p.nkv;
      dst = p.v + (int64_t(m) * p.nkv + vh) * p.hd;
      if (p.vc != nullptr) cdst = p.vc + (o.slot * p.nkv + vh) * p.hd;
    }
    *reinterpret_cast<uint32_t*>(dst + d) = wl;
    *reinterpret_cast<uint32_t*>(dst + hh + d) = wh;
    if (cdst != nullptr) {
      *reinterpret_cast<uint32_t*>(cdst + d) = wl;
      *reinterpret_cast<uint32_t*>(cdst + hh + d) = wh;
    }
    return 0.f;
  }
}

__device__ __forceinline__ void pub_store8(float* p, float a, float b) {
  const uint64_t v = uint64_t(__float_as_uint(a)) | (uint64_t(__float_as_uint(b)) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t pub_load8(const float* p) {
  return __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<float*>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// inv of rows 0 .. M - 1 for K <= 2048 (every partial prefetched by row_stats_issue; the same additions in
// the same order as row_stats_finish, without its loop for longer rows, whose loads would make the
// compiler wait for everything in flight)
__device__ __forceinline__ void pk_row_stats_finish(int ptiles, int M, int K, float eps, const float (&v)[RS_PRE],
                                                    float* s_inv) {
  const int tid = threadIdx.x, m = tid >> 2, g = tid & 3;
  float part = 0.f;
#pragma unroll
  for (int e = 0; e < RS_PRE; ++e)
    if (g + 4 * e < ptiles) part += v[e];
  part += __shfl_xor(part, 1, 64);
  part += __shfl_xor(part, 2, 64);
  if (m < M && g == 0) s_inv[m] = rsqrtf(part / float(K) + eps);
}

constexpr int PK_MERGE = 16;   // slices whose partials one merge round trip loads

// S: k-steps per wave per unit, a compile-time count, so every load and MFMA of a unit is unconditional and
// the compiler's wait counts stay exact (a load guarded by a runtime test turns every later wait into a wait
// for everything, the previous unit's epilogue stores included). Steps past the wave's share of its slice
// re-read the slice's last block and multiply zero activations.
template <int TM, int EPI, bool NX, int NW, int S, bool BIAS>
__global__ __launch_bounds__(NW * 64) void packed_gemm_kernel(PkArgs p) {
  constexpr int NT = NW * 64;
  constexpr bool PAIR = pk_pair<EPI>();
  constexpr int NI = pk_items<TM, EPI>(), IPT = (NI + NT - 1) / NT, JPR = PAIR ? 4 : 8;   // items, per thread, per row
  constexpr int VP = PAIR ? 4 : 2;                                                         // values per item
  static_assert(TM <= NW && S <= PK_SMAX && NT % JPR == 0, "one statistics wave per 16 rows");
  __shared__ __align__(16) float red[2][NW][TM][256];   // partial tiles (MFMA output layout), double-buffered
  __shared__ float s_inv[G_MAX_M];
  __shared__ __align__(16) uint32_t s_nw[NX ? 2 * PK_NX_MAX_K / 4 : 4];   // a normalised input's norm weight
  __shared__ unsigned s_last[PK_MAX_UNITS_PER_WG];
  const int G = gridDim.x, tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, r4 = lane >> 4;
  int u0 = int(blockIdx.x);
  if (p.tb > 1) {
    // token split (one unit per workgroup, no K slices): workgroup g computes 16-row token block b of tile t;
    // in groups of 8 workgroups (one per XCD, workgroup g runs on XCD g % 8), so the blocks of a tile run on
    // one XCD and the second read of its weights hits that XCD's L2
    const int g = u0, tb = p.tb;
    int b, t;
    if (p.tiles % 8 == 0) {
      b = (g >> 3) % tb;
      t = (g & 7) + 8 * ((g >> 3) / tb);
    } else {
      b = g % tb;
      t = g / tb;
    }
    u0 = t;
    const int m0 = 16 * b;
    p.M = min(16, p.M - m0);
    p.x += int64_t(m0) * p.K;
    if constexpr (NX) p.xsq += m0;
    if constexpr (EPI == EPI_STORE) {
      p.y += int64_t(m0) * p.N;
    } else if constexpr (EPI == EPI_RESNORM) {
      p.residual += int64_t(m0) * p.N;
      p.res_out += int64_t(m0) * p.N;
      if (p.sumsq_out != nullptr) p.sumsq_out += m0;
    } else if constexpr (EPI == EPI_SILU) {
      p.y += int64_t(m0) * (p.N >> 1);
    } else {
      p.cosb += int64_t(m0) * p.hd;
      p.sinb += int64_t(m0) * p.hd;
      if (p.slots != nullptr) p.slots += m0;
      p.q += int64_t(m0) * p.nh * p.hd;
      p.k += int64_t(m0) * p.nkv * p.hd;
      p.v += int64_t(m0) * p.nkv * p.hd;
    }
  }
  const int M = p.M, K = p.K, steps = p.steps, units = p.tiles * p.sl;
  const int slice = int(blockIdx.x) % p.sl;
  const int s0 = slice * p.sps, slen = min(p.sps, steps - s0);
  const int kb = s0 + wv * S, nv = max(0, min(S, slen - wv * S));
  const int klast = s0 + slen - 1;                          // last step of the slice (re-read past the share)
  const bool am = p.am_out != nullptr;

  // a normalised input's row statistics and norm weight first, then X: all of them return before the
  // weight stream that follows. The norm weight goes to LDS once (16 bytes per thread) and each wave reads
  // its fragments there: a fragment load from memory would be a 1 KB wave access for 64 distinct bytes.
  const int ptiles = (K + G_NORM_COLS - 1) / G_NORM_COLS;
  float rs[RS_PRE];
  g_u32x4_t nwf[S], nw_part = {};
  if constexpr (NX) {
    if (wv < TM) row_stats_issue(p.xsq, ptiles, M, rs);
    nw_part = *reinterpret_cast<const g_u32x4_t*>(p.xnw + min(8 * tid, K - 8));
  }
  g_u32x4_t xf[S][TM];
#pragma unroll
  for (int i = 0; i < S; ++i)
#pragma unroll
    for (int mb = 0; mb < TM; ++mb)
      xf[i][mb] = *reinterpret_cast<const g_u32x4_t*>(p.x + int64_t(min(16 * mb + c16, M - 1)) * K +
                                                       32 * min(kb + i, klast) + 8 * r4);
  // units of this workgroup: a contiguous block of tiles when K is whole (consecutive tiles write adjacent
  // 32-byte pieces of every output row, which then fill whole lines in this XCD's L2 instead of being
  // written back piecemeal by eight XCDs; the weights stream contiguously too), else every G-th unit (one
  // K slice per workgroup). Blocks go to XCDs in runs (workgroup g runs on XCD g % 8 and takes block
  // (g % 8) G / 8 + g / 8), so each XCD gets an equal contiguous share of the tiles: numbered in launch
  // order, the blocks one unit longer would all land on the same few XCDs.
  const int gb = G % 8 == 0 ? (u0 & 7) * (G >> 3) + (u0 >> 3) : u0;
  const int ub = p.sl == 1 ? (p.tb > 1 ? u0 : int(int64_t(gb) * units / G)) : u0;
  const int ue = p.sl == 1 ? (p.tb > 1 ? u0 + 1 : int(int64_t(gb + 1) * units / G)) : units;
  const int ustep = p.sl == 1 ? 1 : G;
  const int ulast = p.sl == 1 ? ue - 1 : units - 1;
  g_u32x4_t wr[S];
  auto load_w = [&](int u) __attribute__((always_inline)) {
    const int t = min(u, ulast) / p.sl;
    const g_u32x4_t* src = p.wp + int64_t(t) * steps * 64 + lane;
#pragma unroll
    for (int i = 0; i < S; ++i) wr[i] = __builtin_nontemporal_load(src + int64_t(min(kb + i, klast)) * 64);
  };
  auto load_ops = [&](int u, PkOps (&o)[IPT]) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < IPT; ++q) {
      const int it = min(tid + q * NT, NI - 1);
      pk_load_ops<EPI>(p, min(u, units - 1) / p.sl, min(it / JPR, M - 1), it % JPR, o[q]);
    }
  };
  constexpr bool OPS = EPI != EPI_SILU && (EPI != EPI_STORE || BIAS);   // epilogue operands per unit
  PkOps ops[IPT] = {};
  if constexpr (OPS) load_ops(min(ub, units - 1), ops);
  load_w(ub);
  if constexpr (NX) {
    if (wv < TM) pk_row_stats_finish(ptiles, M, K, p.xeps, rs, s_inv);
    if (8 * tid < K) *reinterpret_cast<g_u32x4_t*>(s_nw + 4 * tid) = nw_part;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < S; ++i) nwf[i] = *reinterpret_cast<const g_u32x4_t*>(s_nw + ((32 * min(kb + i, klast) + 8 * r4) >> 1));
    float xinv[TM];
#pragma unroll
    for (int mb = 0; mb < TM; ++mb) xinv[mb] = s_inv[min(16 * mb + c16, M - 1)];
#pragma unroll
    for (int i = 0; i < S; ++i)
#pragma unroll
      for (int mb = 0; mb < TM; ++mb) xf[i][mb] = norm_fragment(xf[i][mb], nwf[i], xinv[mb]);
  }
#pragma unroll
  for (int i = 0; i < S; ++i)   // steps past the wave's share multiply zeros
    if (i >= nv)
#pragma unroll
      for (int mb = 0; mb < TM; ++mb) xf[i][mb] = g_u32x4_t{0u, 0u, 0u, 0u};

  float am_v[IPT];
  int am_i[IPT];
#pragma unroll
  for (int q = 0; q < IPT; ++q) {
    am_v[q] = -INFINITY;
    am_i[q] = INT_MAX;
  }
  // tile values of item (m, j) from red[par], waves added in order: MFMA output row n sits in lane
  // (n / 4) * 16 + m % 16, component n % 4, so rows 2j, 2j + 1 are one 8-byte read
  auto item_values = [&](int par, int m, int j, float (&lo)[2], float (&hi)[2]) __attribute__((always_inline)) {
    const int mb = m >> 4, mr = m & 15;
    const int off_lo = ((2 * j) >> 2) * 64 + mr * 4 + ((2 * j) & 3);
    const int off_hi = ((8 + 2 * j) >> 2) * 64 + mr * 4 + ((2 * j) & 3);
    lo[0] = lo[1] = hi[0] = hi[1] = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float2 a = *reinterpret_cast<const float2*>(&red[par][w][mb][off_lo]);
      lo[0] += a.x;
      lo[1] += a.y;
      if constexpr (PAIR) {
        const float2 b = *reinterpret_cast<const float2*>(&red[par][w][mb][off_hi]);
        hi[0] += b.x;
        hi[1] += b.y;
      }
    }
  };
  int par = 0;
  for (int u = ub; u < ue; u += ustep) {
    const int t = u / p.sl;
    g_float4_t acc[TM];
#pragma unroll
    for (int mb = 0; mb < TM; ++mb) acc[mb] = g_float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < S; ++i)
#pragma unroll
      for (int mb = 0; mb < TM; ++mb)
        acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(g_bf16x8_t, wr[i]),
                                                          __builtin_bit_cast(g_bf16x8_t, xf[i][mb]), acc[mb], 0, 0, 0);
#pragma unroll
    for (int mb = 0; mb < TM; ++mb) *reinterpret_cast<g_float4_t*>(&red[par][wv][mb][lane * 4]) = acc[mb];
    // this unit's epilogue operands, then the next unit's weights
    PkOps cur[IPT];
#pragma unroll
    for (int q = 0; q < IPT; ++q) cur[q] = ops[q];
    if constexpr (OPS) load_ops(min(u + ustep, ulast), ops);
    load_w(u + ustep);
    __syncthreads();   // every wave's partial tile of unit u is in red[par]
#pragma unroll
    for (int q = 0; q < IPT; ++q) {
      const int it = tid + q * NT, m = it / JPR, j = it % JPR;
      float lo[2], hi[2], ss = 0.f;
      if (it < NI) {
        item_values(par, m, j, lo, hi);
        if (p.sl == 1) {
          if (m < M) ss = pk_epilogue<EPI>(p, t, m, j, lo, hi, cur[q], am, am_v[q], am_i[q]);
        } else {   // publish this slice's partial: [tile][slice][item][VP]
          float* dst = p.part + ((int64_t(t) * p.sl + slice) * NI + it) * VP;
          pub_store8(dst, lo[0], lo[1]);
          if constexpr (PAIR) pub_store8(dst + 2, hi[0], hi[1]);
        }
      }
      if constexpr (EPI == EPI_RESNORM) {
        if (p.sl == 1) {   // the row's 16 columns are 8 neighbouring lanes
          ss += __shfl_xor(ss, 1, 64);
          ss += __shfl_xor(ss, 2, 64);
          ss += __shfl_xor(ss, 4, 64);
          if (it < NI && m < M && j == 0 && p.sumsq_out != nullptr) p.sumsq_out[int64_t(t) * G_NORM_ROWS + m] = ss;
        }
      }
    }
    par ^= 1;
  }

  if (p.sl > 1) {
    // count this workgroup's units in; the last slice of a tile to arrive adds the slices in order
    publish_complete();
    __syncthreads();
    const int nmine = u0 < units ? (units - 1 - u0) / G + 1 : 0;
    if (tid < nmine) {
      const int t = (u0 + tid * G) / p.sl;
      unsigned* c = p.cnt + int64_t(t) * p.cstride;
      const unsigned last = publish_count(c) == unsigned(p.sl - 1);
      if (last) publish_reset(c);
      s_last[tid] = last;
    }
    __syncthreads();
    acquire_published();
    for (int jj = 0; jj < nmine; ++jj) {
      if (s_last[jj] == 0u) continue;   // uniform
      const int t = (u0 + jj * G) / p.sl;
      PkOps o[IPT] = {};
      if constexpr (OPS) load_ops(t * p.sl, o);
#pragma unroll
      for (int q = 0; q < IPT; ++q) {
        const int it = tid + q * NT, m = it / JPR, j = it % JPR;
        float lo[2] = {0.f, 0.f}, hi[2] = {0.f, 0.f}, ss = 0.f;
        if (it < NI) {
          for (int sb = 0; sb < p.sl; sb += PK_MERGE) {
            uint64_t va[PK_MERGE], vb[PK_MERGE];
#pragma unroll
            for (int k = 0; k < PK_MERGE; ++k)
              if (sb + k < p.sl) {
                const float* src = p.part + ((int64_t(t) * p.sl + sb + k) * NI + it) * VP;
                va[k] = pub_load8(src);
                if constexpr (PAIR) vb[k] = pub_load8(src + 2);
              }
#pragma unroll
            for (int k = 0; k < PK_MERGE; ++k)
              if (sb + k < p.sl) {
                lo[0] += __uint_as_float(uint32_t(va[k]));
                lo[1] += __uint_as_float(uint32_t(va[k] >> 32));
                if constexpr (PAIR) {
                  hi[0] += __uint_as_float(uint32_t(vb[k]));
                  hi[1] += __uint_as_float(uint32_t(vb[k] >> 32));
                }
              }
          }
          if (m < M) ss = pk_epilogue<EPI>(p, t, m, j, lo, hi, o[q], am, am_v[q], am_i[q]);
        }
        if constexpr (EPI == EPI_RESNORM) {
          ss += __shfl_xor(ss, 1, 64);
          ss += __shfl_xor(ss, 2, 64);
          ss += __shfl_xor(ss, 4, 64);
          if (it < NI && m < M && j == 0 && p.sumsq_out != nullptr) p.sumsq_out[int64_t(t) * G_NORM_ROWS + m] = ss;
        }
      }
    }
  }

  if constexpr (EPI == EPI_STORE) {
    if (am) {
      // each row's best over this workgroup (its 8 items are neighbouring lanes), one 64-bit atomic max per
      // (workgroup, row) into the row's key; the last workgroup turns keys into tokens
#pragma unroll
      for (int q = 0; q < IPT; ++q) {
        float v = am_v[q];
        int ix = am_i[q];
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) {
          const float ov = __shfl_xor(v, o, 64);
          const int oi = __shfl_xor(ix, o, 64);
          if (better(ov, oi, v, ix)) {
            v = ov;
            ix = oi;
          }
        }
        const int it = tid + q * NT, m = it / JPR;
        if (it < NI && it % JPR == 0 && m < M && ix != INT_MAX)
          __hip_atomic_fetch_max(p.am_key + m, argmax_key(v, ix), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      publish_complete();
      __syncthreads();
      if (tid == 0) {
        const unsigned last = publish_count(p.am_cnt) == unsigned(G - 1);
        if (last) publish_reset(p.am_cnt);
        s_last[0] = last;
      }
      __syncthreads();
      if (s_last[0] == 0u) return;
      acquire_published();
      if (tid < M) {
        const unsigned long long key = __hip_atomic_load(p.am_key + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(p.am_key + tid, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        p.am_out[tid] = key == 0ull ? 0 : int64_t(~uint32_t(key));
      }
    }
  }
}

// ------------------------------------------------------------------------------------------- host side
struct PkPlan {
  int cfg, sl, sps, grid;   // cfg: index into PK_CFGS
  int tb;                   // token blocks (1: none)
  size_t bytes;             // workspace: the counter region, then the partial tiles
};

// (waves per workgroup, k-steps per wave): the shapes a unit's K range can take. Measured on the 1.5B decode
// projections: 8 x 6 for gate/up and the LM head (48 steps, unsliced), 4 x 6 for QKV and O (two slices of
// 24 steps), 4 x 7 for down (ten slices of 28 steps).
struct PkCfg {
  int nw, s;
};
constexpr PkCfg PK_CFGS[] = {{8, 8}, {8, 6}, {8, 4}, {4, 7}, {4, 6}};
constexpr int PK_NCFG = int(sizeof(PK_CFGS) / sizeof(PK_CFGS[0]));

static int pk_tm(int M) { return M <= 32 ? 2 : 4; }

// Work split: with several 16-row token blocks, few tiles and K <= 2048 (QKV and O of a 32-row decode
// step), one workgroup per (tile, token block); otherwise K <= 2048 is never sliced (a slice merge costs
// three dependent cross-XCD round trips, more than the idle CUs of a small projection); longer K is cut
// into the fewest 64-step slices when the tiles cover the GPU twice, else into slices of at most 28 steps
// (the down projection). Then the configuration with the least capacity that holds a slice (ties: more
// waves), and the largest grid that is a multiple of the slice count, up to one workgroup per CU (or every
// unit once).
static PkPlan pk_plan(int M, int tiles, int steps) {
  PkPlan p;
  p.tb = 1;
  int sl;
  const int tb = (M + 15) / 16;
  if (tb > 1 && tiles * tb <= PK_CU && steps <= 64) {
    // few tiles, short K: split the tokens instead of K (no cross-workgroup merge)
    p.tb = tb;
    sl = 1;
  } else if (steps <= 64) {
    sl = 1;   // a K merge (three dependent cross-XCD round trips, ~5 us) costs more than idle CUs
  } else if (tiles >= 2 * PK_CU) {
    sl = (steps + 63) / 64;
  } else {
    sl = (steps + 27) / 28;
  }
  p.sps = (steps + sl - 1) / sl;
  p.sl = (steps + p.sps - 1) / p.sps;   // every slice non-empty
  p.cfg = -1;
  for (int c = 0; c < PK_NCFG; ++c) {
    const int cap = PK_CFGS[c].nw * PK_CFGS[c].s;
    if (cap < p.sps) continue;
    if (p.cfg < 0) {
      p.cfg = c;
      continue;
    }
    const int best = PK_CFGS[p.cfg].nw * PK_CFGS[p.cfg].s;
    if (cap < best || (cap == best && PK_CFGS[c].nw > PK_CFGS[p.cfg].nw)) p.cfg = c;
  }
  const int units = tiles * p.sl;
  p.grid = p.tb > 1 ? tiles * p.tb : min(units, (PK_CU / p.sl) * p.sl);
  const size_t part = p.sl > 1 ? sizeof(float) * size_t(tiles) * p.sl * pk_tm(M) * 32 * 8 : 0;
  p.bytes = PK_CNT_BYTES + ((part + 255) & ~size_t(255));
  return p;
}

static int pk_check(const void* x, const void* wp, int M, int N, int K, int dtype) {
  NS_REQUIRE(dtype == NS_DTYPE_BF16, "packed gemm: bf16 only (dtype %d)", dtype);
  NS_REQUIRE(M >= 1 && M <= G_MAX_M, "packed gemm: M=%d outside [1, %d]", M, G_MAX_M);
  NS_REQUIRE(N >= 1 && K >= 32 && K % 32 == 0, "packed gemm: N=%d K=%d (K must be a positive multiple of 32)", N, K);
  NS_REQUIRE(x != nullptr && wp != nullptr, "packed gemm: null operand");
  NS_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(wp) % 16 == 0,
             "packed gemm: operands must be 16-byte aligned");
  return NS_OK;
}

static int pk_bind(PkArgs& a, const PkPlan& pl, int tiles, void* ws, size_t ws_bytes) {
  NS_REQUIRE(pl.cfg >= 0, "packed gemm: no configuration holds %d steps per slice", pl.sps);
  a.tiles = tiles;
  a.steps = a.K / 32;
  a.sl = pl.sl;
  a.sps = pl.sps;
  a.tb = pl.tb;
  if (pl.sl == 1) return NS_OK;
  NS_REQUIRE(tiles <= PK_MAX_TILES, "packed gemm: %d sliced tiles exceed the %d counters", tiles, PK_MAX_TILES);
  if (ws == nullptr || ws_bytes < pl.bytes || reinterpret_cast<uintptr_t>(ws) % 256 != 0) {
    set_error("packed gemm: a zero-initialised, 256-byte aligned workspace of %zu bytes is needed, got %zu", pl.bytes,
              ws == nullptr ? size_t(0) : ws_bytes);
    return NS_E_WORKSPACE;
  }
  const int units = tiles * pl.sl;
  NS_REQUIRE((units + pl.grid - 1) / pl.grid <= PK_MAX_UNITS_PER_WG && (units + pl.grid - 1) / pl.grid <= 4 * 64,
             "packed gemm: %d sliced units over %d workgroups exceed the merge capacity", units, pl.grid);
  unsigned char* b = static_cast<unsigned char*>(ws);
  a.cnt = reinterpret_cast<unsigned*>(b);
  a.cstride = ws_counter_stride(size_t(tiles), size_t(PK_MAX_TILES + 1));
  a.part = reinterpret_cast<float*>(b + PK_CNT_BYTES);
  return NS_OK;
}

template <int EPI, bool NX, int NW, int S, bool BIAS>
static void pk_launch_cfg(const PkArgs& a, int grid, hipStream_t st) {
  const dim3 g{unsigned(grid)}, b{unsigned(NW * 64)};
  if constexpr (NW == 8 && S != 7) {   // token-split plans run 16 tokens per workgroup
    if (a.tb > 1) {
      hipLaunchKernelGGL((packed_gemm_kernel<1, EPI, NX, NW, S, BIAS>), g, b, 0, st, a);
      return;
    }
  }
  if (a.M <= 32)
    hipLaunchKernelGGL((packed_gemm_kernel<2, EPI, NX, NW, S, BIAS>), g, b, 0, st, a);
  else
    hipLaunchKernelGGL((packed_gemm_kernel<4, EPI, NX, NW, S, BIAS>), g, b, 0, st, a);
}

template <int EPI, bool NX, bool BIAS>
static void pk_launch_b(const PkArgs& a, const PkPlan& pl, hipStream_t st) {
  static_assert(PK_NCFG == 5, "one case per configuration");
  switch (pl.cfg) {
    case 0: pk_launch_cfg<EPI, NX, 8, 8, BIAS>(a, pl.grid, st); break;
    case 1: pk_launch_cfg<EPI, NX, 8, 6, BIAS>(a, pl.grid, st); break;
    case 2: pk_launch_cfg<EPI, NX, 8, 4, BIAS>(a, pl.grid, st); break;
    case 3: pk_launch_cfg<EPI, NX, 4, 7, BIAS>(a, pl.grid, st); break;
    default: pk_launch_cfg<EPI, NX, 4, 6, BIAS>(a, pl.grid, st); break;
  }
}

// STORE without a bias reads no epilogue operand per unit; every other epilogue reads its operands
template <int EPI, bool NX>
static void pk_launch(const PkArgs& a, const PkPlan& pl, hipStream_t st) {
  if constexpr (EPI == EPI_STORE) {
    if (a.bias == nullptr) {
      pk_launch_b<EPI, NX, false>(a, pl, st);
      return;
    }
  }
  pk_launch_b<EPI, NX, true>(a, pl, st);
}

static PkArgs pk_args(const void* x, const void* wp, int M, int N, int K, const float* x_sumsq, const void* x_norm_w,
                      float x_eps) {
  PkArgs a{};
  a.x = static_cast<const bf16_t*>(x);
  a.wp = static_cast<const g_u32x4_t*>(wp);
  a.M = M;
  a.N = N;
  a.K = K;
  a.xsq = x_sumsq;
  a.xnw = static_cast<const bf16_t*>(x_norm_w);
  a.xeps = x_eps;
  return a;
}

static int pk_norm_check(int K, const float* x_sumsq, const void* x_norm_w) {
  NS_REQUIRE((x_sumsq == nullptr) == (x_norm_w == nullptr), "packed gemm: x_sumsq and x_norm_w go together");
  NS_REQUIRE(x_norm_w == nullptr || reinterpret_cast<uintptr_t>(x_norm_w) % 16 == 0,
             "packed gemm: norm weight must be 16-byte aligned");
  NS_REQUIRE(x_sumsq == nullptr || K <= PK_NX_MAX_K, "packed gemm: a normalised input needs K <= %d (K=%d)",
             PK_NX_MAX_K, K);
  return NS_OK;
}

}  // namespace ns

using namespace ns;

extern "C" size_t ns_packed_weight_bytes(int N, int K, int order, int head_dim) {
  if (N < 1 || K < 32 || K % 32 != 0 || order < PK_ROWS || order > PK_ROPE) return 0;
  return size_t(pk_tiles(N, order, head_dim)) * size_t(K) * 32;
}

extern "C" int ns_pack_weight(const void* w, void* packed, int N, int K, int order, int head_dim, void* stream) {
  NS_REQUIRE(w != nullptr && packed != nullptr, "pack weight: null pointer");
  NS_REQUIRE(N >= 1 && K >= 32 && K % 32 == 0, "pack weight: N=%d K=%d (K a positive multiple of 32)", N, K);
  NS_REQUIRE(reinterpret_cast<uintptr_t>(w) % 16 == 0 && reinterpret_cast<uintptr_t>(packed) % 16 == 0,
             "pack weight: pointers must be 16-byte aligned");
  NS_REQUIRE(order >= PK_ROWS && order <= PK_ROPE, "pack weight: unknown order %d", order);
  if (order == PK_GATE_UP) NS_REQUIRE(N % 2 == 0, "pack weight: gate/up rows N=%d must be even", N);
  if (order == PK_ROPE)
    NS_REQUIRE((head_dim == 64 || head_dim == 128) && N % head_dim == 0,
               "pack weight: RoPE order needs head_dim 64 or 128 dividing N (N=%d, head_dim=%d)", N, head_dim);
  const int tiles = pk_tiles(N, order, head_dim);
  const int64_t threads = int64_t(tiles) * (K / 32) * 64;
  hipLaunchKernelGGL(pack_weight_kernel, dim3(unsigned((threads + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const g_u32x4_t*>(w), static_cast<g_u32x4_t*>(packed),
                     N, K, order, head_dim, tiles);
  return check_launch("pack weight");
}

extern "C" size_t ns_gemm_packed_workspace_bytes(int M, int N, int K, int order, int head_dim) {
  if (M < 1 || M > G_MAX_M || N < 1 || K < 32 || K % 32 != 0) return 0;
  return pk_plan(M, pk_tiles(N, order, head_dim), K / 32).bytes;
}

extern "C" int ns_gemm_packed(const void* x, const void* w_packed, const void* bias, void* y, int M, int N, int K,
                              int dtype, const float* x_sumsq, const void* x_norm_w, float x_eps, void* workspace,
                              size_t workspace_bytes, void* stream) {
  int rc = pk_check(x, w_packed, M, N, K, dtype);
  if (rc == NS_OK) rc = pk_norm_check(K, x_sumsq, x_norm_w);
  if (rc != NS_OK) return rc;
  NS_REQUIRE(y != nullptr && reinterpret_cast<uintptr_t>(y) % 16 == 0, "packed gemm: y must be 16-byte aligned");
  NS_REQUIRE(N % 8 == 0 && reinterpret_cast<uintptr_t>(bias) % 16 == 0,
             "packed gemm: N=%d must be a multiple of 8 and the bias 16-byte aligned", N);
  PkArgs a = pk_args(x, w_packed, M, N, K, x_sumsq, x_norm_w, x_eps);
  a.bias = static_cast<const bf16_t*>(bias);
  a.y = static_cast<bf16_t*>(y);
  const int tiles = pk_tiles(N, PK_ROWS, 0);
  const PkPlan pl = pk_plan(M, tiles, K / 32);
  if ((rc = pk_bind(a, pl, tiles, workspace, workspace_bytes)) != NS_OK) return rc;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (x_sumsq != nullptr)
    pk_launch<EPI_STORE, true>(a, pl, st);
  else
    pk_launch<EPI_STORE, false>(a, pl, st);
  return check_launch("packed gemm");
}

extern "C" int ns_gemm_argmax_packed_fits(int M, int N, int K) {
  if (M < 1 || M > G_MAX_M || N < 8 || N % 8 != 0 || K < 32 || K % 32 != 0) return 0;
  const PkPlan pl = pk_plan(M, pk_tiles(N, PK_ROWS, 0), K / 32);
  return pl.sl == 1 && pl.tb == 1 && pl.cfg >= 0 ? 1 : 0;
}

extern "C" int ns_gemm_packed_sliced(int M, int N, int K, int order, int head_dim) {
  if (M < 1 || M > G_MAX_M || N < 1 || K < 32 || K % 32 != 0) return 0;
  return pk_plan(M, pk_tiles(N, order, head_dim), K / 32).sl > 1 ? 1 : 0;
}

extern "C" int ns_gemm_argmax_packed(const void* x, const void* w_packed, void* y, int M, int N, int K, int dtype,
                                     const float* x_sumsq, const void* x_norm_w, float x_eps, int64_t* tokens,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  int rc = pk_check(x, w_packed, M, N, K, dtype);
  if (rc == NS_OK) rc = pk_norm_check(K, x_sumsq, x_norm_w);
  if (rc != NS_OK) return rc;
  NS_REQUIRE(ns_gemm_argmax_packed_fits(M, N, K) == 1, "packed argmax gemm: shape M=%d N=%d K=%d not taken", M, N, K);
  NS_REQUIRE(y != nullptr && tokens != nullptr && reinterpret_cast<uintptr_t>(y) % 16 == 0,
             "packed argmax gemm: y (16-byte aligned) and tokens are required");
  NS_REQUIRE(workspace != nullptr && workspace_bytes >= WS_COUNTER_BYTES && reinterpret_cast<uintptr_t>(workspace) % 256 == 0,
             "packed argmax gemm: a zeroed argmax workspace of at least %zu bytes is needed", WS_COUNTER_BYTES);
  PkArgs a = pk_args(x, w_packed, M, N, K, x_sumsq, x_norm_w, x_eps);
  a.y = static_cast<bf16_t*>(y);
  unsigned* words = static_cast<unsigned*>(workspace);
  a.am_cnt = words + WS_AM_FUSED_OFF;
  a.am_key = reinterpret_cast<unsigned long long*>(words + WS_AM_FUSED_OFF + 2);
  a.am_out = tokens;
  const int tiles = pk_tiles(N, PK_ROWS, 0);
  const PkPlan pl = pk_plan(M, tiles, K / 32);
  if ((rc = pk_bind(a, pl, tiles, nullptr, 0)) != NS_OK) return rc;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (x_sumsq != nullptr)
    pk_launch<EPI_STORE, true>(a, pl, st);
  else
    pk_launch<EPI_STORE, false>(a, pl, st);
  return check_launch("packed argmax gemm");
}

extern "C" int ns_gemm_silu_mul_packed(const void* x, const void* w_packed, void* out, int M, int N2, int K, int dtype,
                                       const float* x_sumsq, const void* x_norm_w, float x_eps, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  int rc = pk_check(x, w_packed, M, N2, K, dtype);
  if (rc == NS_OK) rc = pk_norm_check(K, x_sumsq, x_norm_w);
  if (rc != NS_OK) return rc;
  NS_REQUIRE(N2 % 2 == 0, "packed silu gemm: N2=%d must be even (gate rows then up rows)", N2);
  NS_REQUIRE(out != nullptr && reinterpret_cast<uintptr_t>(out) % 16 == 0, "packed silu gemm: out must be 16-byte aligned");
  PkArgs a = pk_args(x, w_packed, M, N2, K, x_sumsq, x_norm_w, x_eps);
  a.y = static_cast<bf16_t*>(out);
  const int tiles = pk_tiles(N2, PK_GATE_UP, 0);
  const PkPlan pl = pk_plan(M, tiles, K / 32);
  if ((rc = pk_bind(a, pl, tiles, workspace, workspace_bytes)) != NS_OK) return rc;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (x_sumsq != nullptr)
    pk_launch<EPI_SILU, true>(a, pl, st);
  else
    pk_launch<EPI_SILU, false>(a, pl, st);
  return check_launch("packed silu gemm");
}

extern "C" int ns_gemm_residual_norm_stats_packed(const void* x, const void* w_packed, const void* residual,
                                                  void* res_out, float* row_sumsq, int M, int N, int K, int dtype,
                                                  void* workspace, size_t workspace_bytes, void* stream) {
  int rc = pk_check(x, w_packed, M, N, K, dtype);
  if (rc != NS_OK) return rc;
  NS_REQUIRE(N % 8 == 0, "packed residual gemm: N=%d must be a multiple of 8", N);
  NS_REQUIRE(residual != nullptr && res_out != nullptr && reinterpret_cast<uintptr_t>(residual) % 16 == 0 &&
                 reinterpret_cast<uintptr_t>(res_out) % 16 == 0,
             "packed residual gemm: residual and res_out (16-byte aligned) are required");
  PkArgs a = pk_args(x, w_packed, M, N, K, nullptr, nullptr, 0.f);
  a.residual = static_cast<const bf16_t*>(residual);
  a.res_out = static_cast<bf16_t*>(res_out);
  a.sumsq_out = row_sumsq;
  const int tiles = pk_tiles(N, PK_ROWS, 0);
  const PkPlan pl = pk_plan(M, tiles, K / 32);
  if ((rc = pk_bind(a, pl, tiles, workspace, workspace_bytes)) != NS_OK) return rc;
  pk_launch<EPI_RESNORM, false>(a, pl, static_cast<hipStream_t>(stream));
  return check_launch("packed residual gemm");
}

extern "C" int ns_gemm_rope_qkv_packed(const void* x, const void* w_packed, const void* bias, const void* cos,
                                       const void* sin, void* q, void* k, void* v, void* k_cache, void* v_cache,
                                       const int64_t* slots, int M, int K, int n_heads, int n_kv_heads, int head_dim,
                                       int dtype, const float* x_sumsq, const void* x_norm_w, float x_eps,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  const int N = (n_heads + 2 * n_kv_heads) * head_dim;
  int rc = pk_check(x, w_packed, M, N, K, dtype);
  if (rc == NS_OK) rc = pk_norm_check(K, x_sumsq, x_norm_w);
  if (rc != NS_OK) return rc;
  NS_REQUIRE((head_dim == 64 || head_dim == 128) && n_heads >= 1 && n_kv_heads >= 1,
             "packed rope gemm: head_dim %d (64 or 128), heads %d / %d", head_dim, n_heads, n_kv_heads);
  NS_REQUIRE(cos != nullptr && sin != nullptr && q != nullptr && k != nullptr && v != nullptr,
             "packed rope gemm: cos, sin, q, k, v are required");
  NS_REQUIRE((k_cache == nullptr) == (v_cache == nullptr) && (k_cache == nullptr || slots != nullptr),
             "packed rope gemm: the caches and slots go together");
  const void* ptrs[] = {bias, cos, sin, q, k, v, k_cache, v_cache};
  for (const void* pp : ptrs)
    NS_REQUIRE(reinterpret_cast<uintptr_t>(pp) % 16 == 0, "packed rope gemm: operands must be 16-byte aligned");
  PkArgs a = pk_args(x, w_packed, M, N, K, x_sumsq, x_norm_w, x_eps);
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
  const int tiles = pk_tiles(N, PK_ROPE, head_dim);
  const PkPlan pl = pk_plan(M, tiles, K / 32);
  if ((rc = pk_bind(a, pl, tiles, workspace, workspace_bytes)) != NS_OK) return rc;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (x_sumsq != nullptr)
    pk_launch<EPI_ROPE, true>(a, pl, st);
  else
    pk_launch<EPI_ROPE, false>(a, pl, st);
  return check_launch("packed rope gemm");
}
