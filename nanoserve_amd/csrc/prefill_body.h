// Paged chunked-prefill attention for gfx950 (MI355X), bf16.
//
// Semantics: nanoserve/model.py:283-318 (Qwen2Model._attend, per-sequence branch) with the pages
// gathered by PagedKVCache.gather (kv_cache.py:281-288). A step may carry several sequences, each with
// ctx cached tokens and T new ones whose K/V rope_qkv has already written into the pages. Query j of a
// sequence (absolute position ctx + j) attends to keys 0 .. ctx + j of that sequence -- the causal
// offset mask of model.py:297-299; a fresh prefill is ctx = 0. GQA: query head h reads KV head
// h / (n_heads / n_kv_heads). Online softmax in fp32; probabilities are rounded to bf16 before P.V, as
// the decode kernel does (paged_attention.py:77).
//
// Design:
//   * Work unit = (head, tile of QT = 128 queries, partition of the tile's keys). A workgroup is 8 waves
//     in two groups of 4 that hold the same 128 queries and walk two key ranges of the partition (group
//     g its half of the stages); wave w of a group owns queries 32w .. 32w+31 as two 16-query MFMA tiles,
//     so every K and V fragment it reads from LDS feeds two products. A tile's keys (64-key stages of 4
//     pages) are split into partitions of at most 2 PS stages; the host picks PS so the whole launch fits
//     PF_SLOTS workgroups (one per CU: each holds 128 KB of LDS) in one round, with the fewest partitions
//     that does.
//   * K/V go straight from HBM into LDS (global_load_lds, 16 bytes per lane; wave w of a group copies
//     page w of the group's stage), double-buffered per group: the copy of stage n+1 runs while stage n
//     is multiplied. The copies are
//     inline asm with a scalar page base and per-lane 32-bit offsets fixed for the whole launch, so
//     issuing one costs no vector arithmetic, and the compiler sees no LDS write in flight (it would
//     otherwise wait for the whole next-stage copy before the current stage's first LDS read). Block ids
//     come from a window of 64 table entries held one per lane and read with readlane. K rows are stored
//     with XOR-swizzled 16-byte chunks so fragment reads are free of bank conflicts.
//   * Per stage and wave, on the matrix cores (mfma 16x16x32 bf16 throughout), in two halves of 32 keys:
//       S^T[16 keys x 16 queries] = K_page[16 x hd] . Q^T[hd x 16]         2 pages x 2 query tiles
//       O^T[hd x 16 queries]    += V^T[hd x 32 keys] . P^T[32 keys x 16]   hd/16 tiles x 2 query tiles
//     S^T comes out with lane = query and 4 consecutive keys per lane; two pages' worth is the 8-key
//     B operand of P^T, so P never leaves registers. V^T fragments come from LDS by transpose reads.
//     The second half's scores are issued before the first half's softmax, so the matrix cores have
//     work while the softmax runs. Row maxima over the four key groups of a query use the gfx950 lane
//     swaps (v_permlane32_swap, v_permlane16_swap) instead of LDS shuffles. The softmax reference point
//     moves only when a score exceeds it by 2^8, so the accumulator is rescaled rarely.
//   * Masks are computed only on stages that cross a query's diagonal or the end of the keys: key k is
//     visible to query j iff k <= ctx + j. Only a stage that reaches keys at or past ctx + T (unwritten
//     slots of the last page, pages past the tile's reach) or holds a bad block id also zeroes those V
//     rows, so garbage there can never turn 0 * x into NaN; a stage that only crosses a diagonal reads
//     written keys, whose weights past the diagonal are exact zeros. Block ids outside [0, num_blocks)
//     are masked pages.
//   * End of a workgroup: the two groups hand their states over through LDS and each folds half of the
//     output tiles (dims), so both halves of a row are complete in one group each. The output rows are
//     staged in LDS and stored whole, 16 bytes per lane. A tile split over several partitions: each
//     group publishes its half's (m, l, acc) with 16-byte agent-scope stores, waits for them to complete,
//     and the workgroup bumps the tile's arrival counter; in the last workgroup to arrive both groups
//     merge their halves over all partitions in partition order (PF_MB partitions loaded per round trip;
//     the result does not depend on arrival order). One launch; the workspace counters are left at zero.
#pragma once

#include "ns_common.h"

#include <algorithm>
#include <type_traits>

namespace ns {

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 pf_bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float pf_float4_t;
typedef short v4i16_t __attribute__((ext_vector_type(4)));

constexpr float PF_LOG2E = 1.4426950408889634f;
constexpr int PF_PAGE = 16;
constexpr int PF_NP = 4;                    // pages per stage
constexpr int PF_KEYS = PF_NP * PF_PAGE;    // 64 keys per stage
constexpr int PF_WAVES = 4;                 // waves of one group (one key range of a tile's queries)
constexpr int PF_THREADS = PF_WAVES * 64;
constexpr int PF_GROUPS = 2;                // groups per workgroup: two key ranges of the same queries
constexpr int PF_WG_THREADS = PF_GROUPS * PF_THREADS;
constexpr int PF_R = 2;                     // 16-query MFMA tiles per wave
constexpr int PF_QT = 16 * PF_R * PF_WAVES; // queries per work unit
constexpr int PF_PS_MIN = 4;                // fewest stages per partition the plan picks
constexpr int PF_SLOTS = 248;               // workgroups per launch the plan aims below: one resident per
                                            // CU (128 KB of LDS) on the 256 CUs (32 per XCD), less a margin
constexpr int PF_MB = 3;                    // partitions loaded per round trip of the merge
constexpr float PF_SLACK = 8.0f;            // log2 headroom of the softmax reference point

template <int HD>
struct PfLds {
  static constexpr int ROW = HD * 2;                  // bytes per token row (K and V), no padding
  static constexpr int CH = HD / 8;                   // 16-byte chunks per row
  static constexpr int K_BYTES = PF_KEYS * ROW;
  static constexpr int STAGE = 2 * K_BYTES;           // K rows, then V rows
  static constexpr int TPI = 1024 / ROW;              // token rows per wave-wide 16-byte load (1 KB)
  static constexpr int IPP = PF_PAGE / TPI;           // such loads per page and tensor
  // K rows are stored with their 16-byte chunks XOR-swizzled by the row, so the 16 rows one fragment
  // read touches land in 16 different bank groups: logical chunk c of stage row t sits at c ^ key(t).
  static __host__ __device__ constexpr int key(int t) { return HD == 128 ? (t & 15) : ((t >> 1) & 7); }
  // V rows likewise, by an even key from the row's low bits: a transpose read takes a 32-byte chunk pair
  // (2 chunks) from each of four consecutive rows, and XOR by even values moves whole pairs, so the four
  // rows' pairs land in four different bank groups.
  static __host__ __device__ constexpr int vkey(int t) { return (t & (CH / 2 - 1)) << 1; }
  // A load's token rows are TPI i + r (r = lane / CH < TPI); both keys split over that sum without carries,
  // key(TPI i + r) = key(TPI i) ^ key(r), so a lane's swizzled chunk offsets are fixed per lane up to a
  // compile-time XOR per load (checked for every token of a page below).
  static constexpr bool keys_split() {
    for (int t = 0; t < PF_PAGE; ++t) {
      const int i = t / TPI, r = t % TPI;
      if (key(t) != (key(TPI * i) ^ key(r)) || vkey(t) != (vkey(TPI * i) ^ vkey(r))) return false;
    }
    return true;
  }
};
static_assert(PF_NP == PF_WAVES, "each wave stages one page of a stage");
static_assert(PfLds<64>::keys_split() && PfLds<128>::keys_split(), "row keys split over a load's token rows");

// two fp32 -> packed bf16 (round to nearest even; v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pf_bf16x2(float lo, float hi) {
  typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
  bf16x2_t r;
  r[0] = static_cast<__bf16>(lo);
  r[1] = static_cast<__bf16>(hi);
  return __builtin_bit_cast(uint32_t, r);
}

// Maximum over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four key groups of one S^T column), by the gfx950 lane
// swaps: permlane32_swap of a register with itself leaves lanes l and l ^ 32 in the two results, and
// permlane16_swap does the same for l and l ^ 16. Every lane of the four gets the same value.
__device__ __forceinline__ float pf_max4(float v) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
// The same four lanes' sum, (x_l + x_l^32) + (x_l^16 + x_l^48) in an order every lane of the four shares.
__device__ __forceinline__ float pf_sum4(float v) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// One wave-wide HBM -> LDS copy of 16 bytes per lane (global_load_lds_dwordx4; lane i fills lds + 16 i) from
// base + off: base is wave-uniform (scalar registers), off the lane's byte offset. Inline asm, so the
// compiler sees no LDS write in flight and puts no wait for it in front of the current stage's LDS reads;
// the stage loop's explicit vmcnt(0) and barrier are the only wait the copies need. M0 holds the
// wave-uniform LDS address; s_nop 0 is the wait state an LDS-DMA load needs after M0 is written.
__device__ __forceinline__ void pf_dma16(const char* base, uint32_t off, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(off), "s"(base), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ uint32_t pf_lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}

struct PrefillArgs {
  const bf16_t* q;
  int64_t q_st, q_sh;               // token / head strides of q (elements)
  const bf16_t* kp;
  const bf16_t* vp;
  int64_t s_blk, s_pos, s_h;        // pool strides (elements)
  const int32_t* bt;                // [S, max_blocks] block tables
  int64_t bt_sb;
  const int32_t* info;              // [S, 4]: q_start, n_new, ctx_len, unused
  bf16_t* out;
  int64_t o_st, o_sh;
  int G, max_blocks, num_blocks, n_heads, n_seqs;
  float scale_log2;
  int tiles_max, parts_max, ps;     // query tiles, partitions per tile (grid), target stages per partition
  unsigned* cnt;                    // [S, n_heads, tiles_max] arrival counters, cstride words apart (zero
  int cstride;                      // between calls)
  float* ws_ml;                     // [unit][R][2][256 threads] (m, l)
  float* ws_acc;                    // [unit][R][NT][256 threads] float4
};

// The kernel's body: bid is the workgroup's index among the prefill workgroups of the launch; lds the
// launch's LDS (at least PF_GROUPS * 2 * PfLds<HD>::STAGE bytes, 16-byte aligned) and s_last one LDS word.
template <int HD>
__device__ __forceinline__ void prefill_body(const PrefillArgs& a, int bid, unsigned char* lds, unsigned& s_last) {
  using L = PfLds<HD>;
  constexpr int KS = HD / 32;   // k-steps of Q.K^T
  constexpr int NT = HD / 16;   // output tiles of P.V
  // lds: per group, stage st0 + i in buffer i % 2; after the loop the same bytes carry the groups' states

  // ---- this workgroup's work unit. The launch's units -- sequence by sequence, a sequence's query tiles
  // from the last (longest) down, a tile's workgroups, then heads -- are numbered from 0, so the busy
  // workgroups are the first of the grid and spread evenly over the XCDs (workgroup i runs on XCD i % 8);
  // the grid is an upper bound and the rest exit at once. A tile's keys split into 2 n_parts key ranges
  // of at most ps stages; workgroup `part` of the tile takes ranges 2 part (group 0) and 2 part + 1
  // (group 1). A sequence with more new tokens than the caller's max_new is not computed.
  int rem = bid, seq = -1, tile = 0, part = 0, h = 0, n_st = 0, n_parts = 0, n_pages = 0;
  for (int sq = 0; sq < a.n_seqs && seq < 0; ++sq) {
    const int Tq = a.info[4 * sq + 1], cq = a.info[4 * sq + 2];
    const int nt = (Tq + PF_QT - 1) / PF_QT;
    if (Tq <= 0 || nt > a.tiles_max) continue;
    for (int tr = 0; tr < nt; ++tr) {
      const int tl = nt - 1 - tr;
      const int np = min((cq + min(PF_QT * (tl + 1), Tq) + PF_PAGE - 1) / PF_PAGE, a.max_blocks);
      const int ns = (np + PF_NP - 1) / PF_NP;
      const int npt = min((ns + 2 * a.ps - 1) / (2 * a.ps), a.parts_max);
      if (rem < npt * a.n_heads) {
        seq = sq;
        tile = tl;
        part = rem / a.n_heads;
        h = rem - part * a.n_heads;
        n_st = ns;
        n_parts = npt;
        n_pages = np;
        break;
      }
      rem -= npt * a.n_heads;
    }
  }
  if (seq < 0) return;
  const int q_start = a.info[4 * seq + 0], T = a.info[4 * seq + 1], ctx = a.info[4 * seq + 2];
  const int qbase = tile * PF_QT;
  const int kv_total = ctx + T;             // keys that exist
  const int n_sub = 2 * n_parts;
  const int tid_wg = threadIdx.x, gi = __builtin_amdgcn_readfirstlane(tid_wg >> 8);   // group (wave-uniform)
  const int sub = 2 * part + gi;
  const int st0 = sub * n_st / n_sub, st1 = (sub + 1) * n_st / n_sub;
  // both groups run the same number of stage-loop iterations (their barriers are the workgroup's)
  const int n_iter = max(((2 * part + 1) * n_st / n_sub) - (2 * part * n_st / n_sub),
                         ((2 * part + 2) * n_st / n_sub) - ((2 * part + 1) * n_st / n_sub));
  const int g = h / a.G;
  const int32_t* table = a.bt + int64_t(seq) * a.bt_sb;
  const int tid = tid_wg & (PF_THREADS - 1), lane = tid & 63, w = tid >> 6;   // thread and wave in the group
  const int c16 = lane & 15, r4 = lane >> 4;

  // this lane's queries (rows past T mirror row T-1 and are not stored)
  int jq[PF_R], jrow[PF_R];
  pf_bf16x8_t qf[PF_R][KS];
#pragma unroll
  for (int rt = 0; rt < PF_R; ++rt) {
    jq[rt] = qbase + 16 * PF_R * w + 16 * rt + c16;
    jrow[rt] = min(jq[rt], T - 1);
    const bf16_t* qrow = a.q + int64_t(q_start + jrow[rt]) * a.q_st + int64_t(h) * a.q_sh;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qf[rt][s] = __builtin_bit_cast(pf_bf16x8_t, *reinterpret_cast<const uint4*>(qrow + 32 * s + 8 * r4));
  }
  const int j_first_w = qbase + 16 * PF_R * w;          // the wave's first query
  const int j_last_w = min(j_first_w + 16 * PF_R - 1, T - 1);
  const bool wave_live = j_first_w < T;

  // ---- staging: block ids of a window of 16 stages in one register (lane i: page 4 * win0 + i), their
  // validity as a wave-wide bit mask; wave w copies page w of a stage straight from HBM into LDS.
  int win0 = st0, pid = 0;
  uint64_t pok = 0;
  auto load_window = [&](int n0) __attribute__((always_inline)) {
    win0 = n0;
    const int p = PF_NP * n0 + lane;
    const int id = table[min(p, n_pages - 1)];
    pok = __ballot(p < n_pages && id >= 0 && id < a.num_blocks);
    pid = (id >= 0 && id < a.num_blocks) ? id : 0;   // masked pages read block 0 (in bounds)
  };
  // validity bits of stage n's 4 pages (n inside the current window)
  auto stage_ok = [&](int n) __attribute__((always_inline)) { return unsigned(pok >> (PF_NP * (n - win0))) & 0xFu; };
  unsigned char* glds = lds + gi * (2 * L::STAGE);   // this group's two stage buffers
  const uint32_t lds0 = pf_lds_addr(glds);
  const uint32_t spos2 = uint32_t(a.s_pos) * 2u;   // token stride in bytes (checked < 2^26 by the host)
  const uint32_t lane_row = uint32_t(lane / L::CH) * spos2;
  const uint32_t lane_kx = 16u * uint32_t((lane % L::CH) ^ L::key(lane / L::CH));
  const uint32_t lane_vx = 16u * uint32_t((lane % L::CH) ^ L::vkey(lane / L::CH));
  auto dma_stage = [&](int n, int buf) __attribute__((always_inline)) {
    const int id = __builtin_amdgcn_readlane(pid, PF_NP * (n - win0) + w);
    const int64_t base = (int64_t(id) * a.s_blk + int64_t(g) * a.s_h) * 2;
    const char* kb = reinterpret_cast<const char*>(a.kp) + base;
    const char* vb = reinterpret_cast<const char*>(a.vp) + base;
    const uint32_t kd = __builtin_amdgcn_readfirstlane(lds0 + uint32_t(buf * L::STAGE + w * (PF_PAGE * L::ROW)));
    // Load i fills LDS slot (token row t = TPI i + r, chunk cp) with the token's chunk cp ^ key(t) (K) or
    // cp ^ vkey(t) (V): the lane's row offset r * spos2 and its chunk offsets for load 0 are kept for the
    // launch, load i flips the chunk offset by the constant 16 key(TPI i) and adds TPI i token rows to the
    // scalar page base. (Opaque copies, so the compiler keeps three registers instead of hoisting all eight
    // offsets.)
    uint32_t lrow = lane_row, kx = lane_kx, vx = lane_vx;
    asm volatile("" : "+v"(lrow), "+v"(kx), "+v"(vx));
#pragma unroll
    for (int i = 0; i < L::IPP; ++i) {
      const int64_t rows = int64_t(L::TPI * i) * spos2;
      pf_dma16(kb + rows, lrow + (kx ^ uint32_t(16 * L::key(L::TPI * i))), kd + 1024 * i);
      pf_dma16(vb + rows, lrow + (vx ^ uint32_t(16 * L::vkey(L::TPI * i))), kd + L::K_BYTES + 1024 * i);
    }
  };

  float m_run[PF_R], l_run[PF_R];
  pf_float4_t acc[PF_R][NT];
#pragma unroll
  for (int rt = 0; rt < PF_R; ++rt) {
    m_run[rt] = -INFINITY;
    l_run[rt] = 0.f;
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[rt][t] = pf_float4_t{0.f, 0.f, 0.f, 0.f};
  }

  // One stage: S^T for all 64 keys (both halves of 32 keys: pages 2 hs, 2 hs + 1), one softmax update
  // per query tile over the whole stage, then P and O^T += V^T . P^T half by half, with the second half's
  // probabilities computed while the first half's products run. MODE 0: every key of the stage is visible
  // to every query of the wave; 1: the stage crosses the wave's diagonal (scores masked); 2: it also reaches
  // past the keys that exist or holds a bad block id (scores masked and those V rows zeroed).
  // (Every array lives inside this one function: passed by reference between helpers, the compiler kept
  // some of them in scratch memory.)
  // hook: called once the score products are issued (group 1 issues the next stage's copies there)
  auto compute = [&](const unsigned char* st, int kb0, unsigned okm, auto mask_c, auto&& hook) __attribute__((always_inline)) {
    constexpr int MODE = decltype(mask_c)::value;
    pf_float4_t sc[2][PF_R][2];   // [half][query tile][page of the half]
    pf_bf16x8_t kf[2][KS];
#pragma unroll
    for (int hs = 0; hs < 2; ++hs) {
      // ---- K fragments of the half (A operands of S^T: lane (c16, r4) holds key c16 of the page, dims
      // 32 s + 8 r4 .. +7), then S^T for both query tiles, the k-step loop outermost so consecutive MFMAs
      // accumulate into different tiles
#pragma unroll
      for (int hp = 0; hp < 2; ++hp) {
        const unsigned char* krow = st + (PF_PAGE * (2 * hs + hp) + c16) * L::ROW;
        const int kk = L::key(c16);
#pragma unroll
        for (int s = 0; s < KS; ++s)
          kf[hp][s] = __builtin_bit_cast(pf_bf16x8_t, *reinterpret_cast<const uint4*>(krow + 16 * ((4 * s + r4) ^ kk)));
      }
#pragma unroll
      for (int rt = 0; rt < PF_R; ++rt)
#pragma unroll
        for (int hp = 0; hp < 2; ++hp) sc[hs][rt][hp] = pf_float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int hp = 0; hp < 2; ++hp)
#pragma unroll
          for (int rt = 0; rt < PF_R; ++rt)
            sc[hs][rt][hp] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[hp][s], qf[rt][s], sc[hs][rt][hp], 0, 0, 0);
    }
    hook();
    // ---- softmax statistics over the stage: masked scores -> -inf, the stage maximum per query, the
    // reference point and the rescale factor
    float mc[PF_R];
#pragma unroll
    for (int rt = 0; rt < PF_R; ++rt) {
      float mx = -INFINITY;
#pragma unroll
      for (int hs = 0; hs < 2; ++hs)
#pragma unroll
        for (int hp = 0; hp < 2; ++hp) {
          // key 4 r4 + e of page pp is visible iff e <= lim (keys past ctx + T lie past every query's
          // diagonal, since jrow <= T - 1); a bad page hides all four
          const int pp = 2 * hs + hp;
          int lim = ctx + jrow[rt] - (kb0 + PF_PAGE * pp + 4 * r4);
          if constexpr (MODE == 2) lim = ((okm >> pp) & 1u) != 0 ? lim : -1;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if constexpr (MODE != 0) sc[hs][rt][hp][e] = e <= lim ? sc[hs][rt][hp][e] : -INFINITY;
            mx = fmaxf(mx, sc[hs][rt][hp][e]);
          }
        }
      mx = pf_max4(mx);
      // Reference point m (scaled units, c = scale * log2(e)): weights are exp2(s * c - m). It moves
      // only when a score exceeds it by more than PF_SLACK, so weights stay below 2^PF_SLACK and the
      // accumulator is rescaled rarely. The normalised result is the same function of the scores; only
      // the bf16 rounding of individual weights (relative 2^-9) depends on where m sits.
      const float mxc = mx * a.scale_log2;
      const bool move = mxc > m_run[rt] + PF_SLACK;
      const float m_new = move ? mxc : m_run[rt];
      mc[rt] = m_new == -INFINITY ? 0.f : m_new;   // nothing visible yet: weights 0
      const float alpha = __builtin_amdgcn_exp2f(m_run[rt] - mc[rt]);
      m_run[rt] = m_new;
      l_run[rt] *= alpha;
      if (__ballot(move)) {   // the reference point moved for some query of the wave
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[rt][t] *= alpha;
      }
    }
    // ---- per half: V^T fragments by transpose reads (ds_read_b64_tr_b16): within each group of 16 lanes,
    // lane j addresses 4 dims (16t + 4 (j % 4) ..) of key row kb + j / 4, and lane i receives dim 16t + i
    // of keys kb .. kb + 3 -- its A-operand slots for one page; k-slots 0..3 = page 2 hs keys 4 r4 + e,
    // 4..7 = page 2 hs + 1 (MODE 2: keys that do not exist, past ctx + T or on a bad page, read as 0).
    // Probabilities P^T (B operands, k-slot e = key 4 r4 + e of each page), then O^T += V^T . P^T.
#pragma unroll
    for (int hs = 0; hs < 2; ++hs) {
      v4i16_t va[2][NT];
#pragma unroll
      for (int hp = 0; hp < 2; ++hp) {
        const int pp = 2 * hs + hp;
        const int vr = PF_PAGE * pp + 4 * r4 + (c16 >> 2);   // the key row this lane addresses
        const unsigned char* vrow = st + L::K_BYTES + vr * L::ROW;
        uint32_t m01 = 0xffffffffu, m23 = 0xffffffffu;
        if constexpr (MODE == 2) {
          const int key0 = kb0 + PF_PAGE * pp + 4 * r4;
          const bool ok = ((okm >> pp) & 1u) != 0;
          m01 = (ok && key0 + 0 < kv_total ? 0x0000ffffu : 0u) | (ok && key0 + 1 < kv_total ? 0xffff0000u : 0u);
          m23 = (ok && key0 + 2 < kv_total ? 0x0000ffffu : 0u) | (ok && key0 + 3 < kv_total ? 0xffff0000u : 0u);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const int dim = 16 * t + 4 * (c16 & 3);
          const int chunk = dim >> 3;
          const unsigned char* src = vrow + 16 * (chunk ^ L::vkey(vr)) + 2 * (dim & 7);
          v4i16_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16_t*)(src));
          if constexpr (MODE == 2) {
            uint2 u = __builtin_bit_cast(uint2, v);
            u.x &= m01;
            u.y &= m23;
            v = __builtin_bit_cast(v4i16_t, u);
          }
          va[hp][t] = v;
        }
      }
#pragma unroll
      for (int rt = 0; rt < PF_R; ++rt) {
        float psum = 0.f;
        uint32_t pb[4];
#pragma unroll
        for (int hp = 0; hp < 2; ++hp) {
          float pv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            pv[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[hs][rt][hp][e], a.scale_log2, -mc[rt]));
            psum += pv[e];
          }
          pb[2 * hp + 0] = pf_bf16x2(pv[0], pv[1]);
          pb[2 * hp + 1] = pf_bf16x2(pv[2], pv[3]);
        }
        l_run[rt] += psum;
        const pf_bf16x8_t pbv = __builtin_bit_cast(pf_bf16x8_t, make_uint4(pb[0], pb[1], pb[2], pb[3]));
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const uint2 lo = __builtin_bit_cast(uint2, va[0][t]), hi = __builtin_bit_cast(uint2, va[1][t]);
          const pf_bf16x8_t vav = __builtin_bit_cast(pf_bf16x8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
          acc[rt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vav, pbv, acc[rt][t], 0, 0, 0);
        }
      }
    }
  };

  // okm: the stage's page validity bits, taken when its copy was issued (the window may move on since)
  auto run_stage = [&](int n, const unsigned char* st, unsigned okm, auto&& hook) __attribute__((always_inline)) {
    const int kb0 = n * PF_KEYS;
    if (wave_live && kb0 <= ctx + j_last_w) {   // the wave sees at least one key of this stage
      if (kb0 + PF_KEYS > kv_total || okm != 0xFu)
        compute(st, kb0, okm, std::integral_constant<int, 2>{}, hook);
      else if (kb0 + PF_KEYS - 1 > ctx + j_first_w)
        compute(st, kb0, okm, std::integral_constant<int, 1>{}, hook);
      else
        compute(st, kb0, okm, std::integral_constant<int, 0>{}, hook);
    } else {
      hook();
    }
  };
  auto issue = [&](int n, int buf) __attribute__((always_inline)) {
    unsigned okm = 0;
    if (n < st1) {
      if (n - win0 >= 16) load_window(n);
      okm = stage_ok(n);
      dma_stage(n, buf);
    }
    return okm;
  };
  // The copy of stage n+1 runs while stage n is multiplied; the barrier before a stage makes every wave's
  // copies of it visible and frees the other buffer. Group 0 issues its copies right after the barrier and
  // group 1 once its score products are issued (hook), so the two groups' 64 KB of copy instructions do not
  // queue at the CU's vector-memory path at the same moment (the issuing wave stalls while they do; 28.7 ->
  // 28.0 us at config 4, bits unchanged). A window of 16 stages of block ids is refreshed between stages. A
  // group whose key range is shorter idles through the last iteration.
  load_window(st0);
  unsigned ok_cur = issue(st0, 0);
  for (int i = 0; i < n_iter; ++i) {
    const int n = st0 + i;
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    const int buf = i & 1;
    unsigned ok_next = 0;
    auto hook = [&]() __attribute__((always_inline)) {
      if (gi == 1) ok_next = issue(n + 1, buf ^ 1);
    };
    if (gi == 0) ok_next = issue(n + 1, buf ^ 1);
    if (n < st1) run_stage(n, glds + buf * L::STAGE, ok_cur, hook);
    else hook();
    ok_cur = ok_next;
  }

#pragma unroll
  for (int rt = 0; rt < PF_R; ++rt) l_run[rt] = pf_sum4(l_run[rt]);
  // ---- the two groups' states meet in LDS. Group g keeps output tiles [g NT/2, (g + 1) NT/2) (its half):
  // it hands its (m, l) and the other half of its accumulators to the other group and folds that group's
  // values of its own half into its own. The fold takes key range 2 part (group 0) first, x0 a0 + x1 a1
  // with one fixed rounding point, so both groups compute the same (m, l) and the bits do not depend on
  // which group folds. From here on each group writes, publishes and merges its half only.
  constexpr int NH2 = NT / 2;
  using G0 = std::integral_constant<int, 0>;
  using G1 = std::integral_constant<int, 1>;
  float* xml = reinterpret_cast<float*>(lds);                       // [group][rt][2][256 threads]
  pf_float4_t* xacc = reinterpret_cast<pf_float4_t*>(lds + 8192);   // [group][rt][NT/2][256 threads]
  auto hand_over = [&](auto g_c) __attribute__((always_inline)) {
    constexpr int G = decltype(g_c)::value;
#pragma unroll
    for (int rt = 0; rt < PF_R; ++rt) {
      xml[((G * PF_R + rt) * 2) * PF_THREADS + tid] = m_run[rt];
      xml[((G * PF_R + rt) * 2 + 1) * PF_THREADS + tid] = l_run[rt];
#pragma unroll
      for (int j = 0; j < NH2; ++j) xacc[((G * PF_R + rt) * NH2 + j) * PF_THREADS + tid] = acc[rt][(1 - G) * NH2 + j];
    }
  };
  auto fold_half = [&](auto g_c) __attribute__((always_inline)) {
    constexpr int G = decltype(g_c)::value;
#pragma unroll
    for (int rt = 0; rt < PF_R; ++rt) {
      const float mo = xml[(((1 - G) * PF_R + rt) * 2) * PF_THREADS + tid];
      const float lo = xml[(((1 - G) * PF_R + rt) * 2 + 1) * PF_THREADS + tid];
      const float m0 = G == 0 ? m_run[rt] : mo, m1 = G == 0 ? mo : m_run[rt];
      const float l0 = G == 0 ? l_run[rt] : lo, l1 = G == 0 ? lo : l_run[rt];
      const float Mn = fmaxf(m0, m1);
      const float a0 = m0 == -INFINITY ? 0.f : exp2f(m0 - Mn), a1 = m1 == -INFINITY ? 0.f : exp2f(m1 - Mn);
      l_run[rt] = __builtin_fmaf(l0, a0, l1 * a1);
      m_run[rt] = Mn;
#pragma unroll
      for (int j = 0; j < NH2; ++j) {
        const pf_float4_t v = xacc[(((1 - G) * PF_R + rt) * NH2 + j) * PF_THREADS + tid];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float own = acc[rt][G * NH2 + j][c];
          acc[rt][G * NH2 + j][c] = __builtin_fmaf(G == 0 ? own : v[c], a0, (G == 0 ? v[c] : own) * a1);
        }
      }
    }
  };
  __syncthreads();   // every wave is done with the stage buffers
  if (gi == 0) hand_over(G0{}); else hand_over(G1{});
  __syncthreads();
  if (gi == 0) fold_half(G0{}); else fold_half(G1{});

  // The output tile goes out through LDS: each group stages its half of every query row (lane holds, for
  // query tile rt and output tile t, query c16 at dims 16 t + 4 r4 .. + 3), then the workgroup stores whole
  // rows, 16 bytes per lane (a wave instruction writes four rows of HD * 2 contiguous bytes), instead of
  // 16 rows x 32 bytes per instruction from the fragments.
  constexpr int OPITCH = HD + 16;   // bytes per staged half row (HD / 2 bf16 + 16 bytes of bank padding)
  unsigned char* obuf = lds + 8192 + 2 * PF_R * NH2 * PF_THREADS * 16;   // [half][128 rows][OPITCH]
  static_assert(8192 + 2 * PF_R * NH2 * PF_THREADS * 16 + 2 * PF_QT * OPITCH <= PF_GROUPS * 2 * L::STAGE,
                "output staging fits the workgroup's LDS");
  auto write_half = [&](auto g_c, int rt, const pf_float4_t* o, float inv) __attribute__((always_inline)) {
    constexpr int G = decltype(g_c)::value;
    unsigned char* orow = obuf + (G * PF_QT + 16 * PF_R * w + 16 * rt + c16) * OPITCH;
#pragma unroll
    for (int j = 0; j < NH2; ++j)
      *reinterpret_cast<uint2*>(orow + 32 * j + 8 * r4) =
          make_uint2(pf_bf16x2(o[j][0] * inv, o[j][1] * inv), pf_bf16x2(o[j][2] * inv, o[j][3] * inv));
  };
  // after a barrier: rows qbase .. min(qbase + QT, T) - 1 of the staged tile to out, 16 bytes per lane
  auto store_tile = [&]() __attribute__((always_inline)) {
    constexpr int CPR = HD / 8;   // 16-byte chunks per row
    const int rows = min(PF_QT, T - qbase);
#pragma unroll
    for (int i = 0; i < PF_QT * CPR / PF_WG_THREADS; ++i) {
      const int c = tid_wg + PF_WG_THREADS * i, row = c / CPR, k = c % CPR;
      const int half = k / (CPR / 2), ch = k % (CPR / 2);
      const uint4 v = *reinterpret_cast<const uint4*>(obuf + (half * PF_QT + row) * OPITCH + 16 * ch);
      if (row < rows)
        *reinterpret_cast<uint4*>(a.out + int64_t(q_start + qbase + row) * a.o_st + int64_t(h) * a.o_sh + 8 * k) = v;
    }
  };
  if (n_parts == 1) {
    auto out_own = [&](auto g_c) __attribute__((always_inline)) {
      constexpr int G = decltype(g_c)::value;
#pragma unroll
      for (int rt = 0; rt < PF_R; ++rt) write_half(g_c, rt, &acc[rt][G * NH2], 1.0f / l_run[rt]);
    };
    if (gi == 0) out_own(G0{}); else out_own(G1{});
    __syncthreads();
    store_tile();
    return;
  }

  // ---- several partitions: each group publishes its half with 16-byte coherent (sc1) buffer stores, the
  // tile's counter, and both groups of the last workgroup to arrive merge their halves in partition order
  const int64_t tile_id = (int64_t(seq) * a.n_heads + h) * a.tiles_max + tile;
  const int64_t unit0 = tile_id * a.parts_max;
  constexpr int SC1 = 16;   // cache policy sc1: device-coherent, bypasses the XCD's L2
  const __amdgpu_buffer_rsrc_t rml = __builtin_amdgcn_make_buffer_rsrc(
      a.ws_ml + unit0 * (PF_R * 2 * PF_THREADS), 0, n_parts * (PF_R * 2 * PF_THREADS * 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t racc = __builtin_amdgcn_make_buffer_rsrc(
      a.ws_acc + unit0 * (PF_R * NT * 4 * PF_THREADS), 0, n_parts * (PF_R * NT * 4 * PF_THREADS * 4), 0x00020000);
  auto ml_off = [&](int x, int rt, int which) { return (((x * PF_R + rt) * 2 + which) * PF_THREADS + tid) * 4; };
  auto acc_off = [&](int x, int rt, int t) { return (((x * PF_R + rt) * NT + t) * PF_THREADS + tid) * 16; };
  auto publish_half = [&](auto g_c) __attribute__((always_inline)) {
    constexpr int G = decltype(g_c)::value;
#pragma unroll
    for (int rt = 0; rt < PF_R; ++rt) {
      if constexpr (G == 0) {   // both groups hold the same (m, l)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(m_run[rt]), rml, ml_off(part, rt, 0), 0, SC1);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(l_run[rt]), rml, ml_off(part, rt, 1), 0, SC1);
      }
#pragma unroll
      for (int j = 0; j < NH2; ++j) {
        const pf_float4_t v = acc[rt][G * NH2 + j];
        __builtin_amdgcn_raw_buffer_store_b128(
            pub_u32x4_t{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])},
            racc, acc_off(part, rt, G * NH2 + j), 0, SC1);
      }
    }
  };
  if (gi == 0) publish_half(G0{}); else publish_half(G1{});
  publish_complete();
  __syncthreads();
  if (tid_wg == 0) {
    const unsigned prev = publish_count(a.cnt + tile_id * a.cstride);
    const unsigned last = prev == unsigned(n_parts - 1);
    if (last) publish_reset(a.cnt + tile_id * a.cstride);
    s_last = last;
  }
  __syncthreads();
  if (s_last == 0u) return;
  acquire_published();
  auto merge_half = [&](auto g_c) __attribute__((always_inline)) {
    constexpr int G = decltype(g_c)::value;
    if (n_parts == 2) {
      // Two partitions (what the plan gives the longest tiles): the other one's half is loaded in one round
      // trip and combined with this one's, kept in registers, as p0 a0 + p1 a1 (the bits do not depend on
      // which of the two merges).
      const int other = part ^ 1;
      float pm[PF_R], pl[PF_R];
      pub_u32x4_t u[PF_R][NH2];
#pragma unroll
      for (int rt = 0; rt < PF_R; ++rt) {
        pm[rt] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rml, ml_off(other, rt, 0), 0, SC1));
        pl[rt] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rml, ml_off(other, rt, 1), 0, SC1));
#pragma unroll
        for (int j = 0; j < NH2; ++j)
          u[rt][j] = __builtin_amdgcn_raw_buffer_load_b128(racc, acc_off(other, rt, G * NH2 + j), 0, SC1);
      }
#pragma unroll
      for (int rt = 0; rt < PF_R; ++rt) {
        const float m0 = part == 0 ? m_run[rt] : pm[rt], m1 = part == 0 ? pm[rt] : m_run[rt];
        const float l0 = part == 0 ? l_run[rt] : pl[rt], l1 = part == 0 ? pl[rt] : l_run[rt];
        const float Mx = fmaxf(m0, m1);
        const float a0 = m0 == -INFINITY ? 0.f : exp2f(m0 - Mx), a1 = m1 == -INFINITY ? 0.f : exp2f(m1 - Mx);
        const float Ls = __builtin_fmaf(l0, a0, l1 * a1);
        pf_float4_t o[NH2];
#pragma unroll
        for (int j = 0; j < NH2; ++j)
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const float v = __uint_as_float(u[rt][j][c]), own = acc[rt][G * NH2 + j][c];
            o[j][c] = __builtin_fmaf(part == 0 ? own : v, a0, (part == 0 ? v : own) * a1);
          }
        write_half(g_c, rt, o, 1.0f / Ls);
      }
      return;
    }
    // More partitions: fold them in partition order with a running maximum (the result does not depend on
    // which partition merges), PF_MB per round trip; the own partition is read back like the others.
#pragma unroll
    for (int rt = 0; rt < PF_R; ++rt) {
      float M = -INFINITY, Lsum = 0.f;
      pf_float4_t O[NH2];
#pragma unroll
      for (int j = 0; j < NH2; ++j) O[j] = pf_float4_t{0.f, 0.f, 0.f, 0.f};
      for (int x0 = 0; x0 < n_parts; x0 += PF_MB) {
        pub_u32x4_t u[PF_MB][NH2];
        float pm[PF_MB], pl[PF_MB];
#pragma unroll
        for (int e = 0; e < PF_MB; ++e) {
          const int x = min(x0 + e, n_parts - 1);   // slots past the end re-load the last partition (unused)
          pm[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rml, ml_off(x, rt, 0), 0, SC1));
          pl[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rml, ml_off(x, rt, 1), 0, SC1));
#pragma unroll
          for (int j = 0; j < NH2; ++j)
            u[e][j] = __builtin_amdgcn_raw_buffer_load_b128(racc, acc_off(x, rt, G * NH2 + j), 0, SC1);
        }
#pragma unroll
        for (int e = 0; e < PF_MB; ++e) {
          if (x0 + e < n_parts) {
            const float Mn = fmaxf(M, pm[e]);
            const float a_old = M == -INFINITY ? 0.f : exp2f(M - Mn);
            const float a_new = pm[e] == -INFINITY ? 0.f : exp2f(pm[e] - Mn);
            Lsum = __builtin_fmaf(Lsum, a_old, pl[e] * a_new);
#pragma unroll
            for (int j = 0; j < NH2; ++j)
#pragma unroll
              for (int c = 0; c < 4; ++c) O[j][c] = __builtin_fmaf(O[j][c], a_old, __uint_as_float(u[e][j][c]) * a_new);
            M = Mn;
          }
        }
      }
      write_half(g_c, rt, O, 1.0f / Lsum);
    }
  };
  if (gi == 0) merge_half(G0{}); else merge_half(G1{});
  __syncthreads();
  store_tile();
}

inline size_t pf_align256(size_t x) { return (x + 255) & ~size_t(255); }

// Partition plan: ps, the most stages one group's key range may hold, and parts, the workgroups per tile (the
// grid's and the workspace's stride; a workgroup takes two key ranges). ps is the smallest value >=
// PF_PS_MIN whose workgroup count -- every tile of n_seqs sequences with max_new new tokens on
// max_kv - max_new cached ones, split into ceil(stages / (2 ps)) workgroups -- stays within PF_SLOTS; with
// none, one workgroup per tile. A function of the arguments only, so the workspace query and the launch
// agree.
struct PfPlan {
  int ps, parts, tiles;
};
inline PfPlan prefill_plan(int n_seqs, int n_heads, int max_new, int max_kv) {
  const int tiles = (max_new + PF_QT - 1) / PF_QT;
  const int ctx = std::max(0, max_kv - max_new);
  auto stages = [&](int kv) { return ((kv + PF_PAGE - 1) / PF_PAGE + PF_NP - 1) / PF_NP; };
  const int n_st_max = std::max(1, stages(max_kv));
  auto wgs = [&](int ps) {
    int64_t n = 0;
    for (int t = 0; t < tiles; ++t) n += (stages(ctx + std::min(PF_QT * (t + 1), max_new)) + 2 * ps - 1) / (2 * ps);
    return n * n_seqs * n_heads;
  };
  int lo = std::min(PF_PS_MIN, n_st_max), hi = n_st_max;
  if (wgs(lo) > PF_SLOTS) {   // smallest ps in (lo, hi] that fits, or hi
    while (hi - lo > 1) {
      const int mid = (lo + hi) / 2;
      if (wgs(mid) <= PF_SLOTS) hi = mid; else lo = mid;
    }
    lo = hi;
  }
  return PfPlan{lo, (n_st_max + 2 * lo - 1) / (2 * lo), tiles};
}


// Host side shared by the launches that run prefill workgroups: the workspace the plan needs, and the
// argument checks and kernel arguments of one call (n_wg_out: its workgroups, 0 when there is nothing to do).
inline size_t prefill_workspace_need(int n_seqs, int n_heads, int head_dim, int max_new, int max_kv) {
  if (n_seqs <= 0 || n_heads <= 0 || max_new <= 0 || max_kv <= 0) return 0;
  if (head_dim != 64 && head_dim != 128) return 0;
  const PfPlan plan = prefill_plan(n_seqs, n_heads, max_new, max_kv);
  if (plan.parts <= 1) return 0;
  const size_t units = size_t(plan.tiles) * n_seqs * n_heads * plan.parts;
  return WS_COUNTER_BYTES + pf_align256(units * PF_R * 2 * PF_THREADS * sizeof(float)) +
         pf_align256(units * PF_R * (head_dim / 16) * 4 * PF_THREADS * sizeof(float));
}

inline int prefill_prepare(const void* q, int64_t q_st, int64_t q_sh, const void* k_pool, const void* v_pool,
                           int64_t kv_sblk, int64_t kv_spos, int64_t kv_sh, const int32_t* block_tables, int64_t bt_sb,
                           const int32_t* seq_info, int n_seqs, int max_new, int max_kv, void* out, int64_t o_st,
                           int64_t o_sh, int n_heads, int n_kv_heads, int head_dim, int block_size, int max_blocks,
                           int num_blocks, float scale, int dtype, void* workspace, size_t workspace_bytes,
                           PrefillArgs* a_out, int64_t* n_wg_out) {
  NS_REQUIRE(dtype == NS_DTYPE_BF16, "paged_attention_prefill: dtype %d not supported (bf16 only)", dtype);
  NS_REQUIRE(head_dim == 64 || head_dim == 128, "paged_attention_prefill: head_dim %d not in {64, 128}", head_dim);
  NS_REQUIRE(block_size == PF_PAGE, "paged_attention_prefill: block_size %d, the kernel needs %d", block_size, PF_PAGE);
  NS_REQUIRE(n_kv_heads > 0 && n_heads > 0 && n_heads % n_kv_heads == 0,
             "paged_attention_prefill: n_heads %d not a multiple of n_kv_heads %d", n_heads, n_kv_heads);
  NS_REQUIRE(n_seqs >= 0 && n_seqs <= 65535 && n_heads <= 65535, "paged_attention_prefill: %d sequences, %d heads",
             n_seqs, n_heads);
  NS_REQUIRE(max_new >= 0 && max_kv >= max_new, "paged_attention_prefill: max_new %d, max_kv %d", max_new, max_kv);
  NS_REQUIRE(max_blocks >= 1 && num_blocks >= 1, "paged_attention_prefill: max_blocks %d num_blocks %d", max_blocks,
             num_blocks);
  NS_REQUIRE(q_st % 8 == 0 && q_sh % 8 == 0 && kv_sblk % 8 == 0 && kv_spos % 8 == 0 && kv_sh % 8 == 0 &&
                 o_st % 8 == 0 && o_sh % 8 == 0,
             "paged_attention_prefill: strides must be multiples of 8 elements");
  NS_REQUIRE(kv_spos >= 0 && kv_spos * 2 < (int64_t(1) << 26),
             "paged_attention_prefill: token stride %lld too large for 32-bit page offsets", (long long)kv_spos);
  NS_REQUIRE((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_pool) | reinterpret_cast<uintptr_t>(v_pool) |
              reinterpret_cast<uintptr_t>(out)) %
                     16 ==
                 0,
             "paged_attention_prefill: q / k_pool / v_pool / out must be 16-byte aligned");
  *n_wg_out = 0;
  if (n_seqs == 0 || max_new == 0) return NS_OK;
  const PfPlan plan = prefill_plan(n_seqs, n_heads, max_new, max_kv);
  unsigned* cnt = nullptr;
  int cstride = 1;
  float* ws_ml = nullptr;
  float* ws_acc = nullptr;
  if (plan.parts > 1) {
    const size_t need = prefill_workspace_need(n_seqs, n_heads, head_dim, max_new, max_kv);
    if (workspace == nullptr || workspace_bytes < need) {
      set_error("paged_attention_prefill: zero-initialised workspace of %zu bytes needed, got %zu", need,
                workspace == nullptr ? size_t(0) : workspace_bytes);
      return NS_E_WORKSPACE;
    }
    NS_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "paged_attention_prefill: workspace not 256-byte aligned");
    const size_t ntile = size_t(plan.tiles) * n_seqs * n_heads, units = ntile * plan.parts;
    NS_REQUIRE(ntile <= size_t(WS_MAX_COUNTERS), "paged_attention_prefill: %zu query tiles x heads exceed %d",
               ntile, WS_MAX_COUNTERS);
    char* wsb = static_cast<char*>(workspace);
    cnt = reinterpret_cast<unsigned*>(wsb);
    cstride = ws_counter_stride(ntile, size_t(WS_MAX_COUNTERS));
    ws_ml = reinterpret_cast<float*>(wsb + WS_COUNTER_BYTES);
    ws_acc = reinterpret_cast<float*>(wsb + WS_COUNTER_BYTES + pf_align256(units * PF_R * 2 * PF_THREADS * sizeof(float)));
  }
  *a_out = PrefillArgs{static_cast<const bf16_t*>(q), q_st, q_sh, static_cast<const bf16_t*>(k_pool),
                static_cast<const bf16_t*>(v_pool), kv_sblk, kv_spos, kv_sh, block_tables, bt_sb, seq_info,
                static_cast<bf16_t*>(out), o_st, o_sh, n_heads / n_kv_heads, max_blocks, num_blocks, n_heads,
                n_seqs, scale * PF_LOG2E, plan.tiles, plan.parts, plan.ps, cnt, cstride, ws_ml, ws_acc};
  const int64_t n_wg = int64_t(n_heads) * plan.tiles * plan.parts * n_seqs;   // an upper bound on the units
  NS_REQUIRE(n_wg < (int64_t(1) << 31), "paged_attention_prefill: %lld workgroups", (long long)n_wg);
  *n_wg_out = n_wg;
  return NS_OK;
}
}  // namespace

}  // namespace ns
