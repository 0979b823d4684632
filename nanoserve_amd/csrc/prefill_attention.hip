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
//   * Work unit = (head, tile of QT = 64 queries, partition of the tile's keys). A workgroup is 4 waves;
//     wave w owns queries 16w .. 16w+15, one per MFMA column. A tile's keys (64-key stages of 4 pages) are
//     split into partitions of about PS stages, so a long prefill spreads over many workgroups instead
//     of a few long ones; the grid axis runs over tiles from the last (longest) down.
//   * K/V go straight from HBM into LDS (global_load_lds, 16 bytes per lane; wave w copies page w of a
//     stage), double-buffered: the copy of stage n+1 runs while stage n is multiplied. Block ids come
//     from a window of 64 table entries held one per lane and read with readlane. K rows are stored with
//     XOR-swizzled 16-byte chunks so fragment reads are free of bank conflicts. Two workgroups fit a CU
//     (64 KB of LDS each), two waves per SIMD, so one wave's softmax overlaps the other's products.
//   * Per stage and wave, on the matrix cores (mfma 16x16x32 bf16 throughout):
//       S^T[16 keys x 16 queries] = K_page[16 x hd] . Q^T[hd x 16]                      4 pages
//       O^T[hd x 16 queries]    += V^T[hd x 32 keys] . P^T[32 keys x 16 queries]       2 key steps
//     S^T comes out with lane = query and 4 consecutive keys per lane; two pages' worth is the 8-key
//     B operand of P^T, so P never leaves registers. V^T fragments are built from LDS rows by a 4x4
//     register transpose (v_perm), with the output rows relabelled so every LDS read is a contiguous
//     row slice. The softmax reference point moves only when a score exceeds it by 2^8, so the
//     accumulator is rescaled rarely.
//   * Masks are computed only on stages that cross a query's diagonal or the end of the keys: key k is
//     visible to query j iff k <= ctx + j, and keys at or past ctx + T (unwritten slots of the last
//     page, pages past the tile's reach) are zeroed in V as well, so garbage there can never turn 0 * x
//     into NaN. Block ids outside [0, num_blocks) are masked pages.
//   * A tile split over several partitions: each partition publishes its (m, l, acc) with agent-scope
//     stores, waits for them to complete and bumps the tile's arrival counter; the last to arrive merges
//     all partitions in partition order (the result does not depend on arrival order) and writes the
//     output. One launch; the workspace counters are left at zero.
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
constexpr int PF_WAVES = 4;
constexpr int PF_THREADS = PF_WAVES * 64;
constexpr int PF_R = 1;                     // 16-query MFMA tiles per wave (2 halves the LDS reads per
                                            // product but needs 2x the registers: one wave per SIMD)
constexpr int PF_QT = 16 * PF_R * PF_WAVES; // queries per work unit
constexpr int PF_PS = 8;                    // target stages per partition
constexpr int PF_MB = 4;                    // partitions merged per memory round trip
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
  static __device__ __forceinline__ int key(int t) { return HD == 128 ? (t & 15) : ((t >> 1) & 7); }
  // V rows likewise, by an even key from the row's low bits: a transpose read takes a 32-byte chunk pair
  // (2 chunks) from each of four consecutive rows, and XOR by even values moves whole pairs, so the four
  // rows' pairs land in four different bank groups.
  static __device__ __forceinline__ int vkey(int t) { return (t & (CH / 2 - 1)) << 1; }
};
static_assert(PF_NP == PF_WAVES, "each wave stages one page of a stage");

__device__ __forceinline__ uint32_t pf_pack_lo(uint32_t x, uint32_t y) { return __builtin_amdgcn_perm(y, x, 0x05040100u); }
__device__ __forceinline__ uint32_t pf_pack_hi(uint32_t x, uint32_t y) { return __builtin_amdgcn_perm(y, x, 0x07060302u); }

// two fp32 -> packed bf16 (round to nearest even; v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pf_bf16x2(float lo, float hi) {
  typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
  bf16x2_t r;
  r[0] = static_cast<__bf16>(lo);
  r[1] = static_cast<__bf16>(hi);
  return __builtin_bit_cast(uint32_t, r);
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
  int G, max_blocks, num_blocks, n_heads;
  float scale_log2;
  int tiles_max, parts_max;
  unsigned* cnt;                    // [S, n_heads, tiles_max] arrival counters (zero between calls)
  float* ws_ml;                     // [unit][R][256 threads] (m, l)
  float* ws_acc;                    // [unit][R * NT][256 threads] float4
};

template <int HD>
__global__ __launch_bounds__(PF_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void paged_prefill_bf16_kernel(PrefillArgs a) {
  using L = PfLds<HD>;
  constexpr int KS = HD / 32;   // k-steps of Q.K^T
  constexpr int NT = HD / 16;   // output tiles of P.V
  constexpr int VW = NT / 2;    // dwords of a lane's V row slice
  __shared__ __align__(16) unsigned char lds_a[L::STAGE];   // stages st0, st0 + 2, ...
  __shared__ __align__(16) unsigned char lds_b[L::STAGE];   // stages st0 + 1, st0 + 3, ...
  __shared__ unsigned s_last;

  const int h = blockIdx.x, seq = blockIdx.z;
  const int tile_rev = int(blockIdx.y) / a.parts_max, part = int(blockIdx.y) - tile_rev * a.parts_max;
  const int q_start = a.info[4 * seq + 0], T = a.info[4 * seq + 1], ctx = a.info[4 * seq + 2];
  const int n_tiles = (T + PF_QT - 1) / PF_QT;
  if (tile_rev >= n_tiles || n_tiles > a.tiles_max) return;   // the second: n_new above the caller's max_new
  const int tile = n_tiles - 1 - tile_rev;
  const int qbase = tile * PF_QT;
  const int j_last_wg = min(qbase + PF_QT - 1, T - 1);
  const int kv_end = ctx + j_last_wg + 1;   // keys this tile can see
  const int kv_total = ctx + T;             // keys that exist
  int n_pages = (kv_end + PF_PAGE - 1) / PF_PAGE;
  if (n_pages > a.max_blocks) n_pages = a.max_blocks;
  const int n_st = (n_pages + PF_NP - 1) / PF_NP;
  const int n_parts = min((n_st + PF_PS - 1) / PF_PS, a.parts_max);
  if (part >= n_parts) return;
  const int st0 = part * n_st / n_parts, st1 = (part + 1) * n_st / n_parts;
  const int g = h / a.G;
  const int32_t* table = a.bt + int64_t(seq) * a.bt_sb;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
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
  auto dma_stage = [&](int n, unsigned char* buf) __attribute__((always_inline)) {
    const int id = __builtin_amdgcn_readlane(pid, PF_NP * (n - win0) + w);
    const int64_t base = int64_t(id) * a.s_blk + int64_t(g) * a.s_h;
    unsigned char* kd = buf + w * (PF_PAGE * L::ROW);
    unsigned char* vd = kd + L::K_BYTES;
#pragma unroll
    for (int i = 0; i < L::IPP; ++i) {
      const int t = L::TPI * i + lane / L::CH, cp = lane % L::CH;   // the LDS slot this lane fills
      const int64_t row = base + int64_t(t) * a.s_pos;
      __builtin_amdgcn_global_load_lds(
          (__attribute__((address_space(1))) void*)(a.kp + row + 8 * (cp ^ L::key(t))),
          (__attribute__((address_space(3))) void*)(kd + 1024 * i), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)(a.vp + row + 8 * (cp ^ L::vkey(t))),
                                       (__attribute__((address_space(3))) void*)(vd + 1024 * i), 16, 0, 0);
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

  // One stage on the matrix cores. MASK: the stage crosses a diagonal or the end of the keys, or holds a
  // bad block id; otherwise every key is visible to every query of the wave.
  auto compute = [&](const unsigned char* st, int kb0, unsigned okm, auto mask_c) __attribute__((always_inline)) {
    constexpr bool MASK = decltype(mask_c)::value;
    bool okp[PF_NP];
#pragma unroll
    for (int pp = 0; pp < PF_NP; ++pp) okp[pp] = MASK ? ((okm >> pp) & 1u) != 0 : true;
    // ---- scores of both query tiles, page by page (each K fragment read once, used twice)
    pf_float4_t sc[PF_R][PF_NP];
#pragma unroll
    for (int pp = 0; pp < PF_NP; ++pp) {
      const unsigned char* krow = st + (PF_PAGE * pp + c16) * L::ROW;
      const int kk = L::key(c16);
      pf_bf16x8_t kf[KS];
#pragma unroll
      for (int s = 0; s < KS; ++s)
        kf[s] = __builtin_bit_cast(pf_bf16x8_t, *reinterpret_cast<const uint4*>(krow + 16 * ((4 * s + r4) ^ kk)));
#pragma unroll
      for (int rt = 0; rt < PF_R; ++rt) {
        sc[rt][pp] = pf_float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; ++s)
          sc[rt][pp] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[s], qf[rt][s], sc[rt][pp], 0, 0, 0);
      }
    }
    // ---- probabilities: P^T as B operands, k-slot e = key 4*r4 + e of each page
    uint32_t pb[PF_R][PF_NP][2];
#pragma unroll
    for (int rt = 0; rt < PF_R; ++rt) {
      float mx = -INFINITY;
#pragma unroll
      for (int pp = 0; pp < PF_NP; ++pp)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (MASK) {
            const int key = kb0 + PF_PAGE * pp + 4 * r4 + e;
            if (!(okp[pp] && key <= ctx + jrow[rt])) sc[rt][pp][e] = -INFINITY;
          }
          mx = fmaxf(mx, sc[rt][pp][e]);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      // Reference point m (scaled units, c = scale * log2(e)): weights are exp2(s * c - m). It moves
      // only when a score exceeds it by more than PF_SLACK, so weights stay below 2^PF_SLACK and the
      // accumulator is rescaled rarely. The normalised result is the same function of the scores; only
      // the bf16 rounding of individual weights (relative 2^-9) depends on where m sits.
      const float mxc = mx * a.scale_log2;
      const bool move = mxc > m_run[rt] + PF_SLACK;
      const float m_new = move ? mxc : m_run[rt];
      const float mc = m_new == -INFINITY ? 0.f : m_new;   // nothing visible yet: weights 0
      const float alpha = __builtin_amdgcn_exp2f(m_run[rt] - mc);
      m_run[rt] = m_new;
      float psum = 0.f;
#pragma unroll
      for (int pp = 0; pp < PF_NP; ++pp) {
        float pv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pv[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[rt][pp][e], a.scale_log2, -mc));
          psum += pv[e];
        }
        pb[rt][pp][0] = pf_bf16x2(pv[0], pv[1]);
        pb[rt][pp][1] = pf_bf16x2(pv[2], pv[3]);
      }
      l_run[rt] = l_run[rt] * alpha + psum;
      if (__ballot(move)) {   // the reference point moved for some query of the wave
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[rt][t] *= alpha;
      }
    }
    // ---- P.V over two 32-key steps: k-slots 0..3 = page 2*ks2 keys 4*r4 + e, 4..7 = page 2*ks2 + 1.
    // V^T fragments come straight from LDS by transpose reads (ds_read_b64_tr_b16): within each group of
    // 16 lanes, lane j addresses 4 dims (16t + 4 (j % 4) ..) of key row kb + j / 4, and lane i receives
    // dim 16t + i of keys kb .. kb + 3 -- its A-operand slots for one page. Built once per step, they feed
    // every query tile.
#pragma unroll
    for (int ks2 = 0; ks2 < 2; ++ks2) {
      v4i16_t va[2][NT];
#pragma unroll
      for (int hp = 0; hp < 2; ++hp) {
        const int pp = 2 * ks2 + hp;
        const int vr = PF_PAGE * pp + 4 * r4 + (c16 >> 2);   // the key row this lane addresses
        const unsigned char* vrow = st + L::K_BYTES + vr * L::ROW;
        uint32_t m01 = 0xffffffffu, m23 = 0xffffffffu;
        if constexpr (MASK) {   // keys that do not exist read as 0
          const int key0 = kb0 + PF_PAGE * pp + 4 * r4;
          const bool ok = okp[pp];
          m01 = (ok && key0 + 0 < kv_total ? 0x0000ffffu : 0u) | (ok && key0 + 1 < kv_total ? 0xffff0000u : 0u);
          m23 = (ok && key0 + 2 < kv_total ? 0x0000ffffu : 0u) | (ok && key0 + 3 < kv_total ? 0xffff0000u : 0u);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const int dim = 16 * t + 4 * (c16 & 3);
          const int chunk = dim >> 3;
          const unsigned char* src = vrow + 16 * (chunk ^ L::vkey(vr)) + 2 * (dim & 7);
          v4i16_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16_t*)(src));
          if constexpr (MASK) {
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
        const pf_bf16x8_t pbv = __builtin_bit_cast(
            pf_bf16x8_t, make_uint4(pb[rt][2 * ks2][0], pb[rt][2 * ks2][1], pb[rt][2 * ks2 + 1][0], pb[rt][2 * ks2 + 1][1]));
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
  auto run_stage = [&](int n, const unsigned char* st, unsigned okm) __attribute__((always_inline)) {
    const int kb0 = n * PF_KEYS;
    if (wave_live && kb0 <= ctx + j_last_w) {   // the wave sees at least one key of this stage
      if (kb0 + PF_KEYS - 1 <= ctx + j_first_w && okm == 0xFu)
        compute(st, kb0, okm, std::false_type{});
      else
        compute(st, kb0, okm, std::true_type{});
    }
  };
  auto issue = [&](int n, unsigned char* buf) __attribute__((always_inline)) {
    unsigned okm = 0;
    if (n < st1) {
      if (n - win0 >= 16) load_window(n);
      okm = stage_ok(n);
      dma_stage(n, buf);
    }
    return okm;
  };
  // The copy of stage n+1 runs while stage n is multiplied; the barrier before a stage makes every wave's
  // copies of it visible and frees the other buffer. A window of 16 stages of block ids is refreshed
  // between stages.
  load_window(st0);
  unsigned ok_a = issue(st0, lds_a), ok_b = 0;
  for (int n = st0; n < st1; n += 2) {
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    ok_b = issue(n + 1, lds_b);
    run_stage(n, lds_a, ok_a);
    if (n + 1 >= st1) break;
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    ok_a = issue(n + 2, lds_a);
    run_stage(n + 1, lds_b, ok_b);
  }
  __syncthreads();

#pragma unroll
  for (int rt = 0; rt < PF_R; ++rt) {
    l_run[rt] += __shfl_xor(l_run[rt], 16, 64);
    l_run[rt] += __shfl_xor(l_run[rt], 32, 64);
  }
  // lane holds, for query tile rt, tile t and r = 0..3, query c16 at dim 16 t + 4 r4 + r
  auto write_out = [&](int rt, const pf_float4_t (&o)[NT], float inv) __attribute__((always_inline)) {
    if (jq[rt] >= T) return;
    bf16_t* orow = a.out + int64_t(q_start + jq[rt]) * a.o_st + int64_t(h) * a.o_sh;
#pragma unroll
    for (int t = 0; t < NT; ++t)
      *reinterpret_cast<uint2*>(orow + 16 * t + 4 * r4) =
          make_uint2(pf_bf16x2(o[t][0] * inv, o[t][1] * inv), pf_bf16x2(o[t][2] * inv, o[t][3] * inv));
  };
  if (n_parts == 1) {
#pragma unroll
    for (int rt = 0; rt < PF_R; ++rt) write_out(rt, acc[rt], 1.0f / l_run[rt]);
    return;
  }

  // ---- several partitions: publish, count, and the last to arrive merges in partition order
  const int64_t tile_id = (int64_t(seq) * a.n_heads + h) * a.tiles_max + tile;
  const int64_t unit0 = tile_id * a.parts_max;
#pragma unroll
  for (int rt = 0; rt < PF_R; ++rt) {
    float* ml = a.ws_ml + ((unit0 + part) * PF_R + rt) * (2 * PF_THREADS);
    publish_store(ml + tid, m_run[rt]);
    publish_store(ml + PF_THREADS + tid, l_run[rt]);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const pub_u32x4_t bits = {__float_as_uint(acc[rt][t][0]), __float_as_uint(acc[rt][t][1]),
                                __float_as_uint(acc[rt][t][2]), __float_as_uint(acc[rt][t][3])};
      publish_store16(a.ws_acc + (((unit0 + part) * PF_R + rt) * NT + t) * (4 * PF_THREADS) + 4 * tid, bits);
    }
  }
  publish_complete();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = publish_count(a.cnt + tile_id);
    const unsigned last = prev == unsigned(n_parts - 1);
    if (last) publish_reset(a.cnt + tile_id);
    s_last = last;
  }
  __syncthreads();
  if (s_last == 0u) return;
  acquire_published();
#pragma unroll
  for (int rt = 0; rt < PF_R; ++rt) {
    float M = -INFINITY, Lsum = 0.f;
    pf_float4_t O[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) O[t] = pf_float4_t{0.f, 0.f, 0.f, 0.f};
    for (int x0 = 0; x0 < n_parts; x0 += PF_MB) {
      pub_u32x4_t u[PF_MB * NT];
      float pm[PF_MB], pl[PF_MB];
#pragma unroll
      for (int e = 0; e < PF_MB; ++e) {
        const int x = min(x0 + e, n_parts - 1);
        const float* ml = a.ws_ml + ((unit0 + x) * PF_R + rt) * (2 * PF_THREADS);
        pm[e] = publish_load(ml + tid);
        pl[e] = publish_load(ml + PF_THREADS + tid);
#pragma unroll
        for (int t = 0; t < NT; ++t)
          u[e * NT + t] = publish_load16(a.ws_acc + (((unit0 + x) * PF_R + rt) * NT + t) * (4 * PF_THREADS) + 4 * tid);
      }
#pragma unroll
      for (int e = 0; e < PF_MB; ++e) {
        if (x0 + e < n_parts) {
          const float Mn = fmaxf(M, pm[e]);
          const float a_old = M == -INFINITY ? 0.f : exp2f(M - Mn);
          const float a_new = pm[e] == -INFINITY ? 0.f : exp2f(pm[e] - Mn);
          Lsum = Lsum * a_old + pl[e] * a_new;
#pragma unroll
          for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int c = 0; c < 4; ++c) O[t][c] = O[t][c] * a_old + __uint_as_float(u[e * NT + t][c]) * a_new;
          M = Mn;
        }
      }
    }
    write_out(rt, O, 1.0f / Lsum);
  }
}

int prefill_parts_max(int max_kv) {
  const int n_st = ((max_kv + PF_PAGE - 1) / PF_PAGE + PF_NP - 1) / PF_NP;
  return std::max(1, (n_st + PF_PS - 1) / PF_PS);
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

}  // namespace

}  // namespace ns

using namespace ns;

// Workspace: the fixed counter region (one arrival counter per tile of [n_seqs, n_heads, tiles]; shared
// safely by calls of any shape), then per work unit the (m, l) and the accumulators of a tile's partition.
// Zero bytes when no tile can span more than one partition.
extern "C" size_t ns_prefill_workspace_bytes(int n_seqs, int n_heads, int head_dim, int max_new, int max_kv) {
  if (n_seqs <= 0 || n_heads <= 0 || max_new <= 0 || max_kv <= 0) return 0;
  if (head_dim != 64 && head_dim != 128) return 0;
  const int parts = prefill_parts_max(max_kv);
  if (parts <= 1) return 0;
  const size_t tiles = size_t((max_new + PF_QT - 1) / PF_QT) * n_seqs * n_heads;
  const size_t units = tiles * parts;
  return WS_COUNTER_BYTES + align256(units * PF_R * 2 * PF_THREADS * sizeof(float)) +
         align256(units * PF_R * (head_dim / 16) * 4 * PF_THREADS * sizeof(float));
}

extern "C" int ns_paged_attn_prefill(const void* q, int64_t q_st, int64_t q_sh, const void* k_pool, const void* v_pool,
                                     int64_t kv_sblk, int64_t kv_spos, int64_t kv_sh, const int32_t* block_tables,
                                     int64_t bt_sb, const int32_t* seq_info, int n_seqs, int max_new, int max_kv,
                                     void* out, int64_t o_st, int64_t o_sh, int n_heads, int n_kv_heads,
                                     int head_dim, int block_size, int max_blocks, int num_blocks, float scale,
                                     int dtype, void* workspace, size_t workspace_bytes, void* stream) {
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
  NS_REQUIRE((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_pool) | reinterpret_cast<uintptr_t>(v_pool) |
              reinterpret_cast<uintptr_t>(out)) %
                     16 ==
                 0,
             "paged_attention_prefill: q / k_pool / v_pool / out must be 16-byte aligned");
  if (n_seqs == 0 || max_new == 0) return NS_OK;
  const int tiles = (max_new + PF_QT - 1) / PF_QT;
  const int parts = prefill_parts_max(max_kv);
  NS_REQUIRE(int64_t(tiles) * parts <= 65535, "paged_attention_prefill: %d new tokens over %d keys is too many",
             max_new, max_kv);
  unsigned* cnt = nullptr;
  float* ws_ml = nullptr;
  float* ws_acc = nullptr;
  if (parts > 1) {
    const size_t need = ns_prefill_workspace_bytes(n_seqs, n_heads, head_dim, max_new, max_kv);
    if (workspace == nullptr || workspace_bytes < need) {
      set_error("paged_attention_prefill: zero-initialised workspace of %zu bytes needed, got %zu", need,
                workspace == nullptr ? size_t(0) : workspace_bytes);
      return NS_E_WORKSPACE;
    }
    NS_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "paged_attention_prefill: workspace not 256-byte aligned");
    const size_t ntile = size_t(tiles) * n_seqs * n_heads, units = ntile * parts;
    NS_REQUIRE(ntile <= size_t(WS_MAX_COUNTERS), "paged_attention_prefill: %zu query tiles x heads exceed %d",
               ntile, WS_MAX_COUNTERS);
    char* wsb = static_cast<char*>(workspace);
    cnt = reinterpret_cast<unsigned*>(wsb);
    ws_ml = reinterpret_cast<float*>(wsb + WS_COUNTER_BYTES);
    ws_acc = reinterpret_cast<float*>(wsb + WS_COUNTER_BYTES + align256(units * PF_R * 2 * PF_THREADS * sizeof(float)));
  }
  PrefillArgs a{static_cast<const bf16_t*>(q), q_st, q_sh, static_cast<const bf16_t*>(k_pool),
                static_cast<const bf16_t*>(v_pool), kv_sblk, kv_spos, kv_sh, block_tables, bt_sb, seq_info,
                static_cast<bf16_t*>(out), o_st, o_sh, n_heads / n_kv_heads, max_blocks, num_blocks, n_heads,
                scale * PF_LOG2E, tiles, parts, cnt, ws_ml, ws_acc};
  const dim3 grid{unsigned(n_heads), unsigned(tiles * parts), unsigned(n_seqs)};
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (head_dim == 64)
    hipLaunchKernelGGL(paged_prefill_bf16_kernel<64>, grid, dim3(PF_THREADS), 0, s, a);
  else
    hipLaunchKernelGGL(paged_prefill_bf16_kernel<128>, grid, dim3(PF_THREADS), 0, s, a);
  return check_launch("paged_attention_prefill");
}
