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
//   * Grid (n_heads, query tiles, sequences). A workgroup is 4 waves and owns QT = 64 consecutive
//     queries of one head; wave w owns queries 16w .. 16w+15, one per MFMA column. The tile axis runs
//     from the last (longest) tile down, so the longest tiles are dispatched first.
//   * K/V stream through LDS in stages of 4 pages (64 keys), double-buffered: while the waves multiply
//     stage n, the stage n+1 loads (16-byte loads of whole token rows, every thread a share) are in
//     flight, and they are written to the other buffer after the multiply. The stage's 4 block ids are
//     uniform per workgroup (scalar loads).
//   * Per stage and wave, on the matrix cores:
//       S^T[16 keys x 16 queries] = K_page[16 x hd] . Q^T[hd x 16]        (mfma 16x16x32 bf16), 4 pages
//       O^T[hd x 16 queries]    += V_page^T[hd x 16] . P^T[16 x 16]        (mfma 16x16x16 bf16)
//     S^T comes out with lane = query and 4 consecutive keys per lane, which is the B-operand layout of
//     P^T, so P never leaves registers; V^T fragments are built from LDS rows by a 4x4 register
//     transpose (v_perm), with the output rows relabelled so every LDS read is a contiguous row slice.
//     One max / rescale per stage (64 keys), two butterfly shuffles.
//   * Masks: key k is visible to query j iff k <= ctx + j. Keys at or past ctx + T (unwritten slots of
//     the last page, or whole pages past the end of a stage) are zeroed in V as well, so garbage there
//     can never turn 0 * x into NaN. Block ids outside [0, num_blocks) are treated as masked pages.
#include "ns_common.h"

namespace ns {

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 pf_bf16x8_t;
typedef __attribute__((ext_vector_type(4))) short pf_short4_t;
typedef __attribute__((ext_vector_type(4))) float pf_float4_t;

constexpr float PF_LOG2E = 1.4426950408889634f;
constexpr int PF_PAGE = 16;
constexpr int PF_NP = 4;                    // pages per stage
constexpr int PF_KEYS = PF_NP * PF_PAGE;    // 64 keys per stage
constexpr int PF_WAVES = 4;
constexpr int PF_QT = 16 * PF_WAVES;        // queries per workgroup

template <int HD>
struct PfLds {
  static constexpr int KP = HD * 2 + 16;    // K row pitch (bytes): conflict-free 16-byte fragment reads
  static constexpr int VP = HD * 2;         // V row pitch: lanes read consecutive 16-byte slices of a row
  static constexpr int K_BYTES = PF_KEYS * KP;
  static constexpr int STAGE = K_BYTES + PF_KEYS * VP;
  static constexpr int CH = HD / 8;                             // 16-byte chunks per token row
  static constexpr int LOADS = 2 * PF_KEYS * CH / (PF_WAVES * 64);   // chunks per thread per stage
};

__device__ __forceinline__ uint32_t pf_pack_lo(uint32_t x, uint32_t y) { return __builtin_amdgcn_perm(y, x, 0x05040100u); }
__device__ __forceinline__ uint32_t pf_pack_hi(uint32_t x, uint32_t y) { return __builtin_amdgcn_perm(y, x, 0x07060302u); }

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
  int G, max_blocks, num_blocks;
  float scale_log2;
};

template <int HD>
__global__ __launch_bounds__(PF_WAVES * 64) void paged_prefill_bf16_kernel(PrefillArgs a) {
  using L = PfLds<HD>;
  constexpr int KS = HD / 32;   // k-steps of Q.K^T
  constexpr int NT = HD / 16;   // output tiles of P.V
  constexpr int VW = NT / 2;    // dwords of a lane's V row slice
  __shared__ __align__(16) unsigned char lds[2 * L::STAGE];

  const int h = blockIdx.x, seq = blockIdx.z;
  const int q_start = a.info[4 * seq + 0], T = a.info[4 * seq + 1], ctx = a.info[4 * seq + 2];
  const int n_tiles = (T + PF_QT - 1) / PF_QT;
  if (int(blockIdx.y) >= n_tiles) return;
  const int tile = n_tiles - 1 - int(blockIdx.y);
  const int g = h / a.G;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c16 = lane & 15, r4 = lane >> 4;
  const int qbase = tile * PF_QT;
  const int j_last_wg = min(qbase + PF_QT - 1, T - 1);
  const int kv_end = ctx + j_last_wg + 1;                 // keys this workgroup can see
  const int kv_total = ctx + T;                          // keys that exist
  int n_pages = (kv_end + PF_PAGE - 1) / PF_PAGE;
  if (n_pages > a.max_blocks) n_pages = a.max_blocks;
  const int n_st = (n_pages + PF_NP - 1) / PF_NP;
  const int32_t* table = a.bt + int64_t(seq) * a.bt_sb;

  // this lane's query (clamped: rows past T mirror row T-1 and are not stored)
  const int jq = qbase + 16 * w + c16;
  const int jrow = min(jq, T - 1);
  const int j_last_w = min(qbase + 16 * w + 15, T - 1);
  const bool wave_live = qbase + 16 * w < T;
  pf_bf16x8_t qf[KS];
  {
    const bf16_t* qrow = a.q + int64_t(q_start + jrow) * a.q_st + int64_t(h) * a.q_sh;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qf[s] = __builtin_bit_cast(pf_bf16x8_t, *reinterpret_cast<const uint4*>(qrow + 32 * s + 8 * r4));
  }

  // ---- staging: chunk c = tid + 256 i of the stage; K chunks first, then V chunks
  // one vector value (not an array): the compiler keeps it in registers across the loop
  typedef uint32_t Stage __attribute__((ext_vector_type(4 * L::LOADS)));
  auto page_id = [&](int p) __attribute__((always_inline)) {
    // pages past the workgroup's reach re-read the last live page (in bounds; masked below)
    const int pc = min(p, n_pages - 1);
    const int id = table[pc];
    return (id >= 0 && id < a.num_blocks) ? id : 0;
  };
  auto load_stage = [&](int n) __attribute__((always_inline)) {
    Stage stg;
    int ids[PF_NP];
#pragma unroll
    for (int pp = 0; pp < PF_NP; ++pp) ids[pp] = page_id(n * PF_NP + pp);
#pragma unroll
    for (int i = 0; i < L::LOADS; ++i) {
      constexpr int HALF = L::LOADS / 2;
      const bool is_v = i >= HALF;                               // compile-time per i
      const int cc = tid + (is_v ? i - HALF : i) * PF_WAVES * 64;
      const int tok = cc / L::CH, ch = cc - tok * L::CH;
      const int pp = tok >> 4;
      const int id = pp == 0 ? ids[0] : pp == 1 ? ids[1] : pp == 2 ? ids[2] : ids[3];
      const bf16_t* base = (is_v ? a.vp : a.kp) + int64_t(id) * a.s_blk + int64_t(tok & 15) * a.s_pos +
                           int64_t(g) * a.s_h + 8 * ch;
      const uint4 u = *reinterpret_cast<const uint4*>(base);
      stg[4 * i + 0] = u.x;
      stg[4 * i + 1] = u.y;
      stg[4 * i + 2] = u.z;
      stg[4 * i + 3] = u.w;
    }
    return stg;
  };
  auto store_stage = [&](int buf, const Stage& stg) __attribute__((always_inline)) {
    unsigned char* st = lds + buf * L::STAGE;
#pragma unroll
    for (int i = 0; i < L::LOADS; ++i) {
      constexpr int HALF = L::LOADS / 2;
      const bool is_v = i >= HALF;
      const int cc = tid + (is_v ? i - HALF : i) * PF_WAVES * 64;
      const int tok = cc / L::CH, ch = cc - tok * L::CH;
      unsigned char* dst = is_v ? st + L::K_BYTES + tok * L::VP + 16 * ch : st + tok * L::KP + 16 * ch;
      *reinterpret_cast<uint4*>(dst) = make_uint4(stg[4 * i], stg[4 * i + 1], stg[4 * i + 2], stg[4 * i + 3]);
    }
  };

  float m_run = -INFINITY, l_run = 0.f;
  pf_float4_t acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = pf_float4_t{0.f, 0.f, 0.f, 0.f};

  Stage nxt = load_stage(0);   // n_st >= 1: the tile sees key 0
  store_stage(0, nxt);
  nxt = load_stage(min(1, n_st - 1));
  __syncthreads();
  for (int n = 0; n < n_st; ++n) {
    const int kb0 = n * PF_KEYS;
    if (wave_live && kb0 <= ctx + j_last_w) {   // the wave sees at least one key of this stage
      const unsigned char* st = lds + (n & 1) * L::STAGE;
      pf_float4_t sc[PF_NP];
#pragma unroll
      for (int pp = 0; pp < PF_NP; ++pp) {
        sc[pp] = pf_float4_t{0.f, 0.f, 0.f, 0.f};
        const unsigned char* krow = st + (PF_PAGE * pp + c16) * L::KP + 16 * r4;
#pragma unroll
        for (int s = 0; s < KS; ++s)
          sc[pp] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(pf_bf16x8_t, *reinterpret_cast<const uint4*>(krow + 64 * s)), qf[s], sc[pp], 0, 0, 0);
      }
      // page validity (uniform): inside the workgroup's reach, with a block id in range
      bool okp[PF_NP];
#pragma unroll
      for (int pp = 0; pp < PF_NP; ++pp) {
        const int p = n * PF_NP + pp;
        const int id = table[min(p, n_pages - 1)];
        okp[pp] = p < n_pages && id >= 0 && id < a.num_blocks;
      }
      float mx = -INFINITY;
      float sv[PF_NP][4];
#pragma unroll
      for (int pp = 0; pp < PF_NP; ++pp) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int key = kb0 + PF_PAGE * pp + 4 * r4 + e;
          const bool vis = okp[pp] && key <= ctx + jrow;
          sv[pp][e] = vis ? sc[pp][e] * a.scale_log2 : -INFINITY;
          mx = fmaxf(mx, sv[pp][e]);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;   // nothing visible yet: keep weights at 0
      const float alpha = exp2f(m_run - m_use);
      float psum = 0.f;
      pf_short4_t pb[PF_NP];
#pragma unroll
      for (int pp = 0; pp < PF_NP; ++pp)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float pv = exp2f(sv[pp][e] - m_use);
          psum += pv;
          pb[pp][e] = short(f32_to_bf16(pv));
        }
      l_run = l_run * alpha + psum;
      m_run = m_new;
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] *= alpha;
#pragma unroll
      for (int pp = 0; pp < PF_NP; ++pp) {
        // V rows of keys 4*r4 + e of this page; keys that do not exist are zeroed
        const unsigned char* vrow = st + L::K_BYTES + (PF_PAGE * pp + 4 * r4) * L::VP + NT * 2 * c16;
        uint32_t vw[4][VW];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (VW == 4) {
            const uint4 u = *reinterpret_cast<const uint4*>(vrow + e * L::VP);
            vw[e][0] = u.x;
            vw[e][1] = u.y;
            vw[e][2] = u.z;
            vw[e][3] = u.w;
          } else {
            const uint2 u = *reinterpret_cast<const uint2*>(vrow + e * L::VP);
            vw[e][0] = u.x;
            vw[e][1] = u.y;
          }
        }
        const int key0 = kb0 + PF_PAGE * pp + 4 * r4;
        const bool ok = okp[pp];
        const uint32_t m01 = (ok && key0 + 0 < kv_total ? 0x0000ffffu : 0u) | (ok && key0 + 1 < kv_total ? 0xffff0000u : 0u);
        const uint32_t m23 = (ok && key0 + 2 < kv_total ? 0x0000ffffu : 0u) | (ok && key0 + 3 < kv_total ? 0xffff0000u : 0u);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const int wd = t >> 1;
          uint32_t lo, hi;
          if ((t & 1) == 0) {
            lo = pf_pack_lo(vw[0][wd], vw[1][wd]);
            hi = pf_pack_lo(vw[2][wd], vw[3][wd]);
          } else {
            lo = pf_pack_hi(vw[0][wd], vw[1][wd]);
            hi = pf_pack_hi(vw[2][wd], vw[3][wd]);
          }
          const pf_short4_t va = __builtin_bit_cast(pf_short4_t, make_uint2(lo & m01, hi & m23));
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, pb[pp], acc[t], 0, 0, 0);
        }
      }
    }
    // stage n+1 (in registers since the previous iteration) into the other buffer; then the next loads.
    // Unconditional: past the end the last stage is re-staged (L2 hits, never read), so every path runs
    // the same load sequence and the staging registers stay in registers.
    store_stage((n + 1) & 1, nxt);
    nxt = load_stage(min(n + 2, n_st - 1));
    __syncthreads();
  }

  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  if (jq >= T) return;
  // lane holds, for tile t and r = 0..3, query c16 at dim NT*(4*r4 + r) + t
  const float inv = 1.0f / l_run;
  bf16_t* orow = a.out + int64_t(q_start + jq) * a.o_st + int64_t(h) * a.o_sh;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    uint32_t pk[VW];
#pragma unroll
    for (int t2 = 0; t2 < VW; ++t2)
      pk[t2] = uint32_t(f32_to_bf16(acc[2 * t2][r] * inv)) | (uint32_t(f32_to_bf16(acc[2 * t2 + 1][r] * inv)) << 16);
    bf16_t* o = orow + NT * (4 * r4 + r);
    if constexpr (VW == 4)
      *reinterpret_cast<uint4*>(o) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    else
      *reinterpret_cast<uint2*>(o) = make_uint2(pk[0], pk[1]);
  }
}

}  // namespace

}  // namespace ns

using namespace ns;

extern "C" int ns_paged_attn_prefill(const void* q, int64_t q_st, int64_t q_sh, const void* k_pool, const void* v_pool,
                                     int64_t kv_sblk, int64_t kv_spos, int64_t kv_sh, const int32_t* block_tables,
                                     int64_t bt_sb, const int32_t* seq_info, int n_seqs, int max_new, void* out,
                                     int64_t o_st, int64_t o_sh, int n_heads, int n_kv_heads, int head_dim,
                                     int block_size, int max_blocks, int num_blocks, float scale, int dtype,
                                     void* stream) {
  NS_REQUIRE(dtype == NS_DTYPE_BF16, "paged_attention_prefill: dtype %d not supported (bf16 only)", dtype);
  NS_REQUIRE(head_dim == 64 || head_dim == 128, "paged_attention_prefill: head_dim %d not in {64, 128}", head_dim);
  NS_REQUIRE(block_size == PF_PAGE, "paged_attention_prefill: block_size %d, the kernel needs %d", block_size, PF_PAGE);
  NS_REQUIRE(n_kv_heads > 0 && n_heads > 0 && n_heads % n_kv_heads == 0,
             "paged_attention_prefill: n_heads %d not a multiple of n_kv_heads %d", n_heads, n_kv_heads);
  NS_REQUIRE(n_seqs >= 0 && n_seqs <= 65535 && n_heads <= 65535, "paged_attention_prefill: %d sequences, %d heads",
             n_seqs, n_heads);
  NS_REQUIRE(max_new >= 0, "paged_attention_prefill: max_new %d", max_new);
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
  NS_REQUIRE(tiles <= 65535, "paged_attention_prefill: %d new tokens per sequence is too many", max_new);
  PrefillArgs a{static_cast<const bf16_t*>(q), q_st, q_sh, static_cast<const bf16_t*>(k_pool),
                static_cast<const bf16_t*>(v_pool), kv_sblk, kv_spos, kv_sh, block_tables, bt_sb, seq_info,
                static_cast<bf16_t*>(out), o_st, o_sh, n_heads / n_kv_heads, max_blocks, num_blocks, scale * PF_LOG2E};
  const dim3 grid{unsigned(n_heads), unsigned(tiles), unsigned(n_seqs)};
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (head_dim == 64)
    hipLaunchKernelGGL(paged_prefill_bf16_kernel<64>, grid, dim3(PF_WAVES * 64), 0, s, a);
  else
    hipLaunchKernelGGL(paged_prefill_bf16_kernel<128>, grid, dim3(PF_WAVES * 64), 0, s, a);
  return check_launch("paged_attention_prefill");
}
