// Paged-attention decode for gfx950 (MI355X).
//
// Semantics: nanoserve/kernels/paged_attention.py:34-105. For decode row b and KV head g, the G
// query heads h = g*G .. g*G+G-1 attend over the row's ctx_b cached tokens, which live in 16-token
// pages named by the row's block table. Online softmax keeps an fp32 running max m, sum l and
// accumulator; probabilities are rounded to the value dtype before P.V (paged_attention.py:77).
//
// bf16 design (the hot path):
//   * Split-K over the context: grid = (partitions, n_kv, B). A partition is NW waves x PPW pages;
//     page p0 + w + NW*i goes to wave w. Rows shorter than the grid's reach exit early, so the
//     grid depends on (B, table width) only and the launch can be captured in a hipGraph.
//   * Each wave first reads the block ids of its pages, then issues every K and V load of those
//     pages with no wait in between, then works page by page on the matrix cores. The GQA group
//     makes both products dense (rows >= G of Q are zero):
//       S^T[16 tok x 16 heads] = K_page[16 x hd] . Q^T[hd x 16]            (mfma 16x16x32 bf16)
//       O^T[hd x 16 heads]    += V_page^T[hd x 16 tok] . P^T[16 tok x 16]  (mfma 16x16x16 bf16)
//     The S^T output layout (lane = head, 4 consecutive tokens) is exactly the B-operand layout
//     P^T needs, so P never leaves registers. For V^T the contraction index (token) and the output
//     row (dim) may be relabelled freely: lane (c16, r4) takes dims NT*c16 .. NT*c16+NT-1 of tokens
//     4*r4 .. 4*r4+3, which are four coalesced row-slice loads, and a 4x4 register transpose
//     (v_perm) turns them into the NT operand fragments. No LDS on the per-page path.
//   * Softmax statistics per head: a lane's 4 tokens, then 2 butterfly shuffles (xor 16, xor 32).
//   * Waves merge through LDS; a row with one partition writes its output directly. Otherwise each
//     partition publishes (m, l, acc) to the workspace, bumps the row's arrival counter, and the last
//     partition to arrive merges all of them in partition order and writes the output -- one launch.
//     The hand-off uses agent-scope atomic stores/loads and a store-completion wait before the counter
//     (ns_common.h, publish_*), not device-scope fences, which on gfx950 write back and invalidate the
//     XCD's whole L2 in every workgroup.
// fp32 design: one wave per (row, KV head), VALU dot products with wave reductions; kept simple,
// it serves the fp32 correctness paths.
#include "ns_common.h"
#include "prefill_body.h"

#include <mutex>
#include <type_traits>

namespace ns {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) short short4_t;
typedef __attribute__((ext_vector_type(4))) float float4_t;

constexpr float LOG2E = 1.4426950408889634f;
constexpr int PAGE = 16;  // tokens per KV block

template <int HD>
struct DecodeCfg;
// NW waves per workgroup, PPW pages per wave: one partition covers NW * PPW pages.
template <>
struct DecodeCfg<64> {
  static constexpr int NW = 4, PPW = 4;
};
template <>
struct DecodeCfg<128> {
  static constexpr int NW = 4, PPW = 2;
};

// NT/2 dwords holding NT consecutive bf16 of one token row (the V slice a lane owns).
template <int NW32>
struct Words {
  uint32_t w[NW32];
};
template <int NW32>
__device__ __forceinline__ Words<NW32> load_words(const bf16_t* p) {
  Words<NW32> r;
  if constexpr (NW32 == 2) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    r.w[0] = u.x;
    r.w[1] = u.y;
  } else {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    r.w[0] = u.x;
    r.w[1] = u.y;
    r.w[2] = u.z;
    r.w[3] = u.w;
  }
  return r;
}

// (low halves of x, y) and (high halves of x, y) packed into one dword: v_perm_b32 byte selects.
__device__ __forceinline__ uint32_t pack_lo(uint32_t x, uint32_t y) { return __builtin_amdgcn_perm(y, x, 0x05040100u); }
__device__ __forceinline__ uint32_t pack_hi(uint32_t x, uint32_t y) { return __builtin_amdgcn_perm(y, x, 0x07060302u); }

// Partitions per row (table width / partition pages) the kernel accepts.
template <int HD>
constexpr int MERGE_MAX_PARTS = 256;

template <int HD>
__global__ __launch_bounds__(DecodeCfg<HD>::NW * 64) void paged_decode_bf16_kernel(
    const bf16_t* __restrict__ q, int64_t q_sb, int64_t q_sh, const bf16_t* __restrict__ kp,
    const bf16_t* __restrict__ vp, int64_t s_blk, int64_t s_pos, int64_t s_h, const int32_t* __restrict__ bt,
    int64_t bt_sb, const int32_t* __restrict__ ctxl, bf16_t* __restrict__ out, int64_t o_sb, int64_t o_sh, int G,
    int max_blocks, int num_blocks, float scale_log2, float* __restrict__ ws_acc, float* __restrict__ ws_ml,
    unsigned* __restrict__ ws_cnt, int B_, int nkv_, int n_parts, const int64_t* __restrict__ qrows, int cstride) {
  constexpr int NW = DecodeCfg<HD>::NW, PPW = DecodeCfg<HD>::PPW, PART = NW * PPW;
  constexpr int KS = HD / 32;  // 32-dim k-steps of the QK^T product (8 bf16 per lane per step)
  constexpr int NT = HD / 16;  // 16-row output tiles of the PV product
  constexpr int VW = NT / 2;   // dwords of a lane's V slice per token
  // XCD-aware work map. Workgroup L runs on XCD L % 8, and low partitions are live in every row
  // while high ones only in long rows. With rows = B * n_kv, L = part * rows + k and
  // row = (k + part) % rows: every partition index is spread over all XCDs, a row's partitions
  // rotate across XCDs, and live (low) partitions are dispatched first.
  const int rows = nkv_ * B_;
  const int L = blockIdx.x;
  const int part = L / rows;
  const int row = (L - part * rows + part) % rows;
  const int b = row / nkv_, g = row - (row / nkv_) * nkv_;
  const int64_t qb = qrows != nullptr ? qrows[b] : int64_t(b);   // q / out row of entry b
  const int nkv = nkv_;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c16 = lane & 15;   // MFMA column (head) for B / D; MFMA row for A operands
  const int r4 = lane >> 4;    // k-group: tokens 4*r4 .. 4*r4+3 (PV), dims 8*r4 .. 8*r4+7 (QK^T)
  const int p0 = part * PART;

  // ctx, the partition's block ids and Q are independent: issue them together (one latency).
  // Table entries p < max_blocks are inside the caller's table whatever ctx is.
  const int ctx = ctxl[b];
  int blk[PPW];
#pragma unroll
  for (int i = 0; i < PPW; ++i) {
    const int p = p0 + w + NW * i;
    blk[i] = p < max_blocks ? bt[int64_t(b) * bt_sb + p] : -1;
  }
  bf16x8_t qf[KS];  // B operand of S^T, k = dims 32s + 8*r4 + e; rows >= G zero
  {
    const bool hv = c16 < G;
    const bf16_t* qrow = q + qb * q_sb + int64_t(g * G + (hv ? c16 : 0)) * q_sh;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      uint4 u = *reinterpret_cast<const uint4*>(qrow + 32 * s + 8 * r4);
      if (!hv) u = make_uint4(0u, 0u, 0u, 0u);
      qf[s] = __builtin_bit_cast(bf16x8_t, u);
    }
  }
  int n_pages = ctx > 0 ? (ctx + PAGE - 1) / PAGE : 0;
  if (n_pages > max_blocks) n_pages = max_blocks;
  if (ctx <= 0) {  // no keys: zeros (the row is invalid; nothing to attend to)
    if (part == 0)
      for (int i = tid; i < G * HD; i += NW * 64)
        out[qb * o_sb + int64_t(g * G + i / HD) * o_sh + (i % HD)] = bf16_t(0);
    return;
  }
  if (p0 >= n_pages) return;  // whole workgroup: this partition is past the row's context
  const int n_active = (n_pages + PART - 1) / PART;
#pragma unroll
  for (int i = 0; i < PPW; ++i)
    if (p0 + w + NW * i >= n_pages) blk[i] = -1;   // dead page slot: masked below

  uint4 kf[PPW][KS];
  Words<VW> vr[PPW][4];
  bool okp[PPW];
#pragma unroll
  for (int i = 0; i < PPW; ++i) {
    okp[i] = blk[i] >= 0 && blk[i] < num_blocks;
    const int64_t base = int64_t(okp[i] ? blk[i] : 0) * s_blk + int64_t(g) * s_h;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      kf[i][s] = *reinterpret_cast<const uint4*>(kp + base + int64_t(c16) * s_pos + 32 * s + 8 * r4);
#pragma unroll
    for (int j = 0; j < 4; ++j) vr[i][j] = load_words<VW>(vp + base + int64_t(4 * r4 + j) * s_pos + NT * c16);
  }
  // Keep the scheduler from sinking these loads toward their uses (that would serialise the pages).
  __builtin_amdgcn_sched_barrier(0);

  float m_run = -INFINITY, l_run = 0.f;
  float4_t acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = float4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int i = 0; i < PPW; ++i) {
    const int p = p0 + w + NW * i;
    // S^T = K . Q^T : lane holds tokens 4*r4 + j (j = 0..3) of head c16
    float4_t st = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s)
      st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kf[i][s]), qf[s], st, 0, 0, 0);
    bool valid[4];
    float sv[4];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      valid[j] = okp[i] && (p * PAGE + 4 * r4 + j) < ctx;   // dead pages: p >= n_pages => token >= ctx
      sv[j] = valid[j] ? st[j] * scale_log2 : -INFINITY;
      mx = fmaxf(mx, sv[j]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    // -inf - -inf would be NaN: while nothing is unmasked, subtract 0 instead (all weights stay 0)
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2f(m_run - m_use);
    float pv[4], psum = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pv[j] = exp2f(sv[j] - m_use);
      psum += pv[j];
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
    // P^T as the B operand (k = token 4*r4 + j, n = head c16), rounded to bf16
    short4_t pb;
#pragma unroll
    for (int j = 0; j < 4; ++j) pb[j] = short(f32_to_bf16(pv[j]));
    // V^T fragments: tile t, row c16 = dim NT*c16 + t, k = token 4*r4 + j. Masked tokens read as 0
    // (unwritten slots past ctx may hold anything, and 0 * NaN is NaN).
    const uint32_t m01 = (valid[0] ? 0x0000ffffu : 0u) | (valid[1] ? 0xffff0000u : 0u);
    const uint32_t m23 = (valid[2] ? 0x0000ffffu : 0u) | (valid[3] ? 0xffff0000u : 0u);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int wd = t >> 1;
      uint32_t lo, hi;
      if ((t & 1) == 0) {
        lo = pack_lo(vr[i][0].w[wd], vr[i][1].w[wd]);
        hi = pack_lo(vr[i][2].w[wd], vr[i][3].w[wd]);
      } else {
        lo = pack_hi(vr[i][0].w[wd], vr[i][1].w[wd]);
        hi = pack_hi(vr[i][2].w[wd], vr[i][3].w[wd]);
      }
      const short4_t va = __builtin_bit_cast(short4_t, make_uint2(lo & m01, hi & m23));
      acc[t] *= alpha;
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, pb, acc[t], 0, 0, 0);
    }
  }
  // per-head sum over the 4 lane groups (same running max in all of them)
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);

  // ---- merge the NW waves through LDS: acc layout [wave][head][dim]; lane holds, for tile t and
  // r = 0..3, head c16 at dim NT*(4*r4 + r) + t.
  constexpr int AROW = HD + 4;
  __shared__ float sm_acc[NW][16 * AROW];
  __shared__ float sm_m[NW][16], sm_l[NW][16];
  if (r4 == 0) {
    sm_m[w][c16] = m_run;
    sm_l[w][c16] = l_run;
  }
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) sm_acc[w][c16 * AROW + NT * (4 * r4 + r) + t] = acc[t][r];
  __syncthreads();

  const int64_t bg = int64_t(b) * nkv + g;
  // this partition's softmax state, 4 consecutive dims of one head per item
  auto part_state = [&](int h, int d4, float& M, float& L, float (&A)[4]) __attribute__((always_inline)) {
    M = -INFINITY;
#pragma unroll
    for (int x = 0; x < NW; ++x) M = fmaxf(M, sm_m[x][h]);
    const float Mu = M == -INFINITY ? 0.f : M;
    L = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) A[e] = 0.f;
#pragma unroll
    for (int x = 0; x < NW; ++x) {
      const float wgt = exp2f(sm_m[x][h] - Mu);  // waves without live pages: m = -inf -> weight 0
      L += wgt * sm_l[x][h];
#pragma unroll
      for (int e = 0; e < 4; ++e) A[e] += wgt * sm_acc[x][h * AROW + 4 * d4 + e];
    }
  };
  if (n_active == 1) {   // the row fits one partition: finish it here
    for (int idx = tid; idx < G * (HD / 4); idx += NW * 64) {
      const int h = idx / (HD / 4), d4 = idx - h * (HD / 4);
      float M, L, A[4];
      part_state(h, d4, M, L, A);
      bf16_t* o = out + qb * o_sb + int64_t(g * G + h) * o_sh + 4 * d4;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = f32_to_bf16(A[e] / L);
    }
    return;
  }
  // Publish this partition's (m, l, acc); the last partition of the row to arrive merges all of them
  // in partition order (so the result does not depend on arrival order) and writes the output.
  for (int idx = tid; idx < G * (HD / 4); idx += NW * 64) {
    const int h = idx / (HD / 4), d4 = idx - h * (HD / 4);
    float M, L, A[4];
    part_state(h, d4, M, L, A);
    const pub_u32x4_t bits = {__float_as_uint(A[0]), __float_as_uint(A[1]), __float_as_uint(A[2]), __float_as_uint(A[3])};
    publish_store16(ws_acc + ((bg * n_parts + part) * 16 + h) * HD + 4 * d4, bits);
    if (d4 == 0) {
      publish_store(ws_ml + ((bg * n_parts + part) * 16 + h) * 2 + 0, M);
      publish_store(ws_ml + ((bg * n_parts + part) * 16 + h) * 2 + 1, L);
    }
  }
  publish_complete();
  __shared__ unsigned s_last;
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = publish_count(ws_cnt + bg * cstride);
    const unsigned last = prev == unsigned(n_active - 1);
    if (last) publish_reset(ws_cnt + bg * cstride);
    s_last = last;
  }
  __syncthreads();
  if (s_last == 0u) return;
  acquire_published();
  // Merge in partition order with a running max: every thread loads, for its head and 4 dims, the (m, l,
  // acc) of MB partitions at once (one memory latency per MB partitions) and folds them in.
  const float* ml = ws_ml + bg * n_parts * 32;
  const float* accp = ws_acc + bg * n_parts * (16 * HD);
  constexpr int MB = 8;
  for (int idx = tid; idx < G * (HD / 4); idx += NW * 64) {
    const int h = idx / (HD / 4), d4 = idx - h * (HD / 4);
    float M = -INFINITY, L = 0.f, A[4] = {0.f, 0.f, 0.f, 0.f};
    for (int x0 = 0; x0 < n_active; x0 += MB) {
      pub_u32x4_t u[MB];
      float pm[MB], pl[MB];
#pragma unroll
      for (int e = 0; e < MB; ++e) {
        const int x = min(x0 + e, n_active - 1);
        u[e] = publish_load16(accp + int64_t(x) * (16 * HD) + h * HD + 4 * d4);
        pm[e] = publish_load(ml + x * 32 + h * 2);
        pl[e] = publish_load(ml + x * 32 + h * 2 + 1);
      }
#pragma unroll
      for (int e = 0; e < MB; ++e) {
        if (x0 + e < n_active) {
          const float Mn = fmaxf(M, pm[e]);
          const float a_old = M == -INFINITY ? 0.f : exp2f(M - Mn), a_new = exp2f(pm[e] - Mn);
          L = L * a_old + pl[e] * a_new;
#pragma unroll
          for (int c = 0; c < 4; ++c) A[c] = A[c] * a_old + __uint_as_float(u[e][c]) * a_new;
          M = Mn;
        }
      }
    }
    const float inv = 1.0f / L;
    bf16_t* o = out + qb * o_sb + int64_t(g * G + h) * o_sh + 4 * d4;
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = f32_to_bf16(A[c] * inv);
  }
}

// ---------------------------------------------------------------------------------------------------
// Whole-row variant for token rows of 256 bytes (n_kv * head_dim = 128: hd 64 with 2 KV heads, or hd 128
// with 1) and at most 16 query heads. One workgroup covers every KV head of one row's partition, so a
// block's K (and V) is read as one contiguous 4 KB stretch, and the loads are row-contiguous (each
// instruction reads 4 whole token rows) instead of 16 tokens x 64 bytes:
//   * lane (c16, r4) loads, for token quad j, token 4j + r4's 16-byte chunk c16. K goes through a
//     wave-private LDS page (chunks XOR-swizzled by the token) into MFMA A fragments; V stays in
//     registers and is transposed as in the per-head kernel.
//   * S^T rows are relabelled (row r = token 4(r & 3) + (r >> 2)) so S^T's output layout is again P^T's
//     B layout and matches the V^T fragments' token order.
//   * all KV heads accumulate into one 16-column S^T tile: head h's products see only its own query
//     columns (the others multiply zeros), and O^T rows hold both heads' dims; each lane keeps the rows
//     of its own query's head.
//   * a wave walks PPW pages with D pages of loads in flight (register slot i % D holds page i), so the
//     softmax and MFMA work of early pages overlaps the stream of later ones.
//   * partitions of PART = 32 pages (the last one of a row shorter), so a row's split depends on its own
//     context length only, never on the table width; a row with several merges as the per-head kernel does: 16-byte
//     coherent (sc1) stores of (m, l, acc), a wait for them, the row's counter, and the last partition
//     to arrive loads MB partitions per round trip and folds them in partition order.
constexpr int ROWK_NW = 8, ROWK_PPW = 4, ROWK_D = 2, ROWK_PART = ROWK_NW * ROWK_PPW;
constexpr int ROWK_MB = 8;
constexpr int ROWK_VALU_G = 8, ROWK_VALU_G_PH = 6;   // query heads per KV head the VALU variant takes
constexpr int ROWK_MAX_PARTS = 32;
typedef __attribute__((ext_vector_type(4))) unsigned int rk_u32x4_t;
typedef __attribute__((ext_vector_type(2))) unsigned int rk_u32x2_t;

// Arguments of the whole-row kernel (one struct, so the body can also run inside the mixed launch).
struct RowsArgs {
  const bf16_t* q;
  int64_t q_sb, q_sh;
  const bf16_t* kp;
  const bf16_t* vp;
  int64_t s_blk;
  const int32_t* bt;
  int64_t bt_sb;
  const int32_t* ctxl;
  bf16_t* out;
  int64_t o_sb, o_sh;
  int G, nq, max_blocks, num_blocks;
  float scale_log2;
  unsigned* cnt;
  float* part_acc;
  float* part_ml;
  int B, n_parts, nkv_grid;
  int64_t s_tok, s_h;
  const int64_t* qrows;
  int cstride;
  // optional, one per entry: 1 = entries b and b + 1 read the same block table (speculative verify rows of
  // one sequence) and run as one workgroup row, their query heads side by side in the 16 MFMA columns;
  // -1 = entry b was taken with b - 1; 0 = alone. Only when twice the workgroup's query heads fit in 16.
  const int32_t* pair;
};
template <int HD>
constexpr int rows_lds_bytes() {
  return ROWK_NW * 16 * 256 > ROWK_NW * 16 * (HD + 4) * 4 ? ROWK_NW * 16 * 256 : ROWK_NW * 16 * (HD + 4) * 4;
}

// PH: each KV head is a workgroup row of its own (hd 128, several KV heads); otherwise a row is a token's
// whole 256-byte K row. PAIR: entries that share a block table may run as one workgroup row (ra.pair); a
// compile-time switch, so launches without pairs carry none of the per-column context logic (+0.57 us per
// config-2 call when it was a runtime test). bid: the workgroup's index among the launch's decode-row
// workgroups; lds (at least rows_lds_bytes<HD>()), sm_m, sm_l, s_last: the launch's LDS.
template <int HD, bool PH, bool VALU = false, bool PAIR = false>
__device__ __forceinline__ void decode_rows_body(const RowsArgs& ra, int bid, unsigned char* lds,
                                                 float (*sm_m)[16], float (*sm_l)[16], unsigned& s_last) {
  const bf16_t* __restrict__ q = ra.q;
  const int64_t q_sb = ra.q_sb, q_sh = ra.q_sh;
  const bf16_t* __restrict__ kp = ra.kp;
  const bf16_t* __restrict__ vp = ra.vp;
  const int64_t s_blk = ra.s_blk;
  const int32_t* __restrict__ bt = ra.bt;
  const int64_t bt_sb = ra.bt_sb;
  const int32_t* __restrict__ ctxl = ra.ctxl;
  bf16_t* __restrict__ out = ra.out;
  const int64_t o_sb = ra.o_sb, o_sh = ra.o_sh;
  const int G = ra.G, nq = ra.nq, max_blocks = ra.max_blocks, num_blocks = ra.num_blocks;
  const float scale_log2 = ra.scale_log2;
  unsigned* __restrict__ cnt = ra.cnt;
  float* __restrict__ part_acc = ra.part_acc;
  float* __restrict__ part_ml = ra.part_ml;
  const int B = ra.B, n_parts = ra.n_parts, nkv_grid_arg = ra.nkv_grid;
  const int64_t s_tok_arg = ra.s_tok, s_h = ra.s_h;
  const int64_t* __restrict__ qrows = ra.qrows;
  const int cstride = ra.cstride;
  constexpr int pp = ROWK_PART;
  constexpr int NW = ROWK_NW, PPW = ROWK_PPW, D = ROWK_D;
  // A workgroup's token row: 128 elements (256 bytes) -- all KV heads of a token (nkv_grid == 1), or one
  // KV head of hd 128 when each KV head is a row of its own (nkv_grid == n_kv, token stride s_tok).
  constexpr int NKV = 128 / HD;
  constexpr int KS = HD / 32;
  constexpr int AROW = HD + 4;

  // XCD-aware map as in the per-head kernel: a row's partitions rotate over the XCDs
  const int nkv_grid = PH ? nkv_grid_arg : 1;
  const int64_t s_tok = PH ? s_tok_arg : 128;
  const int R = B * nkv_grid;
  const int L = bid, part = L / R;
  const int row = (L - part * R + part) % R;
  const int b = row / nkv_grid, g = row - b * nkv_grid;
  static_assert(!(PAIR && VALU), "pairs run on the matrix-core products only");
  // the pair entry, both entries' context lengths and q rows load together (entry b + 1's clamped in
  // bounds and used only for a pair), so pairing adds no dependent round trip before the page stream
  const int bn = b + 1 < B ? b + 1 : b;
  const int prw = PAIR ? ra.pair[b] : 0;
  const int ctx0 = ctxl[b];
  const int ctx1_any = PAIR ? ctxl[bn] : ctx0;
  const int64_t qb = qrows != nullptr ? qrows[b] : int64_t(b);   // q / out row of entry b
  const int64_t qb1_any = PAIR ? (qrows != nullptr ? qrows[bn] : int64_t(bn)) : qb;
  if constexpr (PAIR) asm volatile("" : : "s"(prw), "s"(ctx0), "s"(ctx1_any), "s"(qb), "s"(qb1_any));   // one wait
  if (prw < 0) return;   // entry b runs in the workgroups of entry b - 1
  const int np_ = PAIR && prw > 0 ? 2 : 1;   // entries in this workgroup row
  const int64_t qb1 = np_ > 1 ? qb1_any : qb;
  const int nq_w = nkv_grid > 1 ? G : nq;   // query heads of this workgroup: heads g G .. g G + nq_w - 1
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c16 = lane & 15, r4 = lane >> 4;
  const int p0 = part * pp;
  // MFMA column c16 = (entry c16 / nq_w, query head c16 % nq_w) of the workgroup row
  const int cj = PAIR && c16 >= nq_w ? 1 : 0, ch = c16 - cj * nq_w;

  // ctx, this wave's block ids (lane i < PPW holds page i's) and Q go out together; a pair walks the longer
  // context's pages and masks each column's scores at its own entry's context
  const int ctx1 = PAIR && np_ > 1 ? ctx1_any : ctx0;
  const int ctx = PAIR ? max(ctx0, ctx1) : ctx0;
  const int ctx_col = PAIR && cj ? ctx1 : ctx0;
  int blk_lane;
  {
    const int p = p0 + w + NW * (lane < PPW ? lane : 0);
    blk_lane = p < max_blocks ? bt[int64_t(b) * bt_sb + p] : -1;
  }
  const bool qlive = c16 < np_ * nq_w;
  const int gq = qlive ? ch / G : NKV;   // KV head (within the token row) of this lane's query column
  bf16x8_t qf[KS];
  {
    const bf16_t* qrow = q + (cj ? qb1 : qb) * q_sb + int64_t(g * G + (qlive ? ch : 0)) * q_sh;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      rk_u32x4_t u = *reinterpret_cast<const rk_u32x4_t*>(qrow + 32 * s + 8 * r4);
      if (!qlive) u = rk_u32x4_t{0u, 0u, 0u, 0u};
      qf[s] = __builtin_bit_cast(bf16x8_t, u);
    }
  }
  // VALU variant: lane (c16, r4) holds dims 8 c16 .. 8 c16 + 7 of the token row, i.e. of KV head gk, and takes
  // those dims of each query head of gk from the wave's LDS page (staged once; registers go to the
  // accumulators); whole scores come from a sum over the head's HD / 8 lanes
  constexpr int GV = VALU ? (PH ? ROWK_VALU_G_PH : ROWK_VALU_G) : 1;
  const int gk = (8 * c16) / HD;
  if constexpr (VALU) {
    unsigned char* qlds = lds + w * (16 * 256);
    if (r4 < 2) {
#pragma unroll
      for (int j = 0; j < GV / 2; ++j) {
        const int i = 2 * j + r4, hi = gk * G + i;
        const bool live = i < G && hi < nq_w;
        const rk_u32x4_t u = *reinterpret_cast<const rk_u32x4_t*>(q + qb * q_sb + int64_t(g * G + (live ? hi : 0)) * q_sh +
                                                                 ((8 * c16) & (HD - 1)));
        *reinterpret_cast<rk_u32x4_t*>(qlds + (c16 * GV + i) * 16) = live ? u : rk_u32x4_t{0u, 0u, 0u, 0u};
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the wave's q rows are in LDS before any lane reads them
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  }
  int n_pages = ctx > 0 ? (ctx + PAGE - 1) / PAGE : 0;
  if (n_pages > max_blocks) n_pages = max_blocks;
  if (ctx <= 0) {   // no keys: zeros
    if (part == 0)
      for (int i = tid; i < np_ * nq_w * HD; i += NW * 64) {
        const int c = i / HD, j = c >= nq_w ? 1 : 0;
        out[(j ? qb1 : qb) * o_sb + int64_t(g * G + c - j * nq_w) * o_sh + (i % HD)] = bf16_t(0);
      }
    return;
  }
  if (p0 >= n_pages) return;
  const int n_active = (n_pages + pp - 1) / pp;
  const int p_end = min(n_pages, p0 + pp);

  // This wave's pages are p0 + w + NW i, i < PPW. Page i's K and V sit in register slot i % D; a slot is
  // refilled with page i + D once page i is consumed. Pages past the row's end re-load the wave's first
  // page (so every path issues the same loads) and skip the arithmetic.
  int n_live = 0;
#pragma unroll
  for (int i = 0; i < PPW; ++i) n_live += (p0 + w + NW * i < p_end) ? 1 : 0;
  rk_u32x4_t kr[D][4], vr[D][4];
  auto issue = [&](int i, auto sc) __attribute__((always_inline)) {
    constexpr int sl = decltype(sc)::value;
    const int bid = __builtin_amdgcn_readlane(blk_lane, i < n_live ? i : 0);
    const bool ok = n_live > 0 && bid >= 0 && bid < num_blocks;
    const int64_t base = int64_t(ok ? bid : 0) * s_blk + (PH ? int64_t(g) * s_h : 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t off = base + int64_t(4 * j + r4) * s_tok + c16 * 8;
      if constexpr (PH) {   // a KV head's half of a token row: the other head's workgroup reads the rest
        kr[sl][j] = *reinterpret_cast<const rk_u32x4_t*>(kp + off);
        vr[sl][j] = *reinterpret_cast<const rk_u32x4_t*>(vp + off);
      } else {                // whole token rows, read once: streamed past the caches
        kr[sl][j] = __builtin_nontemporal_load(reinterpret_cast<const rk_u32x4_t*>(kp + off));
        vr[sl][j] = __builtin_nontemporal_load(reinterpret_cast<const rk_u32x4_t*>(vp + off));
      }
    }
  };
  unsigned char* kpg = lds + w * (16 * 256);
  float m_run = -INFINITY, l_run = 0.f;
  float4_t acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = float4_t{0.f, 0.f, 0.f, 0.f};
  float vm[GV], vl[GV], vacc[GV][8];   // VALU variant: per query head of gk, this lane's 8 dims
#pragma unroll
  for (int i = 0; i < GV; ++i) {
    vm[i] = -INFINITY;
    vl[i] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) vacc[i][e] = 0.f;
  }
  const int tr = 4 * (c16 & 3) + (c16 >> 2);   // token of S^T row c16
  auto page = [&](int i, auto sc) __attribute__((always_inline)) {
    constexpr int sl = decltype(sc)::value;
    const int p = p0 + w + NW * i;
    const int bid = __builtin_amdgcn_readlane(blk_lane, i);
    const bool okp = bid >= 0 && bid < num_blocks;
    if constexpr (VALU) {
      // lane (c16, r4) has tokens 4 k + r4 (k < 4), dims 8 c16 .. 8 c16 + 7 of K and V
      bool valid[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) valid[k] = okp && (p * PAGE + 4 * k + r4) < ctx;
#pragma unroll
      for (int h = 0; h < GV; ++h) {   // one query head at a time (its scores, softmax update and P.V)
        const rk_u32x4_t qh = *reinterpret_cast<const rk_u32x4_t*>(kpg + (c16 * GV + h) * 16);
        float s4[4], mx = -INFINITY;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          float a = 0.f;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t kw = kr[sl][k][e], qw = qh[e];
            a = fmaf(__uint_as_float(kw << 16), __uint_as_float(qw << 16), a);
            a = fmaf(__uint_as_float(kw & 0xffff0000u), __uint_as_float(qw & 0xffff0000u), a);
          }
#pragma unroll
          for (int o = 1; o < HD / 8; o <<= 1) a += __shfl_xor(a, o, 64);   // the head's HD / 8 chunks
          s4[k] = valid[k] ? a * scale_log2 : -INFINITY;
          mx = fmaxf(mx, s4[k]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(vm[h], mx);
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = exp2f(vm[h] - m_use);
        float pb[4], psum = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float pv = exp2f(s4[k] - m_use);
          psum += pv;
          pb[k] = valid[k] ? __uint_as_float(uint32_t(f32_to_bf16(pv)) << 16) : 0.f;   // P rounded to bf16
        }
        vl[h] = vl[h] * alpha + psum;
        vm[h] = m_new;
#pragma unroll
        for (int e = 0; e < 8; ++e) vacc[h][e] *= alpha;
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t vw = vr[sl][k][e];
            const float v0 = valid[k] ? __uint_as_float(vw << 16) : 0.f;
            const float v1 = valid[k] ? __uint_as_float(vw & 0xffff0000u) : 0.f;
            vacc[h][2 * e] = fmaf(pb[k], v0, vacc[h][2 * e]);
            vacc[h][2 * e + 1] = fmaf(pb[k], v1, vacc[h][2 * e + 1]);
          }
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 4 * j + r4;
      *reinterpret_cast<rk_u32x4_t*>(kpg + t * 256 + ((c16 ^ t) << 4)) = kr[sl][j];
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);        // lgkmcnt(0): the page's K rows are in LDS
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    float4_t st = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int h = 0; h < NKV; ++h)
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const int c = (h * HD + 32 * s + 8 * r4) >> 3;   // 16-byte chunk of the token row
        const rk_u32x4_t a = *reinterpret_cast<const rk_u32x4_t*>(kpg + tr * 256 + ((c ^ tr) << 4));
        const bf16x8_t bq = gq == h ? qf[s] : __builtin_bit_cast(bf16x8_t, rk_u32x4_t{0u, 0u, 0u, 0u});
        st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), bq, st, 0, 0, 0);
      }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);   // the next page's K writes stay behind these reads
    // lane (c16, r4) holds rows 4 r4 + k = tokens 4k + r4 of the page
    bool valid[4], vtok[4];   // vtok: a written key (its V row kept); valid: visible to this lane's column
    float sv[4];
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      vtok[k] = okp && (p * PAGE + 4 * k + r4) < ctx;
      valid[k] = PAIR ? vtok[k] && (p * PAGE + 4 * k + r4) < ctx_col : vtok[k];
      sv[k] = valid[k] ? st[k] * scale_log2 : -INFINITY;
      mx = fmaxf(mx, sv[k]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2f(m_run - m_use);
    float pv[4], psum = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      pv[k] = exp2f(sv[k] - m_use);
      psum += pv[k];
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
    short4_t pb;
#pragma unroll
    for (int k = 0; k < 4; ++k) pb[k] = short(f32_to_bf16(pv[k]));
    // V^T tile t: row c16 = 16-byte chunk c16 (dim 8 c16 + t of the row), k = token 4j + r4
    const uint32_t m01 = (vtok[0] ? 0x0000ffffu : 0u) | (vtok[1] ? 0xffff0000u : 0u);
    const uint32_t m23 = (vtok[2] ? 0x0000ffffu : 0u) | (vtok[3] ? 0xffff0000u : 0u);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int wd = t >> 1;
      uint32_t lo, hi;
      if ((t & 1) == 0) {
        lo = pack_lo(vr[sl][0][wd], vr[sl][1][wd]);
        hi = pack_lo(vr[sl][2][wd], vr[sl][3][wd]);
      } else {
        lo = pack_hi(vr[sl][0][wd], vr[sl][1][wd]);
        hi = pack_hi(vr[sl][2][wd], vr[sl][3][wd]);
      }
      const short4_t va = __builtin_bit_cast(short4_t, make_uint2(lo & m01, hi & m23));
      acc[t] *= alpha;
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, pb, acc[t], 0, 0, 0);
    }
  };
  using Z0 = std::integral_constant<int, 0>;
  using Z1 = std::integral_constant<int, 1>;
  using Z2 = std::integral_constant<int, 2>;
  using Z3 = std::integral_constant<int, 3>;
  if constexpr (D == 4) {   // every page of the wave in flight at once
    static_assert(PPW == 4, "four slots hold the wave's four pages");
    issue(0, Z0{});
    issue(1, Z1{});
    issue(2, Z2{});
    issue(3, Z3{});
    if (0 < n_live) page(0, Z0{});   // wave-uniform
    if (1 < n_live) page(1, Z1{});
    if (2 < n_live) page(2, Z2{});
    if (3 < n_live) page(3, Z3{});
  } else {
    static_assert(D == 2 && PPW % 2 == 0, "the page loop is unrolled for two slots");
    issue(0, Z0{});
    issue(1, Z1{});
#pragma unroll
    for (int i0 = 0; i0 < PPW; i0 += 2) {
      if (i0 < n_live) page(i0, Z0{});       // wave-uniform
      if (i0 + 2 < PPW) issue(i0 + 2, Z0{});
      if (i0 + 1 < n_live) page(i0 + 1, Z1{});
      if (i0 + 3 < PPW) issue(i0 + 3, Z1{});
    }
  }
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  if constexpr (VALU) {   // sums over the four token groups r4
#pragma unroll
    for (int h = 0; h < GV; ++h) {
      vl[h] += __shfl_xor(vl[h], 16, 64);
      vl[h] += __shfl_xor(vl[h], 32, 64);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        vacc[h][e] += __shfl_xor(vacc[h][e], 16, 64);
        vacc[h][e] += __shfl_xor(vacc[h][e], 32, 64);
      }
    }
  }

  // ---- merge the waves through LDS: [wave][query][dim]; a lane keeps the O^T rows of its query's head
  __syncthreads();   // every wave is done with its K page: the buffer is reused
  float* sm_acc = reinterpret_cast<float*>(lds);
  if constexpr (VALU) {
    if (r4 == 0) {
#pragma unroll
      for (int h = 0; h < GV; ++h) {
        const int hi = gk * G + h;
        if (h < G && hi < nq_w) {
          if ((c16 & (HD / 8 - 1)) == 0) {
            sm_m[w][hi] = vm[h];
            sm_l[w][hi] = vl[h];
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) sm_acc[(w * 16 + hi) * AROW + ((8 * c16) & (HD - 1)) + e] = vacc[h][e];
        }
      }
    }
  } else if (r4 == 0) {
    sm_m[w][c16] = m_run;
    sm_l[w][c16] = l_run;
  }
  if constexpr (!VALU) {
    const int head = NKV == 2 ? (r4 >> 1) : 0;   // rows 4 r4 + k are chunks of head (4 r4 + k) / (HD / 8)
    if (head == gq) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int t = 0; t < 8; ++t) sm_acc[(w * 16 + c16) * AROW + ((8 * (4 * r4 + k) + t) & (HD - 1))] = acc[t][k];
    }
  }
  __syncthreads();
  auto part_state = [&](int h, int d4, float& M, float& Ls, float (&A)[4]) __attribute__((always_inline)) {
    M = -INFINITY;
#pragma unroll
    for (int x = 0; x < NW; ++x) M = fmaxf(M, sm_m[x][h]);
    const float Mu = M == -INFINITY ? 0.f : M;
    Ls = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) A[e] = 0.f;
#pragma unroll
    for (int x = 0; x < NW; ++x) {
      const float wgt = exp2f(sm_m[x][h] - Mu);   // waves without live pages: m = -inf -> weight 0
      Ls += wgt * sm_l[x][h];
      const float4_t v = *reinterpret_cast<const float4_t*>(sm_acc + (x * 16 + h) * AROW + 4 * d4);
#pragma unroll
      for (int e = 0; e < 4; ++e) A[e] += wgt * v[e];
    }
  };
  auto store_out = [&](int h, int d4, float Ls, const float (&A)[4]) __attribute__((always_inline)) {
    const float inv = Ls > 0.f ? 1.0f / Ls : 0.f;
    const uint2 pk = make_uint2(uint32_t(f32_to_bf16(A[0] * inv)) | (uint32_t(f32_to_bf16(A[1] * inv)) << 16),
                                uint32_t(f32_to_bf16(A[2] * inv)) | (uint32_t(f32_to_bf16(A[3] * inv)) << 16));
    const int j = PAIR && h >= nq_w ? 1 : 0;   // column h = (entry j, query head h - j nq_w)
    *reinterpret_cast<uint2*>(out + (j ? qb1 : qb) * o_sb + int64_t(g * G + h - j * nq_w) * o_sh + 4 * d4) = pk;
  };
  constexpr int ITEMS = (16 * (HD / 4) + NW * 64 - 1) / (NW * 64);
  const int n_items = np_ * nq_w * (HD / 4);
  if (n_active == 1) {
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      const int idx = tid + it * NW * 64;
      if (idx < n_items) {
        const int h = idx / (HD / 4), d4 = idx % (HD / 4);
        float M, Ls, A[4];
        part_state(h, d4, M, Ls, A);
        store_out(h, d4, Ls, A);
      }
    }
    return;
  }
  // publish (m, l, acc) with 16-byte coherent stores, wait for them, then the row's counter
  const __amdgpu_buffer_rsrc_t racc =
      __builtin_amdgcn_make_buffer_rsrc(part_acc + int64_t(row) * n_parts * (16 * HD), 0, n_parts * (16 * HD) * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t rml =
      __builtin_amdgcn_make_buffer_rsrc(part_ml + int64_t(row) * n_parts * 32, 0, n_parts * 32 * 4, 0x00020000);
  constexpr int SC1 = 16;   // cache policy sc1: device-coherent, bypasses the XCD's L2
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int idx = tid + it * NW * 64;
    if (idx < n_items) {
      const int h = idx / (HD / 4), d4 = idx % (HD / 4);
      float M, Ls, A[4];
      part_state(h, d4, M, Ls, A);
      __builtin_amdgcn_raw_buffer_store_b128(
          rk_u32x4_t{__float_as_uint(A[0]), __float_as_uint(A[1]), __float_as_uint(A[2]), __float_as_uint(A[3])}, racc,
          ((part * 16 + h) * HD + 4 * d4) * 4, 0, SC1);
      if (d4 == 0)
        __builtin_amdgcn_raw_buffer_store_b64(rk_u32x2_t{__float_as_uint(M), __float_as_uint(Ls)}, rml,
                                              (part * 32 + 2 * h) * 4, 0, SC1);
    }
  }
  publish_complete();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = publish_count(cnt + row * cstride);
    const unsigned lst = prev == unsigned(n_active - 1);
    if (lst) publish_reset(cnt + row * cstride);
    s_last = lst;
  }
  __syncthreads();
  if (s_last == 0u) return;
  acquire_published();
  // the last partition: MB partitions per round trip, folded in partition order with a running max
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int idx = tid + it * NW * 64;
    if (idx < n_items) {
      const int h = idx / (HD / 4), d4 = idx % (HD / 4);
      float M = -INFINITY, Ls = 0.f, A[4] = {0.f, 0.f, 0.f, 0.f};
      for (int x0 = 0; x0 < n_active; x0 += ROWK_MB) {
        rk_u32x4_t ua[ROWK_MB];
        rk_u32x2_t um[ROWK_MB];
#pragma unroll
        for (int e = 0; e < ROWK_MB; ++e) {
          const int x = min(x0 + e, n_active - 1);
          ua[e] = __builtin_amdgcn_raw_buffer_load_b128(racc, ((x * 16 + h) * HD + 4 * d4) * 4, 0, SC1);
          um[e] = __builtin_amdgcn_raw_buffer_load_b64(rml, (x * 32 + 2 * h) * 4, 0, SC1);
        }
#pragma unroll
        for (int e = 0; e < ROWK_MB; ++e) {
          if (x0 + e < n_active) {
            const float pm = __uint_as_float(um[e][0]), pl = __uint_as_float(um[e][1]);
            const float Mn = fmaxf(M, pm);
            const float a_old = M == -INFINITY ? 0.f : exp2f(M - Mn);
            const float a_new = pm == -INFINITY ? 0.f : exp2f(pm - Mn);
            Ls = Ls * a_old + pl * a_new;
#pragma unroll
            for (int c = 0; c < 4; ++c) A[c] = A[c] * a_old + __uint_as_float(ua[e][c]) * a_new;
            M = Mn;
          }
        }
      }
      store_out(h, d4, Ls, A);
    }
  }
}

template <int HD, bool PH, bool VALU, bool PAIR>
__global__ __launch_bounds__(ROWK_NW * 64) void paged_decode_rows_bf16_kernel(RowsArgs a) {
  __shared__ __align__(16) unsigned char lds[rows_lds_bytes<HD>()];
  __shared__ float sm_m[ROWK_NW][16], sm_l[ROWK_NW][16];
  __shared__ unsigned s_last;
  decode_rows_body<HD, PH, VALU, PAIR>(a, int(blockIdx.x), lds, sm_m, sm_l, s_last);
}

// A mixed step's attention in one launch: workgroups [0, n_pf) are the chunked-prefill kernel's
// (prefill_body.h), the rest the whole-row decode kernel's for the step's decode rows. The two write disjoint
// rows of the output and keep their merges in separate workspaces; neither waits on a workgroup of the
// other kind. Issued as two kernels on one stream the second would wait for the first's last workgroup.
// Workgroups start in index order and every one reserves the launch's LDS (the prefill's 128 KB, one per
// CU), so the prefill units, planned to fill the CUs in one round, go first; the decode workgroups start on
// the CUs left over and on those the prefill's shorter units free. (With the decode workgroups first, the
// prefill units that found no free CU started ~10 us late and the launch took 37 us against 28 us for the
// prefill alone. Two streams overlap them too, but a graph's cross-queue fork and join idle the GPU for
// longer than that saves.)
template <int HD, bool PH>
__global__ __launch_bounds__(PF_WG_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void mixed_attn_kernel(
    PrefillArgs pa, int n_pf, RowsArgs ra) {
  static_assert(PF_WG_THREADS == ROWK_NW * 64, "one workgroup size for both kinds");
  constexpr int PF_BYTES = PF_GROUPS * 2 * PfLds<HD>::STAGE;
  constexpr int BYTES = PF_BYTES > rows_lds_bytes<HD>() ? PF_BYTES : rows_lds_bytes<HD>();
  __shared__ __align__(16) unsigned char lds[BYTES];
  __shared__ float sm_m[ROWK_NW][16], sm_l[ROWK_NW][16];
  __shared__ unsigned s_last;
  if (int(blockIdx.x) < n_pf)
    prefill_body<HD>(pa, int(blockIdx.x), lds, s_last);
  else
    decode_rows_body<HD, PH>(ra, int(blockIdx.x) - n_pf, lds, sm_m, sm_l, s_last);
}

// fp32: one wave per (row, KV head). Lane owns dims lane and lane + 64 (hd 128).
template <int HD>
__global__ __launch_bounds__(64) void paged_decode_f32_kernel(
    const float* __restrict__ q, int64_t q_sb, int64_t q_sh, const float* __restrict__ kp,
    const float* __restrict__ vp, int64_t s_blk, int64_t s_pos, int64_t s_h, const int32_t* __restrict__ bt,
    int64_t bt_sb, const int32_t* __restrict__ ctxl, float* __restrict__ out, int64_t o_sb, int64_t o_sh, int G,
    int max_blocks, int num_blocks, float scale, const int64_t* __restrict__ qrows) {
  constexpr int DL = HD / 64;  // dims per lane
  const int g = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  const int64_t qb = qrows != nullptr ? qrows[b] : int64_t(b);   // q / out row of entry b
  const int ctx = ctxl[b];
  int n_pages = ctx > 0 ? (ctx + PAGE - 1) / PAGE : 0;
  if (n_pages > max_blocks) n_pages = max_blocks;
  const int n_tok = ctx < n_pages * PAGE ? ctx : n_pages * PAGE;
  float qv[16][DL], acc[16][DL], m[16], l[16];
#pragma unroll
  for (int h = 0; h < 16; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < DL; ++e) {
      qv[h][e] = h < G ? q[qb * q_sb + int64_t(g * G + h) * q_sh + lane + 64 * e] : 0.f;
      acc[h][e] = 0.f;
    }
  }
  for (int t = 0; t < n_tok; ++t) {
    const int blk = bt[int64_t(b) * bt_sb + t / PAGE];
    const bool ok = blk >= 0 && blk < num_blocks;
    const int64_t off = int64_t(ok ? blk : 0) * s_blk + int64_t(t % PAGE) * s_pos + int64_t(g) * s_h;
    float kv[DL], vv[DL];
#pragma unroll
    for (int e = 0; e < DL; ++e) {
      kv[e] = ok ? kp[off + lane + 64 * e] : 0.f;
      vv[e] = ok ? vp[off + lane + 64 * e] : 0.f;
    }
#pragma unroll
    for (int h = 0; h < 16; ++h) {
      if (h < G) {
        float part = 0.f;
#pragma unroll
        for (int e = 0; e < DL; ++e) part = fmaf(qv[h][e], kv[e], part);
        const float s = wave_sum(part) * scale;
        const float m_new = fmaxf(m[h], s);
        const float alpha = expf(m[h] - m_new);
        const float p = expf(s - m_new);
        l[h] = l[h] * alpha + p;
#pragma unroll
        for (int e = 0; e < DL; ++e) acc[h][e] = acc[h][e] * alpha + p * vv[e];
        m[h] = m_new;
      }
    }
  }
#pragma unroll
  for (int h = 0; h < 16; ++h)
    if (h < G)
#pragma unroll
      for (int e = 0; e < DL; ++e)
        out[qb * o_sb + int64_t(g * G + h) * o_sh + lane + 64 * e] = n_tok > 0 ? acc[h][e] / l[h] : 0.f;
}

static inline int decode_parts(int head_dim, int max_blocks) {
  const int part = head_dim == 64 ? DecodeCfg<64>::NW * DecodeCfg<64>::PPW : DecodeCfg<128>::NW * DecodeCfg<128>::PPW;
  return (max_blocks + part - 1) / part;
}
static inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

}  // namespace ns

using namespace ns;

// Whole-row kernel: n_kv * head_dim == 128 (one 256-byte token row), <= 16 query heads, token rows
// contiguous in the pool, and a table width its merge covers.
// KV heads that are workgroup rows of their own: 1 when a token's K row (all KV heads) is 256 bytes
// (n_kv * head_dim == 128, token rows contiguous), n_kv for hd 128 with several KV heads (one head's 256
// bytes per workgroup row, tokens kv_spos apart); 0 when the whole-row kernel does not apply.
static inline int rows_kernel_grid_heads(int n_heads, int n_kv_heads, int head_dim, int64_t kv_spos, int64_t kv_sh,
                                         int max_blocks) {
  if ((max_blocks + ROWK_PART - 1) / ROWK_PART > ROWK_MAX_PARTS) return 0;
  if (n_kv_heads * head_dim == 128 && n_heads <= 16 && kv_sh == head_dim && kv_spos == 128) return 1;
  if (head_dim == 128 && n_kv_heads > 1 && n_heads / n_kv_heads <= 16 && kv_sh == 128 && kv_spos % 8 == 0)
    return n_kv_heads;
  return 0;
}
static inline size_t per_head_ws_bytes(int B, int n_kv_heads, int head_dim, int max_blocks) {
  const size_t parts = size_t(decode_parts(head_dim, max_blocks));
  if (parts <= 1) return 0;
  const size_t rows = size_t(B) * n_kv_heads, slots = rows * parts;
  return WS_COUNTER_BYTES + align256(slots * 16 * 2 * sizeof(float)) + align256(slots * 16 * size_t(head_dim) * sizeof(float));
}
static inline int rows_parts(int max_blocks) { return (max_blocks + ROWK_PART - 1) / ROWK_PART; }
static inline size_t rows_ws_bytes(int B, int head_dim, int max_blocks) {
  const size_t parts = size_t(rows_parts(max_blocks));
  if (parts <= 1) return 0;
  return WS_COUNTER_BYTES + align256(size_t(B) * parts * 32 * sizeof(float)) +
         align256(size_t(B) * parts * 16 * size_t(head_dim) * sizeof(float));
}

// Workspace: WS_COUNTER_BYTES of per-row arrival counters at offset 0 (zeroed once by the owner; every
// launch leaves them at zero, and no launch stores anything else there, so calls of any shape may share
// one buffer), then the partitions' (m, l) and accumulators. Sized for whichever kernel the shape takes.
extern "C" size_t ns_decode_workspace_bytes(int B, int n_kv_heads, int head_dim, int max_blocks, int dtype) {
  if (dtype != NS_DTYPE_BF16 || B <= 0 || n_kv_heads <= 0 || max_blocks <= 0) return 0;
  if (head_dim != 64 && head_dim != 128) return 0;
  const size_t a = per_head_ws_bytes(B, n_kv_heads, head_dim, max_blocks);
  const int rows_per_b = n_kv_heads * head_dim == 128 ? 1 : (head_dim == 128 ? n_kv_heads : 0);
  const size_t r = rows_per_b > 0 ? rows_ws_bytes(B * rows_per_b, head_dim, max_blocks) : 0;
  return a > r ? a : r;
}

// A whole-row launch prepared but not issued (paged_decode_launch with `defer`).
struct RowsLaunch {
  RowsArgs a;
  unsigned grid;
  int rgh, head_dim;
};
template <bool VALU, bool PAIR>
static void launch_rows_v(const RowsArgs& a, unsigned grid, int rgh, int head_dim, hipStream_t s) {
  if (rgh > 1)
    hipLaunchKernelGGL((paged_decode_rows_bf16_kernel<128, true, VALU, PAIR>), dim3(grid), dim3(ROWK_NW * 64), 0, s, a);
  else if (head_dim == 64)
    hipLaunchKernelGGL((paged_decode_rows_bf16_kernel<64, false, VALU, PAIR>), dim3(grid), dim3(ROWK_NW * 64), 0, s, a);
  else
    hipLaunchKernelGGL((paged_decode_rows_bf16_kernel<128, false, VALU, PAIR>), dim3(grid), dim3(ROWK_NW * 64), 0, s, a);
}
static void launch_rows(const RowsArgs& a, unsigned grid, int rgh, int head_dim, hipStream_t s, bool valu = false) {
  if (valu)
    launch_rows_v<true, false>(a, grid, rgh, head_dim, s);
  else if (a.pair != nullptr)
    launch_rows_v<false, true>(a, grid, rgh, head_dim, s);
  else
    launch_rows_v<false, false>(a, grid, rgh, head_dim, s);
}

// defer: when the whole-row kernel takes the call, fill *defer instead of launching (other kernels launch
// directly; defer->grid stays as the caller set it).
static int paged_decode_launch(const void* q, int64_t q_sb, int64_t q_sh, const void* k_pool, const void* v_pool,
                               int64_t kv_sblk, int64_t kv_spos, int64_t kv_sh, const int32_t* block_tables,
                               int64_t bt_sb, const int32_t* context_lens, void* out, int64_t o_sb, int64_t o_sh, int B,
                               int n_heads, int n_kv_heads, int head_dim, int block_size, int max_blocks,
                               int num_blocks, float scale, int dtype, void* workspace, size_t workspace_bytes,
                               void* stream, const int64_t* qrows = nullptr, RowsLaunch* defer = nullptr,
                               bool valu = false, const int32_t* pairs = nullptr) {
  NS_REQUIRE(dtype == NS_DTYPE_F32 || dtype == NS_DTYPE_BF16, "paged_attention_decode: dtype %d not supported",
             dtype);
  NS_REQUIRE(head_dim == 64 || head_dim == 128, "paged_attention_decode: head_dim %d not in {64, 128}", head_dim);
  NS_REQUIRE(block_size == PAGE, "paged_attention_decode: block_size %d, the kernels need %d", block_size, PAGE);
  NS_REQUIRE(n_kv_heads > 0 && n_heads > 0 && n_heads % n_kv_heads == 0,
             "paged_attention_decode: n_heads %d not a multiple of n_kv_heads %d", n_heads, n_kv_heads);
  const int G = n_heads / n_kv_heads;
  NS_REQUIRE(G <= 16, "paged_attention_decode: GQA group %d > 16", G);
  NS_REQUIRE(B >= 0 && B <= 65535 && n_kv_heads <= 65535, "paged_attention_decode: B=%d n_kv=%d out of range", B,
             n_kv_heads);
  NS_REQUIRE(max_blocks >= 1 && num_blocks >= 1, "paged_attention_decode: max_blocks %d num_blocks %d", max_blocks,
             num_blocks);
  if (B == 0) return NS_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (dtype == NS_DTYPE_F32) {
    if (head_dim == 64)
      hipLaunchKernelGGL(paged_decode_f32_kernel<64>, dim3(n_kv_heads, B), dim3(64), 0, s,
                         static_cast<const float*>(q), q_sb, q_sh, static_cast<const float*>(k_pool),
                         static_cast<const float*>(v_pool), kv_sblk, kv_spos, kv_sh, block_tables, bt_sb, context_lens,
                         static_cast<float*>(out), o_sb, o_sh, G, max_blocks, num_blocks, scale, qrows);
    else
      hipLaunchKernelGGL(paged_decode_f32_kernel<128>, dim3(n_kv_heads, B), dim3(64), 0, s,
                         static_cast<const float*>(q), q_sb, q_sh, static_cast<const float*>(k_pool),
                         static_cast<const float*>(v_pool), kv_sblk, kv_spos, kv_sh, block_tables, bt_sb, context_lens,
                         static_cast<float*>(out), o_sb, o_sh, G, max_blocks, num_blocks, scale, qrows);
    return check_launch("paged_attention_decode(f32)");
  }
  // bf16: 16-byte fragment loads need 8-element aligned strides and 16-byte aligned bases.
  NS_REQUIRE(q_sb % 8 == 0 && q_sh % 8 == 0 && kv_sblk % 8 == 0 && kv_spos % 8 == 0 && kv_sh % 8 == 0,
             "paged_attention_decode: bf16 strides must be multiples of 8 elements");
  NS_REQUIRE((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_pool) |
              reinterpret_cast<uintptr_t>(v_pool)) %
                     16 ==
                 0,
             "paged_attention_decode: q / k_pool / v_pool must be 16-byte aligned");
  const float sl2 = scale * LOG2E;
  const int rgh = rows_kernel_grid_heads(n_heads, n_kv_heads, head_dim, kv_spos, kv_sh, max_blocks);
  if (rgh > 0) {
    NS_REQUIRE(!valu || G <= (rgh > 1 ? ROWK_VALU_G_PH : ROWK_VALU_G),
               "paged_attention_decode_valu: GQA group %d above %d for this shape", G, rgh > 1 ? ROWK_VALU_G_PH : ROWK_VALU_G);
    const int rparts = rows_parts(max_blocks);
    const int rrows = B * rgh;
    NS_REQUIRE(rrows <= WS_MAX_COUNTERS, "paged_attention_decode: %d rows x KV heads exceed %d", rrows,
               WS_MAX_COUNTERS);
    unsigned* rcnt = nullptr;
    float* rml = nullptr;
    float* racc = nullptr;
    if (rparts > 1) {
      const size_t need = ns_decode_workspace_bytes(B, n_kv_heads, head_dim, max_blocks, dtype);
      if (workspace == nullptr || workspace_bytes < need) {
        set_error("paged_attention_decode: zero-initialised workspace of %zu bytes needed, got %zu", need,
                  workspace == nullptr ? size_t(0) : workspace_bytes);
        return NS_E_WORKSPACE;
      }
      NS_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0,
                 "paged_attention_decode: workspace not 256-byte aligned");
      char* w = static_cast<char*>(workspace);
      rcnt = reinterpret_cast<unsigned*>(w);
      rml = reinterpret_cast<float*>(w + WS_COUNTER_BYTES);
      racc = reinterpret_cast<float*>(w + WS_COUNTER_BYTES + align256(size_t(rrows) * rparts * 32 * sizeof(float)));
    }
    const int rstride = ws_counter_stride(size_t(rrows), size_t(WS_MAX_COUNTERS));
    RowsArgs ra{static_cast<const bf16_t*>(q), q_sb, q_sh, static_cast<const bf16_t*>(k_pool),
                static_cast<const bf16_t*>(v_pool), kv_sblk, block_tables, bt_sb, context_lens,
                static_cast<bf16_t*>(out), o_sb, o_sh, G, n_heads, max_blocks, num_blocks, sl2, rcnt, racc, rml, B,
                rparts, rgh, rgh > 1 ? kv_spos : int64_t(128), kv_sh, qrows, rstride};
    if (pairs != nullptr && !valu && 2 * (rgh > 1 ? G : n_heads) <= 16) ra.pair = pairs;
    const unsigned rgrid = unsigned(rparts) * unsigned(rrows);
    if (defer != nullptr) {   // the caller launches these workgroups (beside others)
      *defer = RowsLaunch{ra, rgrid, rgh, head_dim};
      return NS_OK;
    }
    launch_rows(ra, rgrid, rgh, head_dim, s, valu);
    return check_launch("paged_attention_decode(bf16 rows)");
  }
  NS_REQUIRE(!valu, "paged_attention_decode_valu: not a whole-row shape (n_kv * head_dim == 128, or head_dim 128 "
                    "with several KV heads)");
  const int parts = decode_parts(head_dim, max_blocks);
  const int max_parts = head_dim == 64 ? MERGE_MAX_PARTS<64> : MERGE_MAX_PARTS<128>;
  NS_REQUIRE(parts <= max_parts, "paged_attention_decode: %d partitions (table width %d) exceed %d", parts, max_blocks,
             max_parts);
  float* ws_acc = nullptr;
  float* ws_ml = nullptr;
  unsigned* ws_cnt = nullptr;
  if (parts > 1) {
    const size_t need = per_head_ws_bytes(B, n_kv_heads, head_dim, max_blocks);
    if (workspace == nullptr || workspace_bytes < need) {
      set_error("paged_attention_decode: zero-initialised workspace of %zu bytes needed, got %zu", need,
                workspace == nullptr ? size_t(0) : workspace_bytes);
      return NS_E_WORKSPACE;
    }
    NS_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "paged_attention_decode: workspace not 256-byte aligned");
    const size_t rows = size_t(B) * n_kv_heads, slots = rows * parts;
    NS_REQUIRE(rows <= size_t(WS_MAX_COUNTERS), "paged_attention_decode: %zu rows x KV heads exceed %d", rows,
               WS_MAX_COUNTERS);
    char* w = static_cast<char*>(workspace);
    ws_cnt = reinterpret_cast<unsigned*>(w);
    ws_ml = reinterpret_cast<float*>(w + WS_COUNTER_BYTES);
    ws_acc = reinterpret_cast<float*>(w + WS_COUNTER_BYTES + align256(slots * 16 * 2 * sizeof(float)));
  }
  const int pstride = ws_counter_stride(size_t(B) * n_kv_heads, size_t(WS_MAX_COUNTERS));
  const dim3 grid(unsigned(parts) * unsigned(n_kv_heads) * unsigned(B));
  if (head_dim == 64)
    hipLaunchKernelGGL(paged_decode_bf16_kernel<64>, grid, dim3(DecodeCfg<64>::NW * 64), 0, s,
                       static_cast<const bf16_t*>(q), q_sb, q_sh, static_cast<const bf16_t*>(k_pool),
                       static_cast<const bf16_t*>(v_pool), kv_sblk, kv_spos, kv_sh, block_tables, bt_sb, context_lens,
                       static_cast<bf16_t*>(out), o_sb, o_sh, G, max_blocks, num_blocks, sl2, ws_acc, ws_ml, ws_cnt, B,
                       n_kv_heads, parts, qrows, pstride);
  else
    hipLaunchKernelGGL(paged_decode_bf16_kernel<128>, grid, dim3(DecodeCfg<128>::NW * 64), 0, s,
                       static_cast<const bf16_t*>(q), q_sb, q_sh, static_cast<const bf16_t*>(k_pool),
                       static_cast<const bf16_t*>(v_pool), kv_sblk, kv_spos, kv_sh, block_tables, bt_sb, context_lens,
                       static_cast<bf16_t*>(out), o_sb, o_sh, G, max_blocks, num_blocks, sl2, ws_acc, ws_ml, ws_cnt, B,
                       n_kv_heads, parts, qrows, pstride);
  return check_launch("paged_attention_decode(bf16)");
}

extern "C" int ns_paged_attn_decode_rows(const void* q, int64_t q_sb, int64_t q_sh, const void* k_pool,
                                         const void* v_pool, int64_t kv_sblk, int64_t kv_spos, int64_t kv_sh,
                                         const int32_t* block_tables, int64_t bt_sb, const int32_t* context_lens,
                                         const int64_t* q_rows, void* out, int64_t o_sb, int64_t o_sh, int B,
                                         int n_heads, int n_kv_heads, int head_dim, int block_size, int max_blocks,
                                         int num_blocks, float scale, int dtype, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  NS_REQUIRE(q_rows != nullptr, "paged_attention_decode_rows: q_rows is NULL");
  return paged_decode_launch(q, q_sb, q_sh, k_pool, v_pool, kv_sblk, kv_spos, kv_sh, block_tables, bt_sb,
                             context_lens, out, o_sb, o_sh, B, n_heads, n_kv_heads, head_dim, block_size, max_blocks,
                             num_blocks, scale, dtype, workspace, workspace_bytes, stream, q_rows);
}

extern "C" int ns_paged_attn_mixed(const void* q, int64_t q_sb, int64_t q_sh, const void* k_pool, const void* v_pool,
                                   int64_t kv_sblk, int64_t kv_spos, int64_t kv_sh, const int32_t* pf_block_tables,
                                   int64_t pf_bt_sb, const int32_t* seq_info, int n_seqs, int max_new, int max_kv,
                                   int pf_max_blocks, void* pf_workspace, size_t pf_workspace_bytes,
                                   const int32_t* dec_block_tables, int64_t dec_bt_sb, const int32_t* context_lens,
                                   const int64_t* q_rows, int B, int dec_max_blocks, void* dec_workspace,
                                   size_t dec_workspace_bytes, void* out, int64_t o_sb, int64_t o_sh, int n_heads,
                                   int n_kv_heads, int head_dim, int block_size, int num_blocks, float scale, int dtype,
                                   void* stream) {
  NS_REQUIRE(q_rows != nullptr || B == 0, "paged_attention_mixed: q_rows is NULL");
  PrefillArgs pa;
  int64_t n_pf = 0;
  int st = prefill_prepare(q, q_sb, q_sh, k_pool, v_pool, kv_sblk, kv_spos, kv_sh, pf_block_tables, pf_bt_sb, seq_info,
                           n_seqs, max_new, max_kv, out, o_sb, o_sh, n_heads, n_kv_heads, head_dim, block_size,
                           pf_max_blocks, num_blocks, scale, dtype, pf_workspace, pf_workspace_bytes, &pa, &n_pf);
  if (st != NS_OK) return st;
  RowsLaunch rl{};
  rl.grid = 0;
  if (B > 0) {   // validates the decode rows; launches them itself unless the whole-row kernel takes them
    st = paged_decode_launch(q, q_sb, q_sh, k_pool, v_pool, kv_sblk, kv_spos, kv_sh, dec_block_tables, dec_bt_sb,
                             context_lens, out, o_sb, o_sh, B, n_heads, n_kv_heads, head_dim, block_size,
                             dec_max_blocks, num_blocks, scale, dtype, dec_workspace, dec_workspace_bytes, stream,
                             q_rows, &rl);
    if (st != NS_OK) return st;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (n_pf == 0 || rl.grid == 0) {   // one side only: its own kernel
    if (rl.grid > 0) launch_rows(rl.a, rl.grid, rl.rgh, rl.head_dim, s);
    if (n_pf > 0) {
      const dim3 grid{unsigned(n_pf)};
      if (head_dim == 64)   // every workgroup a prefill one
        hipLaunchKernelGGL((mixed_attn_kernel<64, false>), grid, dim3(PF_WG_THREADS), 0, s, pa, int(n_pf), rl.a);
      else
        hipLaunchKernelGGL((mixed_attn_kernel<128, false>), grid, dim3(PF_WG_THREADS), 0, s, pa, int(n_pf), rl.a);
    }
    return check_launch("paged_attention_mixed");
  }
  // the prefill part padded to a multiple of 8 workgroups (the extra ones find no unit and return), so the
  // decode workgroups keep the XCD rotation they have in their own kernel (workgroup i runs on XCD i % 8)
  const int64_t n_pf8 = (n_pf + 7) & ~int64_t(7);
  NS_REQUIRE(n_pf8 + int64_t(rl.grid) < (int64_t(1) << 31), "paged_attention_mixed: %lld workgroups",
             (long long)(n_pf8 + rl.grid));
  const dim3 grid{unsigned(n_pf8 + rl.grid)};
  const int npf = int(n_pf8);
  if (rl.rgh > 1)
    hipLaunchKernelGGL((mixed_attn_kernel<128, true>), grid, dim3(PF_WG_THREADS), 0, s, pa, npf, rl.a);
  else if (rl.head_dim == 64)
    hipLaunchKernelGGL((mixed_attn_kernel<64, false>), grid, dim3(PF_WG_THREADS), 0, s, pa, npf, rl.a);
  else
    hipLaunchKernelGGL((mixed_attn_kernel<128, false>), grid, dim3(PF_WG_THREADS), 0, s, pa, npf, rl.a);
  return check_launch("paged_attention_mixed");
}

extern "C" int ns_paged_attn_decode(const void* q, int64_t q_sb, int64_t q_sh, const void* k_pool,
                                    const void* v_pool, int64_t kv_sblk, int64_t kv_spos, int64_t kv_sh,
                                    const int32_t* block_tables, int64_t bt_sb, const int32_t* context_lens,
                                    void* out, int64_t o_sb, int64_t o_sh, int B, int n_heads, int n_kv_heads,
                                    int head_dim, int block_size, int max_blocks, int num_blocks, float scale,
                                    int dtype, void* workspace, size_t workspace_bytes, void* stream) {
  return paged_decode_launch(q, q_sb, q_sh, k_pool, v_pool, kv_sblk, kv_spos, kv_sh, block_tables, bt_sb,
                             context_lens, out, o_sb, o_sh, B, n_heads, n_kv_heads, head_dim, block_size, max_blocks,
                             num_blocks, scale, dtype, workspace, workspace_bytes, stream);
}

extern "C" int ns_paged_attn_decode_pairs(const void* q, int64_t q_sb, int64_t q_sh, const void* k_pool,
                                          const void* v_pool, int64_t kv_sblk, int64_t kv_spos, int64_t kv_sh,
                                          const int32_t* block_tables, int64_t bt_sb, const int32_t* context_lens,
                                          const int32_t* pairs, void* out, int64_t o_sb, int64_t o_sh, int B,
                                          int n_heads, int n_kv_heads, int head_dim, int block_size, int max_blocks,
                                          int num_blocks, float scale, int dtype, void* workspace,
                                          size_t workspace_bytes, void* stream) {
  NS_REQUIRE(pairs != nullptr, "paged_attention_decode_pairs: pairs is NULL");
  return paged_decode_launch(q, q_sb, q_sh, k_pool, v_pool, kv_sblk, kv_spos, kv_sh, block_tables, bt_sb,
                             context_lens, out, o_sb, o_sh, B, n_heads, n_kv_heads, head_dim, block_size, max_blocks,
                             num_blocks, scale, dtype, workspace, workspace_bytes, stream, nullptr, nullptr, false,
                             pairs);
}

extern "C" int ns_paged_attn_decode_valu(const void* q, int64_t q_sb, int64_t q_sh, const void* k_pool,
                                         const void* v_pool, int64_t kv_sblk, int64_t kv_spos, int64_t kv_sh,
                                         const int32_t* block_tables, int64_t bt_sb, const int32_t* context_lens,
                                         void* out, int64_t o_sb, int64_t o_sh, int B, int n_heads, int n_kv_heads,
                                         int head_dim, int block_size, int max_blocks, int num_blocks, float scale,
                                         int dtype, void* workspace, size_t workspace_bytes, void* stream) {
  NS_REQUIRE(dtype == NS_DTYPE_BF16, "paged_attention_decode_valu: bf16 only (dtype %d)", dtype);
  NS_REQUIRE(n_kv_heads > 0 && n_heads % n_kv_heads == 0 && n_heads / n_kv_heads <= ROWK_VALU_G,
             "paged_attention_decode_valu: GQA group %d / %d above %d", n_heads, n_kv_heads, ROWK_VALU_G);
  return paged_decode_launch(q, q_sb, q_sh, k_pool, v_pool, kv_sblk, kv_spos, kv_sh, block_tables, bt_sb,
                             context_lens, out, o_sb, o_sh, B, n_heads, n_kv_heads, head_dim, block_size, max_blocks,
                             num_blocks, scale, dtype, workspace, workspace_bytes, stream, nullptr, nullptr, true);
}

// ---------------------------------------------------------------------------------------------------------
// Allocation-free variant: the split-K workspace is a file-scope device array instead of a caller buffer.
// In host code `scratch` names a host-side stand-in, not device memory: its device address is looked up
// once per device with hipGetSymbolAddress and only that address is passed to kernels.
// ---------------------------------------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[NS_DECODE_SCRATCH_BYTES];

namespace ns {

__global__ void zero_words_kernel(uint32_t* p, size_t n_words) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n_words; i += size_t(gridDim.x) * blockDim.x)
    p[i] = 0u;
}

constexpr int MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[MAX_DEVICES] = {};

// Device address of this device's `scratch`, looked up (and cleared, by a fill kernel on `s`, ordered
// before the caller's launch) the first time a call runs with the device current.
static int scratch_for_current_device(hipStream_t s, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("paged_attention_decode_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return NS_E_HIP_BASE + int(e);
  }
  NS_REQUIRE(dev >= 0 && dev < MAX_DEVICES, "paged_attention_decode_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("paged_attention_decode_noalloc: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
      return NS_E_HIP_BASE + int(e == hipSuccess ? hipErrorInvalidSymbol : e);
    }
    hipLaunchKernelGGL(zero_words_kernel, dim3(256), dim3(256), 0, s, static_cast<uint32_t*>(p),
                       size_t(NS_DECODE_SCRATCH_BYTES) / 4);
    const int st = check_launch("paged_attention_decode_noalloc(scratch clear)");
    if (st != NS_OK) return st;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return NS_OK;
}

}  // namespace ns

extern "C" int ns_paged_attn_decode_noalloc(const void* q, int64_t q_sb, int64_t q_sh, const void* k_pool,
                                            const void* v_pool, int64_t kv_sblk, int64_t kv_spos, int64_t kv_sh,
                                            const int32_t* block_tables, int64_t bt_sb, const int32_t* context_lens,
                                            void* out, int64_t o_sb, int64_t o_sh, int B, int n_heads,
                                            int n_kv_heads, int head_dim, int block_size, int max_blocks,
                                            int num_blocks, float scale, int dtype, void* stream) {
  const size_t need = ns_decode_workspace_bytes(B, n_kv_heads, head_dim, max_blocks, dtype);
  NS_REQUIRE(need <= size_t(NS_DECODE_SCRATCH_BYTES),
             "paged_attention_decode_noalloc: this shape (B=%d, n_kv=%d, head_dim=%d, table width %d) needs %zu "
             "bytes of split-K scratch, more than the library's fixed %zu",
             B, n_kv_heads, head_dim, max_blocks, need, size_t(NS_DECODE_SCRATCH_BYTES));
  void* ws = nullptr;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (need > 0) {
    const int st = scratch_for_current_device(s, &ws);
    if (st != NS_OK) return st;
  }
  return paged_decode_launch(q, q_sb, q_sh, k_pool, v_pool, kv_sblk, kv_spos, kv_sh, block_tables, bt_sb,
                             context_lens, out, o_sb, o_sh, B, n_heads, n_kv_heads, head_dim, block_size, max_blocks,
                             num_blocks, scale, dtype, ws, need > 0 ? size_t(NS_DECODE_SCRATCH_BYTES) : 0, stream);
}
