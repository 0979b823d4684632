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
//   * Each wave issues every K and V load of its pages up front (16-byte, coalesced per token row),
//     then works page by page with matrix cores. The GQA group makes both products dense:
//       S^T[16 tok x 16 heads] = K_page[16 x hd] . Q^T[hd x 16]            (mfma 16x16x32 bf16)
//       O^T[hd x 16 heads]    += V_page^T[hd x 16 tok] . P^T[16 tok x 16]  (mfma 16x16x16 bf16)
//     Rows >= G of Q are zero. The S^T output layout (lane = head, 4 consecutive tokens) is exactly
//     the B-operand layout P^T needs, so P never leaves registers; only V is transposed, through a
//     wave-private LDS tile of one page.
//   * Softmax statistics per head: a lane's 4 tokens, then 2 butterfly shuffles (xor 16, xor 32).
//   * Waves merge through LDS; a row with one partition writes its output directly, otherwise each
//     partition writes (m, l, acc) to the workspace and the last one to arrive (device-scope
//     counter) merges them and resets the counter to zero for the next call.
// fp32 design: one wave per (row, KV head), VALU dot products with wave reductions; kept simple,
// it serves the fp32 correctness paths.
#include "ns_common.h"

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

__device__ __forceinline__ uint4 zero4() { return make_uint4(0u, 0u, 0u, 0u); }

template <int HD>
__global__ __launch_bounds__(DecodeCfg<HD>::NW * 64) void paged_decode_bf16_kernel(
    const bf16_t* __restrict__ q, int64_t q_sb, int64_t q_sh, const bf16_t* __restrict__ kp,
    const bf16_t* __restrict__ vp, int64_t s_blk, int64_t s_pos, int64_t s_h, const int32_t* __restrict__ bt,
    int64_t bt_sb, const int32_t* __restrict__ ctxl, bf16_t* __restrict__ out, int64_t o_sb, int64_t o_sh, int G,
    int max_blocks, int num_blocks, float scale_log2, float* __restrict__ ws_acc, float* __restrict__ ws_ml,
    uint32_t* __restrict__ counters) {
  constexpr int NW = DecodeCfg<HD>::NW, PPW = DecodeCfg<HD>::PPW, PART = NW * PPW;
  constexpr int KS = HD / 32;  // 32-dim k-steps of the QK^T product (8 bf16 per lane per step)
  constexpr int NT = HD / 16;  // 16-dim output tiles of the PV product
  constexpr int VROW = HD + 8; // LDS row pitch of the V tile (bf16), padded against bank conflicts
  const int part = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int nkv = gridDim.y, n_parts = gridDim.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c16 = lane & 15;   // MFMA column: head (QK^T B / output) or token row (A operands)
  const int r4 = lane >> 4;    // MFMA row group: owns rows / k-values 4*r4 .. 4*r4+3 (8*r4.. for x32)

  const int ctx = ctxl[b];
  int n_pages = ctx > 0 ? (ctx + PAGE - 1) / PAGE : 0;
  if (n_pages > max_blocks) n_pages = max_blocks;
  const int p0 = part * PART;
  if (ctx <= 0) {  // no keys: zeros (the row is invalid; nothing to attend to)
    if (part == 0)
      for (int i = tid; i < G * HD; i += NW * 64)
        out[int64_t(b) * o_sb + int64_t(g * G + i / HD) * o_sh + (i % HD)] = bf16_t(0);
    return;
  }
  if (p0 >= n_pages) return;  // whole workgroup: this partition is past the row's context
  const int n_active = (n_pages + PART - 1) / PART;

  // ---- issue loads: Q (B operand, zero rows >= G), then every K and V fragment of this wave's pages
  bf16x8_t qf[KS];
  {
    const bool hv = c16 < G;
    const bf16_t* qrow = q + int64_t(b) * q_sb + int64_t(g * G + (hv ? c16 : 0)) * q_sh;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      uint4 u = hv ? *reinterpret_cast<const uint4*>(qrow + 32 * s + 8 * r4) : zero4();
      qf[s] = __builtin_bit_cast(bf16x8_t, u);
    }
  }
  uint4 kf[PPW][KS], vf[PPW][KS];
  int my_pages = 0;
#pragma unroll
  for (int i = 0; i < PPW; ++i) {
    const int p = p0 + w + NW * i;
    const bool live = p < n_pages;
    my_pages += live ? 1 : 0;
    int blk = live ? bt[int64_t(b) * bt_sb + p] : -1;
    const bool ok = live && blk >= 0 && blk < num_blocks;
    const int64_t off = int64_t(ok ? blk : 0) * s_blk + int64_t(c16) * s_pos + int64_t(g) * s_h + 8 * r4;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      kf[i][s] = ok ? *reinterpret_cast<const uint4*>(kp + off + 32 * s) : zero4();
      vf[i][s] = ok ? *reinterpret_cast<const uint4*>(vp + off + 32 * s) : zero4();
    }
  }

  __shared__ __align__(16) bf16_t vtile[NW][PAGE * VROW];
  bf16_t* vt = vtile[w];

  float m_run = -INFINITY, l_run = 0.f;
  float4_t acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = float4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int i = 0; i < PPW; ++i) {
    if (i < my_pages) {
      const int p = p0 + w + NW * i;
      // S^T = K . Q^T : lane holds tokens 4*r4 + j (j = 0..3) of head c16
      float4_t st = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s)
        st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kf[i][s]), qf[s], st, 0, 0, 0);
      float sv[4];
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tok = p * PAGE + 4 * r4 + j;
        sv[j] = tok < ctx ? st[j] * scale_log2 : -INFINITY;
        mx = fmaxf(mx, sv[j]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx);
      const float alpha = exp2f(m_run - m_new);
      float pv[4], psum = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pv[j] = exp2f(sv[j] - m_new);
        psum += pv[j];
      }
      l_run = l_run * alpha + psum;
      m_run = m_new;
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] *= alpha;
      // P^T as the B operand (k = token 4*r4 + j, n = head c16), rounded to bf16
      short4_t pb;
#pragma unroll
      for (int j = 0; j < 4; ++j) pb[j] = short(f32_to_bf16(pv[j]));

      // V page -> LDS (natural [token][dim] layout), then read V^T fragments.
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int s = 0; s < KS; ++s) *reinterpret_cast<uint4*>(vt + c16 * VROW + 32 * s + 8 * r4) = vf[i][s];
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        short4_t va;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int tok = p * PAGE + 4 * r4 + j;
          const bf16_t x = vt[(4 * r4 + j) * VROW + 16 * t + c16];
          va[j] = short(tok < ctx ? x : bf16_t(0));  // keys past ctx contribute exactly nothing
        }
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, pb, acc[t], 0, 0, 0);
      }
    }
  }
  // per-head sum over the 4 lane groups (same running max in all of them)
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);

  // ---- merge the NW waves through LDS: acc layout [wave][head][dim]
  constexpr int AROW = HD + 4;
  __shared__ float sm_acc[NW][16 * AROW];
  __shared__ float sm_m[NW][16], sm_l[NW][16];
  __shared__ int sm_last;
  if (r4 == 0) {
    sm_m[w][c16] = m_run;
    sm_l[w][c16] = l_run;
  }
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) sm_acc[w][c16 * AROW + 16 * t + 4 * r4 + j] = acc[t][j];
  __syncthreads();

  const int64_t bg = int64_t(b) * nkv + g;
  for (int idx = tid; idx < G * HD; idx += NW * 64) {
    const int h = idx / HD, d = idx - (idx / HD) * HD;
    float M = -INFINITY;
#pragma unroll
    for (int x = 0; x < NW; ++x) M = fmaxf(M, sm_m[x][h]);
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int x = 0; x < NW; ++x) {
      const float wgt = exp2f(sm_m[x][h] - M);  // waves without pages: m = -inf -> weight 0
      L += wgt * sm_l[x][h];
      A += wgt * sm_acc[x][h * AROW + d];
    }
    if (n_active == 1) {
      out[int64_t(b) * o_sb + int64_t(g * G + h) * o_sh + d] = f32_to_bf16(A / L);
    } else {
      ws_acc[(bg * n_parts + part) * (16 * HD) + h * HD + d] = A;
      if (d == 0) {
        ws_ml[((bg * n_parts + part) * 16 + h) * 2 + 0] = M;
        ws_ml[((bg * n_parts + part) * 16 + h) * 2 + 1] = L;
      }
    }
  }
  if (n_active == 1) return;

  // ---- cross-partition merge by the last partition to finish
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = atomicAdd(&counters[bg], 1u);
    sm_last = (prev == uint32_t(n_active - 1)) ? 1 : 0;
  }
  __syncthreads();
  if (!sm_last) return;
  __threadfence();
  for (int idx = tid; idx < G * HD; idx += NW * 64) {
    const int h = idx / HD, d = idx - (idx / HD) * HD;
    float M = -INFINITY;
    for (int x = 0; x < n_active; ++x) M = fmaxf(M, ws_ml[((bg * n_parts + x) * 16 + h) * 2]);
    float L = 0.f, A = 0.f;
    for (int x = 0; x < n_active; ++x) {
      const float wgt = exp2f(ws_ml[((bg * n_parts + x) * 16 + h) * 2] - M);
      L += wgt * ws_ml[((bg * n_parts + x) * 16 + h) * 2 + 1];
      A += wgt * ws_acc[(bg * n_parts + x) * (16 * HD) + h * HD + d];
    }
    out[int64_t(b) * o_sb + int64_t(g * G + h) * o_sh + d] = f32_to_bf16(A / L);
  }
  if (tid == 0) counters[bg] = 0u;  // ready for the next call / graph replay
}

// fp32: one wave per (row, KV head). Lane owns dims lane and lane + 64 (hd 128).
template <int HD>
__global__ __launch_bounds__(64) void paged_decode_f32_kernel(
    const float* __restrict__ q, int64_t q_sb, int64_t q_sh, const float* __restrict__ kp,
    const float* __restrict__ vp, int64_t s_blk, int64_t s_pos, int64_t s_h, const int32_t* __restrict__ bt,
    int64_t bt_sb, const int32_t* __restrict__ ctxl, float* __restrict__ out, int64_t o_sb, int64_t o_sh, int G,
    int max_blocks, int num_blocks, float scale) {
  constexpr int DL = HD / 64;  // dims per lane
  const int g = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
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
      qv[h][e] = h < G ? q[int64_t(b) * q_sb + int64_t(g * G + h) * q_sh + lane + 64 * e] : 0.f;
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
        out[int64_t(b) * o_sb + int64_t(g * G + h) * o_sh + lane + 64 * e] = n_tok > 0 ? acc[h][e] / l[h] : 0.f;
}

static inline int decode_parts(int head_dim, int max_blocks) {
  const int part = head_dim == 64 ? DecodeCfg<64>::NW * DecodeCfg<64>::PPW : DecodeCfg<128>::NW * DecodeCfg<128>::PPW;
  return (max_blocks + part - 1) / part;
}
static inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

}  // namespace ns

using namespace ns;

extern "C" size_t ns_decode_counter_bytes(int B, int n_kv_heads) {
  if (B <= 0 || n_kv_heads <= 0) return 0;
  return align256(size_t(B) * n_kv_heads * sizeof(uint32_t));
}

extern "C" size_t ns_decode_workspace_bytes(int B, int n_kv_heads, int head_dim, int max_blocks, int dtype) {
  if (dtype != NS_DTYPE_BF16 || B <= 0 || n_kv_heads <= 0 || max_blocks <= 0) return 0;
  if (head_dim != 64 && head_dim != 128) return 0;
  const size_t parts = size_t(decode_parts(head_dim, max_blocks));
  if (parts <= 1) return 0;
  const size_t slots = size_t(B) * n_kv_heads * parts;
  return ns_decode_counter_bytes(B, n_kv_heads) + align256(slots * 16 * 2 * sizeof(float)) +
         align256(slots * 16 * size_t(head_dim) * sizeof(float));
}

extern "C" int ns_paged_attn_decode(const void* q, int64_t q_sb, int64_t q_sh, const void* k_pool,
                                    const void* v_pool, int64_t kv_sblk, int64_t kv_spos, int64_t kv_sh,
                                    const int32_t* block_tables, int64_t bt_sb, const int32_t* context_lens,
                                    void* out, int64_t o_sb, int64_t o_sh, int B, int n_heads, int n_kv_heads,
                                    int head_dim, int block_size, int max_blocks, int num_blocks, float scale,
                                    int dtype, void* workspace, size_t workspace_bytes, void* stream) {
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
                         static_cast<float*>(out), o_sb, o_sh, G, max_blocks, num_blocks, scale);
    else
      hipLaunchKernelGGL(paged_decode_f32_kernel<128>, dim3(n_kv_heads, B), dim3(64), 0, s,
                         static_cast<const float*>(q), q_sb, q_sh, static_cast<const float*>(k_pool),
                         static_cast<const float*>(v_pool), kv_sblk, kv_spos, kv_sh, block_tables, bt_sb, context_lens,
                         static_cast<float*>(out), o_sb, o_sh, G, max_blocks, num_blocks, scale);
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
  const int parts = decode_parts(head_dim, max_blocks);
  NS_REQUIRE(parts <= 65535, "paged_attention_decode: %d partitions exceed the grid limit", parts);
  float* ws_acc = nullptr;
  float* ws_ml = nullptr;
  uint32_t* counters = nullptr;
  if (parts > 1) {
    const size_t need = ns_decode_workspace_bytes(B, n_kv_heads, head_dim, max_blocks, dtype);
    if (workspace == nullptr || workspace_bytes < need) {
      set_error("paged_attention_decode: workspace of %zu bytes needed, got %zu", need,
                workspace == nullptr ? size_t(0) : workspace_bytes);
      return NS_E_WORKSPACE;
    }
    NS_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "paged_attention_decode: workspace not 256-byte aligned");
    char* base = static_cast<char*>(workspace);
    const size_t slots = size_t(B) * n_kv_heads * parts;
    counters = reinterpret_cast<uint32_t*>(base);
    ws_ml = reinterpret_cast<float*>(base + ns_decode_counter_bytes(B, n_kv_heads));
    ws_acc = reinterpret_cast<float*>(base + ns_decode_counter_bytes(B, n_kv_heads) +
                                      align256(slots * 16 * 2 * sizeof(float)));
  }
  const float sl2 = scale * LOG2E;
  const dim3 grid(parts, n_kv_heads, B);
  if (head_dim == 64)
    hipLaunchKernelGGL(paged_decode_bf16_kernel<64>, grid, dim3(DecodeCfg<64>::NW * 64), 0, s,
                       static_cast<const bf16_t*>(q), q_sb, q_sh, static_cast<const bf16_t*>(k_pool),
                       static_cast<const bf16_t*>(v_pool), kv_sblk, kv_spos, kv_sh, block_tables, bt_sb, context_lens,
                       static_cast<bf16_t*>(out), o_sb, o_sh, G, max_blocks, num_blocks, sl2, ws_acc, ws_ml, counters);
  else
    hipLaunchKernelGGL(paged_decode_bf16_kernel<128>, grid, dim3(DecodeCfg<128>::NW * 64), 0, s,
                       static_cast<const bf16_t*>(q), q_sb, q_sh, static_cast<const bf16_t*>(k_pool),
                       static_cast<const bf16_t*>(v_pool), kv_sblk, kv_spos, kv_sh, block_tables, bt_sb, context_lens,
                       static_cast<bf16_t*>(out), o_sb, o_sh, G, max_blocks, num_blocks, sl2, ws_acc, ws_ml, counters);
  return check_launch("paged_attention_decode(bf16)");
}
