// Chunked-prefill attention launch (the kernel's body and its design notes: prefill_body.h).
#include "prefill_body.h"

namespace ns {
namespace {

template <int HD>
__global__ __launch_bounds__(PF_WG_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void paged_prefill_bf16_kernel(PrefillArgs a) {
  __shared__ __align__(16) unsigned char lds[PF_GROUPS * 2 * PfLds<HD>::STAGE];
  __shared__ unsigned s_last;
  prefill_body<HD>(a, int(blockIdx.x), lds, s_last);
}

}  // namespace
}  // namespace ns

using namespace ns;

// Workspace: the fixed counter region (one arrival counter per tile of [n_seqs, n_heads, tiles]; shared
// safely by calls of any shape), then per work unit the (m, l) and the accumulators of a tile's partition.
// Zero bytes when no tile can span more than one partition.
extern "C" size_t ns_prefill_workspace_bytes(int n_seqs, int n_heads, int head_dim, int max_new, int max_kv) {
  return prefill_workspace_need(n_seqs, n_heads, head_dim, max_new, max_kv);
}

extern "C" int ns_paged_attn_prefill(const void* q, int64_t q_st, int64_t q_sh, const void* k_pool, const void* v_pool,
                                     int64_t kv_sblk, int64_t kv_spos, int64_t kv_sh, const int32_t* block_tables,
                                     int64_t bt_sb, const int32_t* seq_info, int n_seqs, int max_new, int max_kv,
                                     void* out, int64_t o_st, int64_t o_sh, int n_heads, int n_kv_heads,
                                     int head_dim, int block_size, int max_blocks, int num_blocks, float scale,
                                     int dtype, void* workspace, size_t workspace_bytes, void* stream) {
  PrefillArgs a;
  int64_t n_wg = 0;
  const int st = prefill_prepare(q, q_st, q_sh, k_pool, v_pool, kv_sblk, kv_spos, kv_sh, block_tables, bt_sb, seq_info,
                                 n_seqs, max_new, max_kv, out, o_st, o_sh, n_heads, n_kv_heads, head_dim, block_size,
                                 max_blocks, num_blocks, scale, dtype, workspace, workspace_bytes, &a, &n_wg);
  if (st != NS_OK || n_wg == 0) return st;
  const dim3 grid{unsigned(n_wg)};
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (head_dim == 64)
    hipLaunchKernelGGL(paged_prefill_bf16_kernel<64>, grid, dim3(PF_WG_THREADS), 0, s, a);
  else
    hipLaunchKernelGGL(paged_prefill_bf16_kernel<128>, grid, dim3(PF_WG_THREADS), 0, s, a);
  return check_launch("paged_attention_prefill");
}
