/*
 * nanoserve_hip.h — C ABI of libnanoserve_hip.so, the gfx950 kernels of the decode token loop.
 *
 * Every entry point:
 *   - takes raw device pointers and sizes (no framework types), plus the hipStream_t to launch on
 *     (passed as void*; torch's torch.cuda.current_stream().cuda_stream on PyTorch-ROCm);
 *   - only enqueues work: it never synchronises, never allocates or frees device memory, and its
 *     launch grid depends on its integer arguments only, so it can be recorded into a hipGraph;
 *   - returns 0 on success or a nonzero status (NS_E_* below, or a hipError_t value + 1000). The
 *     message for the last failure on the calling thread is returned by ns_last_error().
 *
 * dtype codes: NS_DTYPE_F32 = 0, NS_DTYPE_BF16 = 1. Pool layout of one layer's K or V cache:
 * [num_blocks, block_size, n_kv_heads, head_dim] with head_dim contiguous (strides in elements).
 *
 * Each function cites the reference interface it replaces (darshanseenivasakumar/nanoserve,
 * Triton kernels called from nanoserve/model.py).
 */
#ifndef NANOSERVE_HIP_H
#define NANOSERVE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NS_DTYPE_F32 0
#define NS_DTYPE_BF16 1

/* Row statistics of an RMSNorm input (r and, per 16 columns, the row sums of r^2) are fp32
 * [ceil(n / 16)][NS_NORM_ROWS]: row m of 16-column group p at p * NS_NORM_ROWS + m, for up to NS_NORM_ROWS rows. */
#define NS_NORM_ROWS 128

/* Split-K workspaces (ns_paged_attn_decode, ns_paged_attn_prefill, ns_argmax_rows) begin with this many
 * bytes of arrival counters. Every call leaves them at zero and nothing else is ever stored there, so one
 * zero-filled workspace may serve calls of any shape, in any order, on one stream. */
#define NS_WS_COUNTER_BYTES (256u << 10)

#define NS_OK 0
#define NS_E_INVALID 1      /* argument outside what the kernels support (message says which) */
#define NS_E_WORKSPACE 2    /* workspace pointer missing or smaller than ns_decode_workspace_bytes */
#define NS_E_HIP_BASE 1000  /* 1000 + hipError_t of a failed launch */

/* Message of the last failing call on this thread ("" if none). */
const char* ns_last_error(void);

/* Library version string (build id of the kernels). */
const char* ns_version(void);

/*
 * Paged-attention decode: for each row b and query head h (KV head g = h / (n_heads / n_kv_heads)),
 *   out[b, h, :] = softmax(q[b, h, :] . K[0:ctx_b]^T * scale) . V[0:ctx_b]
 * where token t of row b lives at pool block block_tables[b, t / block_size], position t % block_size.
 * Online softmax with fp32 running max / sum / accumulator; probabilities are rounded to the value
 * dtype before the P.V product. Pages named by table entries past ceil(ctx_b / block_size) are never
 * read; the entries themselves may be (block ids are loaded before the context length is known), so each
 * row must hold max_blocks readable int32 entries, whatever their values.
 * Replaces nanoserve/kernels/paged_attention.py:85 paged_attention_decode (kernel :34-82).
 *
 * Limits: head_dim in {64, 128}; block_size == 16; n_heads / n_kv_heads <= 16; ctx_b >= 1
 * (a row with ctx_b <= 0 gets zeros). Guards that keep every access inside the caller's buffers:
 * a row's page count is clamped to max_blocks (the table width), and the tokens of a table entry
 * outside [0, num_blocks) are masked out (no memory outside the pool is read).
 * Long contexts are split into partitions that run in parallel (split-K); in the same launch the last
 * partition of a row to finish merges their partial softmax states in partition order. That needs
 * `workspace` of at least ns_decode_workspace_bytes(B, n_kv_heads, head_dim, max_blocks, dtype) bytes
 * (256-byte aligned, zero-filled once by the owner: it starts with the NS_WS_COUNTER_BYTES counter region,
 * which every call leaves at zero; 0 bytes means none is needed). Calls of any shape may share one
 * workspace if they are ordered (same stream), which every caller in the decode loop is. A row's
 * partitions are fixed runs of pages (32 for the whole-row kernel, 16 / 8 for hd 64 / 128 otherwise), so
 * the result depends on the row's context and pages only, not on the table width.
 */
int ns_paged_attn_decode(const void* q, int64_t q_sb, int64_t q_sh,
                         const void* k_pool, const void* v_pool,
                         int64_t kv_sblk, int64_t kv_spos, int64_t kv_sh,
                         const int32_t* block_tables, int64_t bt_sb, const int32_t* context_lens,
                         void* out, int64_t o_sb, int64_t o_sh,
                         int B, int n_heads, int n_kv_heads, int head_dim, int block_size,
                         int max_blocks, int num_blocks, float scale, int dtype,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * ns_paged_attn_decode with entries that share a block table computed together: pairs[b] = 1 when entry b + 1
 * reads the same block table as entry b (any context lengths; pairs[b + 1] is then -1), 0 for an entry on its
 * own. A pair runs as one workgroup row of the whole-row kernel, its two query-head groups side by side in
 * the 16 MFMA columns, so each page is read once for both (speculative verification: the k + 1 rows of a
 * sequence share its table, nanoserve/speculative.py:193-211). Results are bitwise those of
 * ns_paged_attn_decode (a column's arithmetic does not depend on the other columns). Shapes where two
 * groups do not fit in 16 columns, or outside the whole-row kernel, ignore pairs.
 */
int ns_paged_attn_decode_pairs(const void* q, int64_t q_sb, int64_t q_sh,
                               const void* k_pool, const void* v_pool,
                               int64_t kv_sblk, int64_t kv_spos, int64_t kv_sh,
                               const int32_t* block_tables, int64_t bt_sb, const int32_t* context_lens,
                               const int32_t* pairs, void* out, int64_t o_sb, int64_t o_sh,
                               int B, int n_heads, int n_kv_heads, int head_dim, int block_size,
                               int max_blocks, int num_blocks, float scale, int dtype,
                               void* workspace, size_t workspace_bytes, void* stream);

/*
 * ns_paged_attn_decode with the two products on the vector ALUs instead of the matrix cores: same arguments,
 * partitions, loads and merge; per lane fp32 FMAs over its 8 dims of a token and wave64 shuffle sums for the
 * scores (probabilities rounded to bf16 before P.V as in the MFMA kernel). bf16 whole-row shapes only
 * (n_kv * head_dim == 128, or head_dim 128 with several KV heads) with a GQA group of at most 8 (6 for
 * head_dim 128 with several KV heads). No counterpart in the reference: it exists to measure the MFMA design
 * choice against the VALU one on the same kernel (bench.py --attention-ab). Results agree with
 * ns_paged_attn_decode within bf16 tolerances, not bitwise (another summation order).
 */
int ns_paged_attn_decode_valu(const void* q, int64_t q_sb, int64_t q_sh,
                              const void* k_pool, const void* v_pool,
                              int64_t kv_sblk, int64_t kv_spos, int64_t kv_sh,
                              const int32_t* block_tables, int64_t bt_sb, const int32_t* context_lens,
                              void* out, int64_t o_sb, int64_t o_sh,
                              int B, int n_heads, int n_kv_heads, int head_dim, int block_size,
                              int max_blocks, int num_blocks, float scale, int dtype,
                              void* workspace, size_t workspace_bytes, void* stream);

size_t ns_decode_workspace_bytes(int B, int n_kv_heads, int head_dim, int max_blocks, int dtype);

/*
 * ns_paged_attn_decode for decode rows scattered through a step's token rows (a mixed prefill + decode
 * step: the gather q[0][decode_meta.token_idx] and index_copy_ of nanoserve/model.py:274-281): entry b reads its queries from
 * row q_rows[b] of q and writes row q_rows[b] of out (int64, device memory, each a valid row of both), so
 * the rows need no gather before and no scatter after. Everything else as ns_paged_attn_decode (block
 * tables and context lengths per entry, same workspace).
 */
int ns_paged_attn_decode_rows(const void* q, int64_t q_sb, int64_t q_sh,
                              const void* k_pool, const void* v_pool,
                              int64_t kv_sblk, int64_t kv_spos, int64_t kv_sh,
                              const int32_t* block_tables, int64_t bt_sb, const int32_t* context_lens,
                              const int64_t* q_rows, void* out, int64_t o_sb, int64_t o_sh,
                              int B, int n_heads, int n_kv_heads, int head_dim, int block_size,
                              int max_blocks, int num_blocks, float scale, int dtype,
                              void* workspace, size_t workspace_bytes, void* stream);

/*
 * ns_paged_attn_decode without the workspace argument, for callers that cannot allocate device memory
 * (code under hipGraph capture that must not call hipMalloc, tight serving loops, harnesses that forbid
 * allocation). No counterpart in the reference: nanoserve's Triton kernel needs no workspace.
 * The split-K workspace is a fixed array of NS_DECODE_SCRATCH_BYTES in the library's device memory, one
 * per GPU, held until the process ends; its address is looked up on the first call with that GPU current
 * (which also clears it with a kernel on `stream`). This call allocates nothing: a shape whose
 * ns_decode_workspace_bytes exceeds NS_DECODE_SCRATCH_BYTES is rejected with NS_E_INVALID.
 * Every call on one GPU shares that GPU's array: calls that may overlap in time on one GPU (different
 * streams, different threads without ordering) race and give wrong results; calls on one stream are safe.
 * Results are bitwise those of ns_paged_attn_decode with a caller workspace.
 */
#define NS_DECODE_SCRATCH_BYTES (16u << 20)
int ns_paged_attn_decode_noalloc(const void* q, int64_t q_sb, int64_t q_sh,
                                 const void* k_pool, const void* v_pool,
                                 int64_t kv_sblk, int64_t kv_spos, int64_t kv_sh,
                                 const int32_t* block_tables, int64_t bt_sb, const int32_t* context_lens,
                                 void* out, int64_t o_sb, int64_t o_sh,
                                 int B, int n_heads, int n_kv_heads, int head_dim, int block_size,
                                 int max_blocks, int num_blocks, float scale, int dtype, void* stream);

/*
 * Paged chunked-prefill attention: several sequences' new tokens attend to their cached context plus
 * themselves, causally. seq_info (device, int32 [n_seqs, 4]) holds per sequence s:
 *   q_start (first row of s in q / out), n_new (T, its new tokens), ctx_len (tokens cached before this
 *   step), and an unused fourth entry.
 * New token j of s (absolute position ctx_len + j) and query head h (KV head g = h / (n_heads / n_kv_heads))
 *   out[q_start + j, h, :] = softmax(q[q_start + j, h, :] . K[0 : ctx_len + j + 1]^T * scale) . V[...]
 * with token t of s at pool block block_tables[s, t / block_size], position t % block_size; the new tokens'
 * K/V must already be in the pages (rope_qkv writes them). This is the causal-offset mask of
 * nanoserve/model.py:292-309 (continuation) and the causal SDPA of :310-318 (fresh prefill, ctx_len = 0),
 * over the pages PagedKVCache.gather (kv_cache.py:281-288) would gather; the reference computes it with
 * gather + repeat_interleave + SDPA. Online softmax in fp32; probabilities rounded to bf16 before P.V.
 * max_new = max over s of n_new and max_kv = max over s of ctx_len + n_new size the grid (sequences with
 * fewer tokens exit early); a sequence with more new tokens than max_new is not computed.
 *
 * Limits: bf16 only; head_dim in {64, 128}; block_size == 16; strides multiples of 8 elements and
 * 16-byte aligned bases. Pages past ceil((ctx_len + n_new) / 16) are never read and a sequence's page
 * count is clamped to max_blocks; the tokens of a table entry outside [0, num_blocks) are masked out.
 * Rows of out that belong to no sequence are not written.
 * Long contexts split a query tile's keys over several workgroups; in the same launch the last of them
 * merges the partial softmax states in order. That needs `workspace` of at least
 * ns_prefill_workspace_bytes(n_seqs, n_heads, head_dim, max_new, max_kv) bytes (256-byte aligned,
 * zero-filled once by the owner: it starts with the NS_WS_COUNTER_BYTES counter region, which every call
 * leaves at zero; 0 bytes means none is needed). Calls of any shape may share one workspace if they are
 * ordered (same stream).
 */
int ns_paged_attn_prefill(const void* q, int64_t q_st, int64_t q_sh,
                          const void* k_pool, const void* v_pool,
                          int64_t kv_sblk, int64_t kv_spos, int64_t kv_sh,
                          const int32_t* block_tables, int64_t bt_sb, const int32_t* seq_info,
                          int n_seqs, int max_new, int max_kv, void* out, int64_t o_st, int64_t o_sh,
                          int n_heads, int n_kv_heads, int head_dim, int block_size,
                          int max_blocks, int num_blocks, float scale, int dtype,
                          void* workspace, size_t workspace_bytes, void* stream);

size_t ns_prefill_workspace_bytes(int n_seqs, int n_heads, int head_dim, int max_new, int max_kv);

/*
 * A mixed step's attention in one launch: ns_paged_attn_prefill over the chunk rows (pf_block_tables,
 * seq_info, n_seqs, max_new, max_kv, pf_max_blocks, pf_workspace) and ns_paged_attn_decode_rows over the B
 * decode rows (dec_block_tables, context_lens, q_rows, dec_max_blocks, dec_workspace), with the same
 * arguments, limits, workspaces and results as those two calls (both write into out, at disjoint rows).
 * Replaces the per-sequence attention loop of nanoserve/model.py:277-318 for a step holding both decode
 * rows and chunks. When the decode rows take the whole-row kernel, the two kinds of workgroups share one
 * grid, so the decode rows run beside the prefill instead of after it; otherwise the two are launched
 * one after the other on `stream`. n_seqs or B may be 0.
 */
int ns_paged_attn_mixed(const void* q, int64_t q_sb, int64_t q_sh, const void* k_pool, const void* v_pool,
                        int64_t kv_sblk, int64_t kv_spos, int64_t kv_sh, const int32_t* pf_block_tables,
                        int64_t pf_bt_sb, const int32_t* seq_info, int n_seqs, int max_new, int max_kv,
                        int pf_max_blocks, void* pf_workspace, size_t pf_workspace_bytes,
                        const int32_t* dec_block_tables, int64_t dec_bt_sb, const int32_t* context_lens,
                        const int64_t* q_rows, int B, int dec_max_blocks, void* dec_workspace,
                        size_t dec_workspace_bytes, void* out, int64_t o_sb, int64_t o_sh, int n_heads,
                        int n_kv_heads, int head_dim, int block_size, int num_blocks, float scale, int dtype,
                        void* stream);

/*
 * RMSNorm over rows of length n (row-major, contiguous):
 *   if residual != NULL: r = round(residual + x) is stored to res_out and replaces x;
 *   out = round(w * round(x * rsqrt(mean(x^2) + eps)))     (statistics in fp32)
 * round() = to the tensor dtype, where PyTorch's unfused ops round.
 * Replaces nanoserve/kernels/fused.py:45 rms_norm (kernel :26-42).
 */
int ns_rms_norm(const void* x, const void* residual, const void* weight, void* out, void* res_out,
                int64_t rows, int n, float eps, int dtype, void* stream);

/*
 * SwiGLU activation on the merged gate/up projection: x = [rows, 2n] holding [gate | up],
 *   out[r, c] = round(round(silu(gate[r, c])) * up[r, c]),  silu(g) = g / (1 + exp(-g)) in fp32.
 * Replaces nanoserve/kernels/fused.py:75 silu_mul (kernel :63-72).
 */
int ns_silu_mul(const void* x, void* out, int64_t rows, int n, int dtype, void* stream);

/*
 * RoPE on the merged QKV projection + paged KV write, one token per row of qkv
 * [n_tok, (n_heads + 2 n_kv) head_dim]:
 *   q/k heads: out_lo = r(r(x_lo c_lo) - r(x_hi s_lo)), out_hi = r(r(x_hi c_hi) + r(x_lo s_hi))
 *   (r = round to bf16, ties to even, for bf16; identity for fp32; no fused multiply-add),
 *   v heads copied. q -> [n_tok, n_heads, hd], k, v -> [n_tok, n_kv, hd].
 *   If k_cache != NULL: k and v of token t are also stored at flat pool position slots[t]
 *   (pool viewed as [num_blocks * block_size, n_kv, hd]). cos/sin: [n_tok, hd] in the same dtype.
 * Replaces nanoserve/kernels/fused.py:156 rope_qkv (kernel :107-153, rounding :87-104).
 */
int ns_rope_qkv(const void* qkv, const void* cos, const void* sin, void* q, void* k, void* v,
                void* k_cache, void* v_cache, const int64_t* slots,
                int64_t n_tok, int n_heads, int n_kv_heads, int head_dim, int dtype, void* stream);

/*
 * The first ops of a forward step in one launch: x[i] = embed[token_ids[i]] ([vocab, hidden], row-major;
 * an id outside [0, vocab) gives a zero row) and the RoPE tables cos/sin[i] = cat(f, f).cos() / .sin()
 * rounded to the dtype, f = float(positions[i]) * inv_freq (fp32 [head_dim / 2]); x_out [n_tokens, hidden],
 * cos/sin [n_tokens, head_dim]. row_sumsq (fp32 [ceil(hidden / 16)][NS_NORM_ROWS], may be NULL; n_tokens <=
 * NS_NORM_ROWS then)
 * receives the first RMSNorm's statistics in the layout ns_gemm_residual_norm_stats writes, so the first
 * projection can normalise on load. hidden a multiple of 16.
 * Replaces F.embedding (nanoserve/model.py:341) and Qwen2Model.rope (model.py:212-217).
 */
int ns_embed_rope(const int64_t* token_ids, const int64_t* positions, int64_t n_tokens, const void* embed,
                  int64_t vocab, int hidden, const float* inv_freq, int head_dim, void* x_out, void* cos_out,
                  void* sin_out, float* row_sumsq, int dtype, void* stream);

/*
 * dst[i] = src[rows[i]] for i < n_rows: rows of row_bytes bytes (a multiple of 16), src rows src_stride_bytes
 * apart (n_src of them), dst rows dst_stride_bytes apart; a row index outside [0, n_src) gives a zero row.
 * Replaces the LM head's row selection x[:, logits, :] / the last row of each sequence
 * (nanoserve/model.py:353-356).
 */
int ns_gather_rows(const void* src, int64_t src_stride_bytes, int64_t n_src, const int64_t* rows, int64_t n_rows,
                   int64_t row_bytes, void* dst, int64_t dst_stride_bytes, void* stream);

/*
 * GEMMs of the decode loop (bf16, K a multiple of 32; skinny kernels for 1 <= M <= 64, and for ns_gemm and
 * ns_gemm_silu_mul a tiled kernel above that; W row-major [N, K], x [M, K],
 * outputs row-major, every pointer 16-byte aligned). They replace the F.linear calls of
 * nanoserve/model.py:231,256-257,362 for decode-sized batches: y = x W^T (+ bias) with fp32 accumulation
 * and one rounding to bf16, like F.linear; each fused variant rounds where the unfused ops it replaces
 * round. One launch per call: the weight tiles are shared out evenly over the GPU, and a tile that two
 * workgroups share is summed by the later of them in a fixed order, so results are deterministic.
 * Every entry point needs `workspace`: at least ns_gemm_workspace_bytes(M, N, K) bytes, 256-byte
 * aligned, ZERO-FILLED once before its first use. Each call leaves its counters at zero again, so the
 * buffer can be reused by any later call on the same stream without clearing (calls that share a
 * workspace must not overlap in time).
 */
size_t ns_gemm_workspace_bytes(int M, int N, int K);

/*
 * Normalised inputs. The projections that follow an RMSNorm in the model (QKV after ln1, gate/up after
 * ln2, the LM head after the final norm) take the un-normalised r = residual + ... and normalise each
 * activation fragment as they load it: h = round(w * round(r * inv)), inv = rsqrt(sum / K + eps), where
 * sum adds the per-16-column row sums of r^2 that ns_gemm_residual_norm_stats wrote (x_sumsq, fp32
 * [ceil(K/16)][NS_NORM_ROWS], row m at column m) in one fixed order. So the RMSNorm never runs as a separate pass,
 * and every consumer sees bitwise the same h; ns_rms_norm_apply materialises h where a tensor is needed.
 * x_sumsq == NULL: x is used as is (x_norm_w, x_eps ignored).
 */

/*
 * y = round(x W^T + bias); bias may be NULL.
 * Any M >= 1: above 64 rows (prefill chunks, mixed steps, speculative verify batches; nanoserve/model.py:231,
 * 256-257 on the large-token path) x_sumsq must be NULL (materialise a normalised input with
 * ns_rms_norm_apply first). Up to 192 rows a projection with K <= 2048 and at most 8,192 rows of W runs on the
 * tile-16 kernel in 16-token blocks; otherwise a tiled MFMA kernel computes the product (128 x 128 or
 * 256 x 256 output tiles, K sliced and the slices summed in a fixed order for long K and few tiles), its
 * workspace sized by ns_gemm_workspace_bytes(M, N, K) as for the skinny kernels.
 */
int ns_gemm(const void* x, const void* w, const void* bias, void* y, int M, int N, int K, int dtype,
            const float* x_sumsq, const void* x_norm_w, float x_eps,
            void* workspace, size_t workspace_bytes, void* stream);

/*
 * LM head of a decode step with the greedy choice fused: y = round(x W^T) exactly as ns_gemm (no bias), and
 * tokens[m] = ns_argmax_rows' result on row m of the stored y (first maximal index, NaN above every
 * number), in one launch. Replaces F.linear(x, self.lm_head) (nanoserve/model.py:362) followed by
 * logits.argmax(-1) (nanoserve/engine.py:239). Applies where ns_gemm_argmax_fused(M, N, K) returns 1 (at most
 * 32 rows, K <= 2048, at least four 64-row weight tiles per CU: the persistent LM-head kernel); elsewhere
 * call ns_gemm and ns_argmax_rows. argmax_workspace: the ns_argmax_rows workspace (zero-filled once,
 * 256-byte aligned, at least NS_WS_COUNTER_BYTES bytes); the last 1 KB of its counter region holds this
 * launch's arrival counter and per-row keys, which every launch leaves at zero. tokens may be pinned host
 * memory.
 */
int ns_gemm_argmax_fused(int M, int N, int K);
int ns_gemm_argmax(const void* x, const void* w, void* y, int M, int N, int K, int dtype,
                   const float* x_sumsq, const void* x_norm_w, float x_eps, int64_t* tokens,
                   void* argmax_workspace, size_t argmax_workspace_bytes, void* stream);

/*
 * Merged gate/up projection + SwiGLU: w_gate_up = [gate; up] ([N2, K], N2 = 2 * intermediate);
 * out[M, N2/2] = round(round(silu(round(x Wg^T))) * round(x Wu^T)).
 * Replaces silu_mul(F.linear(h, gate_up_w)) (nanoserve/model.py:257, fused.py:75).
 * Workspace: ns_gemm_workspace_bytes(M, N2, K). Any M >= 1 (above 64 rows: the tiled kernel, as ns_gemm).
 */
int ns_gemm_silu_mul(const void* x, const void* w_gate_up, void* out, int M, int N2, int K, int dtype,
                     const float* x_sumsq, const void* x_norm_w, float x_eps,
                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * Projection + residual add + the statistics of the RMSNorm that follows: o = round(x W^T);
 * res_out = round(residual + o); row_sumsq[p][m] = sum over columns 16p .. 16p+15 of res_out[m]^2 (fp32,
 * [ceil(N/16)][NS_NORM_ROWS], may be NULL). N a multiple of 8. M <= NS_NORM_ROWS, or any M above 192 with
 * row_sumsq NULL (the tiled kernel's residual epilogue: prefill chunks and mixed steps, whose RMSNorm then
 * runs as ns_rms_norm on res_out).
 * With a normalised consumer (or ns_rms_norm_apply) this replaces rms_norm(F.linear(o, o_w), ln2, eps,
 * residual=x) (nanoserve/model.py:256, fused.py:45) and x + F.linear(a, down_w) followed by the next
 * layer's rms_norm (model.py:257, :227-231).
 */
int ns_gemm_residual_norm_stats(const void* x, const void* w, const void* residual, void* res_out,
                                float* row_sumsq, int M, int N, int K, int dtype,
                                void* workspace, size_t workspace_bytes, void* stream);

/*
 * h = round(norm_w * round(r * rsqrt(sum / n + eps))) with sum from row_sumsq exactly as the GEMMs
 * compute it on load (rows <= 64, n a multiple of 8). Completes nanoserve/kernels/fused.py:45 rms_norm
 * for rows whose statistics came from ns_gemm_residual_norm_stats.
 */
int ns_rms_norm_apply(const void* r, const float* row_sumsq, const void* norm_w, float eps, void* h,
                      int64_t rows, int n, int dtype, void* stream);

/*
 * Merged QKV projection + bias + RoPE + paged KV write: qkv = round(x W^T + bias), then the
 * ns_rope_qkv contract on it (q, k, v outputs; k/v stored at slots when k_cache is given).
 * head_dim 64 or 128. Replaces rope_qkv(F.linear(h, qkv_w, qkv_b), ...) (nanoserve/model.py:231-234).
 */
/* 1 when ns_gemm_rope_qkv takes M rows (normed: a normalised input): any M <= 64; above that any plain input
 * (up to 192 rows with K <= 2048 the tile-16 kernel token-split: speculative verify batches; otherwise the tiled
 * kernel, whose epilogue rotates whole heads of its output tile: prefill chunks and mixed steps), and a
 * normalised one with K <= 2048 up to NS_NORM_ROWS rows. No counterpart in the reference; it tells the caller
 * when to run the GEMM and ns_rope_qkv separately instead. */
int ns_gemm_rope_qkv_fits(int M, int K, int n_heads, int n_kv_heads, int head_dim, int normed);
int ns_gemm_rope_qkv(const void* x, const void* w, const void* bias, const void* cos, const void* sin,
                     void* q, void* k, void* v, void* k_cache, void* v_cache, const int64_t* slots, int M,
                     int K, int n_heads, int n_kv_heads, int head_dim, int dtype,
                     const float* x_sumsq, const void* x_norm_w, float x_eps,
                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * Fragment-packed weights for decode-sized products (M <= 64). The reference has no counterpart for the
 * layout itself (its projections are cuBLAS calls on row-major weights); the products below replace the same
 * F.linear calls as their row-major twins above (nanoserve/model.py:231,256-257,362), with the same epilogues
 * and rounding points, and exist because the layout streams from HBM much faster.
 * Layout: W [N, K] row-major taken in 16-row tiles (order 0: rows 16t .. 16t+15; order 1, a merged
 * [gate; up] weight of N = 2I rows: gate rows 8t .. 8t+7 then the matching up rows; order 2, a merged QKV
 * weight of head_dim-wide heads: dims 8f .. 8f+7 of a head then the dims head_dim/2 further), rows past the
 * end clamped to the last one; block (t, s) = 1 KB holds, for lane l = 0..63, the 8 bf16
 * W[row(t, l % 16)][32 s + 8 (l / 16) .. +7], blocks in (tile, k-step) order. K a multiple of 32.
 * ns_packed_weight_bytes gives the size (0 for a shape that cannot be packed); ns_pack_weight writes it
 * (one launch, 16-byte aligned pointers).
 * Workspaces: ns_gemm_packed_workspace_bytes(M, N, K, order, head_dim) bytes, 256-byte aligned, zero-filled
 * once, as for the row-major kernels (long-K and few-tile shapes split K over workgroups and merge in the
 * same launch; every call leaves the counters at zero). Results are deterministic.
 */
size_t ns_packed_weight_bytes(int N, int K, int order, int head_dim);
int ns_pack_weight(const void* w, void* packed, int N, int K, int order, int head_dim, void* stream);
size_t ns_gemm_packed_workspace_bytes(int M, int N, int K, int order, int head_dim);
/* 1 when the packed plan for this shape splits K over workgroups (K > 2048), whose merge in the same launch
 * costs three dependent cross-XCD round trips: the row-major kernels are the faster choice there. */
int ns_gemm_packed_sliced(int M, int N, int K, int order, int head_dim);
/* As ns_gemm on a packed weight of order 0 (N a multiple of 8, bias NULL or 16-byte aligned). */
int ns_gemm_packed(const void* x, const void* w_packed, const void* bias, void* y, int M, int N, int K, int dtype,
                   const float* x_sumsq, const void* x_norm_w, float x_eps,
                   void* workspace, size_t workspace_bytes, void* stream);
/* As ns_gemm_argmax on a packed weight of order 0, where ns_gemm_argmax_packed_fits(M, N, K) is 1 (K unsplit,
 * N a multiple of 8); workspace = the argmax workspace (ns_argmax_workspace_bytes), as for ns_gemm_argmax. */
int ns_gemm_argmax_packed_fits(int M, int N, int K);
int ns_gemm_argmax_packed(const void* x, const void* w_packed, void* y, int M, int N, int K, int dtype,
                          const float* x_sumsq, const void* x_norm_w, float x_eps, int64_t* tokens,
                          void* workspace, size_t workspace_bytes, void* stream);
/* As ns_gemm_silu_mul on a packed weight of order 1. */
int ns_gemm_silu_mul_packed(const void* x, const void* w_packed, void* out, int M, int N2, int K, int dtype,
                            const float* x_sumsq, const void* x_norm_w, float x_eps,
                            void* workspace, size_t workspace_bytes, void* stream);
/* As ns_gemm_residual_norm_stats on a packed weight of order 0 (N a multiple of 8). */
int ns_gemm_residual_norm_stats_packed(const void* x, const void* w_packed, const void* residual, void* res_out,
                                       float* row_sumsq, int M, int N, int K, int dtype,
                                       void* workspace, size_t workspace_bytes, void* stream);
/* As ns_gemm_rope_qkv on a packed weight of order 2 (head_dim 64 or 128, 16-byte aligned operands). */
int ns_gemm_rope_qkv_packed(const void* x, const void* w_packed, const void* bias, const void* cos, const void* sin,
                            void* q, void* k, void* v, void* k_cache, void* v_cache, const int64_t* slots, int M,
                            int K, int n_heads, int n_kv_heads, int head_dim, int dtype,
                            const float* x_sumsq, const void* x_norm_w, float x_eps,
                            void* workspace, size_t workspace_bytes, void* stream);

/*
 * Greedy selection: out[r] = index of the first maximal element of row r of x (rows x n, row stride
 * ld elements); NaN ranks above every number (torch.argmax semantics). int64 output.
 * Replaces logits.argmax(-1) of nanoserve/engine.py:239 / sampling.py:59-60.
 * workspace (optional, zero-initialised once by the caller, 256-byte aligned, at least
 * ns_argmax_workspace_bytes(rows, n) bytes, which is 0 above 65,280 rows): rows are split over several
 * workgroups merged in the same launch; every call leaves the counter region at zero, so calls with any row
 * count may share one workspace. NULL: one workgroup per row.
 */
size_t ns_argmax_workspace_bytes(int64_t rows, int n);
int ns_argmax_rows(const void* x, int64_t ld, int64_t rows, int n, int dtype, int64_t* out, void* workspace,
                   size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NANOSERVE_HIP_H */
