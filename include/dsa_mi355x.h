/*
 * C ABI of the MI355X (gfx950) DeepSeek Sparse Attention kernels:
 * lightning indexer -> top-k selector -> sparse MLA forward.
 *
 * Conventions (all entry points):
 *  - Plain device pointers and sizes; tensors are dense row-major (C order).
 *  - The library never allocates device memory.  Outputs and workspaces are
 *    allocated by the caller (the Python layer uses torch's caching allocator);
 *    workspace sizes come from the *_workspace_size queries.
 *  - `stream` is a hipStream_t passed as void* (NULL = the legacy default stream).
 *    Work is enqueued asynchronously; the call returns once it is launched.
 *  - Return value: 0 on success, otherwise a hipError_t code
 *    (hipErrorInvalidValue = 1 for rejected arguments; dsa_last_error_message()
 *    names the offending argument).  The reference's generated entry returns
 *    void (src/target/codegen_ascend.cc:1138-1225); errors are reported here
 *    instead of being dropped.
 *  - Kernels are stateless and reentrant; concurrent calls on different
 *    streams are safe (except dsa_sparse_mla_fwd_noalloc, whose calls on one
 *    GPU share a scratch array).
 */
#ifndef DSA_MI355X_H_
#define DSA_MI355X_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element kinds for the indexer's q/k. */
#define DSA_KIND_FP8_E4M3 0 /* OCP float8 e4m3fn (torch.float8_e4m3fn) */
#define DSA_KIND_BF16 1
#define DSA_KIND_FP16 2
#define DSA_KIND_FP32 3 /* act_quant input */
#define DSA_KIND_INT8 4 /* act_quant output */

/* Library ABI version (major * 100 + minor). */
int dsa_abi_version(void);

/* Human-readable description of the last argument error on this thread. */
const char* dsa_last_error_message(void);

/*
 * Row-wise top-k selector.
 * Replaces the compiled `simple_topk_selector` kernel's `call()` entry
 * (examples/topk_selector/example_topk_selector.py:10-54, entry emitted by
 * src/target/codegen_ascend.cc:1138-1225) and the top-k stage of the
 * lightning indexer (examples/deepseek_v4/lightning_indexer.py:945-1033).
 *
 *  x        [rows, ld] fp32, the first n columns of each row are scored
 *  row_len  [rows] int32 or NULL: columns >= row_len[r] are excluded
 *  out_idx  [rows, k] int32; out_val [rows, k] fp32 or NULL
 *  sorted   1: (value desc, index asc); 0: a fixed data-determined order
 * Ties go to the lower index; scores <= -1e30, -inf and NaN never take a slot;
 * unfilled slots hold -1 (value -inf).  1 <= k <= 8192, n < 2^31.
 */
int dsa_topk_select(const float* x, int64_t ld, int64_t rows, int64_t n, int64_t k, const int32_t* row_len,
                    int sorted, int32_t* out_idx, float* out_val, void* stream);

/* Workspace bytes dsa_topk_select_ws needs (0: rows short enough for one pass). */
size_t dsa_topk_select_workspace_size(int64_t rows, int64_t n, int64_t k);

/*
 * dsa_topk_select with a caller-provided workspace, for rows longer than
 * 32768 scores (the 128K-context indexer rows): the rows are selected in
 * segments, then over the segments' candidates, instead of by repeated radix
 * passes over the whole row.  Same reference interface and results as
 * dsa_topk_select; the workspace plays the role of the reference kernels'
 * workspace buffers (tilelang/jit/__init__.py:212-255, workspace_idx).
 */
int dsa_topk_select_ws(const float* x, int64_t ld, int64_t rows, int64_t n, int64_t k, const int32_t* row_len,
                       int sorted, int32_t* out_idx, float* out_val, void* workspace, size_t workspace_bytes,
                       void* stream);

/*
 * Lightning-indexer logits (fp32, masked positions = -inf).
 * Replaces the QK/ReLU/weighted-head-sum stage of `make_lightning_indexer_kernel`
 * (examples/deepseek_v4/lightning_indexer.py:338-1197, stages :756-763 and
 * :868-937) and of `indexer` (examples/lightning_indexer/example_lightning_indexer.py:19-125).
 *
 *  q        [B, S1, H, D] of `kind`, D in {64, 128}
 *  k        [B, S2, D] of `kind`, or with block_table a paged pool
 *           [num_blocks, block_size, D]
 *  k_scale  per-key fp32 scale ([B, S2] or [num_blocks, block_size]) or NULL
 *  weights  [B, S1, H] fp32
 *  actual_q_len / actual_k_len [B] int32 or NULL (= S1 / S2)
 *  block_table [B, max_blocks] int32 or NULL
 *  sparse_mode 0 (no mask) or 3 (causal, bottom-right aligned)
 *  logits   [B, S1, ld] fp32, ld >= S2
 * 1 <= H <= 64 (the reference's N1 <= 64, lightning_indexer.py:1282-1283).
 */
int dsa_indexer_logits(int kind, const void* q, const void* k, const float* k_scale, const float* weights,
                       int64_t B, int64_t S1, int64_t S2, int64_t H, int64_t D, const int32_t* actual_q_len,
                       const int32_t* actual_k_len, const int32_t* block_table, int64_t block_size,
                       int64_t max_blocks, int sparse_mode, float* logits, int64_t ld, void* stream);

/* Workspace bytes dsa_lightning_indexer needs: the fp32 logits of all rows,
 * plus the top-k candidate buffer when S2 > 32768. */
size_t dsa_lightning_indexer_workspace_size(int64_t B, int64_t S1, int64_t S2, int64_t sparse_count);

/*
 * Lightning indexer: logits then top-`sparse_count` per query row.
 * Replaces the `lightning_indexer` wrapper's kernel call
 * (examples/deepseek_v4/lightning_indexer.py:1202-1370, BSND / PA_BSND keys).
 *  out_idx [B, S1, sparse_count] int32 (the reference's [B, S1, 1, K])
 *  out_val [B, S1, sparse_count] fp32 or NULL
 * The selection is sorted by (score desc, index asc), -1 padded.
 */
int dsa_lightning_indexer(int kind, const void* q, const void* k, const float* k_scale, const float* weights,
                          int64_t B, int64_t S1, int64_t S2, int64_t H, int64_t D, const int32_t* actual_q_len,
                          const int32_t* actual_k_len, const int32_t* block_table, int64_t block_size,
                          int64_t max_blocks, int sparse_mode, int64_t sparse_count, int32_t* out_idx,
                          float* out_val, void* workspace, size_t workspace_bytes, void* stream);

/* 1 when dsa_lightning_indexer_fused streams the top-k for this shape (else it
 * runs dsa_lightning_indexer). */
int dsa_lightning_indexer_fused_applies(int64_t B, int64_t S1, int64_t S2, int64_t sparse_count);

/* Workspace bytes dsa_lightning_indexer_fused needs (at least those of
 * dsa_lightning_indexer). */
size_t dsa_lightning_indexer_fused_workspace_size(int64_t B, int64_t S1, int64_t S2, int64_t sparse_count);

/*
 * dsa_lightning_indexer with the top-k streamed out of the indexer: same
 * arguments and the same output bit for bit, without writing the logits of
 * every row.  Replaces the same wrapper call as dsa_lightning_indexer; the
 * fused sort + merge design of the reference's kernel
 * (examples/deepseek_v4/lightning_indexer.py:945-1033) is what it stands for.
 * A sample of each row's logits sets a threshold, the indexer keeps only the
 * keys that reach it, and the top-k runs over those; rows whose threshold turns
 * out too high take the dense path.  Applies when S2 >= max(16384, 8 *
 * sparse_count) and sparse_count <= 4096; otherwise this call runs
 * dsa_lightning_indexer.
 */
int dsa_lightning_indexer_fused(int kind, const void* q, const void* k, const float* k_scale, const float* weights,
                                int64_t B, int64_t S1, int64_t S2, int64_t H, int64_t D, const int32_t* actual_q_len,
                                const int32_t* actual_k_len, const int32_t* block_table, int64_t block_size,
                                int64_t max_blocks, int sparse_mode, int64_t sparse_count, int32_t* out_idx,
                                float* out_val, void* workspace, size_t workspace_bytes, void* stream);

/* Diagnostic for the fused path: after a dsa_lightning_indexer_fused call on
 * `workspace` (same shape), writes to device int *count the number of rows that
 * went back to dense logits because their sampled threshold was too high or a key
 * chunk overflowed its candidate slot (rows the register top-k handed to the
 * exact kernel are not counted).  No counterpart in the reference. */
int dsa_lightning_indexer_fused_fallback_rows(const void* workspace, int64_t B, int64_t S1, int64_t S2,
                                              int64_t sparse_count, int32_t* count, void* stream);

/*
 * Packed (TND) query rows.  The reference converts TND to padded BSND on the
 * host and back (examples/deepseek_v4/lightning_indexer.py:48-190 helpers,
 * used at :1257-1268 and :1363-1368); here the kernels address the packed rows
 * directly.  Batch b owns query rows cu_q[b-1] .. cu_q[b]-1 (cu_q[-1] = 0):
 *  q        [T, H, D], weights [T, H] fp32, T = cu_q[B-1]
 *  cu_q     [B] int32 inclusive prefix sums of the query lengths
 *           (actual_seq_lengths_query of layout "TND")
 *  keys, either packed (cu_k != NULL, layout "TND"):
 *           k [Tk, D], k_scale [Tk] or NULL, cu_k [B] prefix sums
 *  or paged (block_table != NULL, layout "PA_BSND"):
 *           k [num_blocks, block_size, D], actual_k_len [B] per-batch lengths
 *  S1_max   >= every query length; S2_max >= every key length (grid bounds)
 *  logits   [T, ld] fp32, ld >= S2_max
 * The logits of a row are those of its (b, t) row in the padded layout.
 */
int dsa_indexer_logits_tnd(int kind, const void* q, const void* k, const float* k_scale, const float* weights,
                           int64_t B, int64_t T, int64_t S1_max, int64_t S2_max, int64_t H, int64_t D,
                           const int32_t* cu_q, const int32_t* cu_k, const int32_t* actual_k_len,
                           const int32_t* block_table, int64_t block_size, int64_t max_blocks, int sparse_mode,
                           float* logits, int64_t ld, void* stream);

/* Workspace bytes dsa_lightning_indexer_tnd needs for T packed query rows. */
size_t dsa_lightning_indexer_tnd_workspace_size(int64_t T, int64_t S2_max, int64_t sparse_count);

/*
 * Lightning indexer over packed (TND) query rows: the `lightning_indexer`
 * wrapper with layout_query "TND" (examples/deepseek_v4/lightning_indexer.py:1202-1370),
 * arguments as dsa_indexer_logits_tnd.
 *  out_idx [T, sparse_count] int32 (the reference's [T, 1, K])
 *  out_val [T, sparse_count] fp32 or NULL
 * With S2_max == 0 nothing is launched and the outputs are left to the caller
 * (the reference fills -1 / -inf on that early exit, :1287-1294).
 */
int dsa_lightning_indexer_tnd(int kind, const void* q, const void* k, const float* k_scale, const float* weights,
                              int64_t B, int64_t T, int64_t S1_max, int64_t S2_max, int64_t H, int64_t D,
                              const int32_t* cu_q, const int32_t* cu_k, const int32_t* actual_k_len,
                              const int32_t* block_table, int64_t block_size, int64_t max_blocks, int sparse_mode,
                              int64_t sparse_count, int32_t* out_idx, float* out_val, void* workspace,
                              size_t workspace_bytes, void* stream);

/* Workspace bytes dsa_lightning_indexer_tnd_fused needs (at least those of
 * dsa_lightning_indexer_tnd). */
size_t dsa_lightning_indexer_tnd_fused_workspace_size(int64_t B, int64_t T, int64_t S1_max, int64_t S2_max,
                                                      int64_t sparse_count);

/*
 * dsa_lightning_indexer_tnd with the top-k streamed out of the indexer, as
 * dsa_lightning_indexer_fused does for padded rows: same arguments, same output
 * bit for bit.  Replaces the same wrapper call (TND queries,
 * examples/deepseek_v4/lightning_indexer.py:1202-1370).  Applies under the
 * conditions of dsa_lightning_indexer_fused (S2_max in place of S2); otherwise
 * runs dsa_lightning_indexer_tnd.
 */
int dsa_lightning_indexer_tnd_fused(int kind, const void* q, const void* k, const float* k_scale,
                                    const float* weights, int64_t B, int64_t T, int64_t S1_max, int64_t S2_max,
                                    int64_t H, int64_t D, const int32_t* cu_q, const int32_t* cu_k,
                                    const int32_t* actual_k_len, const int32_t* block_table, int64_t block_size,
                                    int64_t max_blocks, int sparse_mode, int64_t sparse_count, int32_t* out_idx,
                                    float* out_val, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes dsa_sparse_mla_fwd needs (0 when no split of the index list is used). */
size_t dsa_sparse_mla_workspace_size(int64_t B, int64_t S, int64_t H, int64_t topk);

/*
 * Sparse MLA forward with LSE.
 * Replaces `sparse_attention_fwd` (examples/sparse_flash_attention/example_sparse_flash_attn.py:18-243,
 * paged variant example_sparse_flash_attn_mask_pa.py:13-333) and adds the LSE output
 * of `sparse_flash_mla(..., return_softmax_lse=True)`
 * (examples/deepseek_v4/sparse_flash_mla/sparse_flash_mla_api.py:94-253).
 *
 *  kind     DSA_KIND_BF16 or DSA_KIND_FP16 (q, kv and out share it)
 *  q        [B, S, H, d_qk]
 *  kv       [B, Skv, d_qk], or with block_table a paged pool
 *           [num_blocks, block_size, d_qk]; V = kv[..., :d_v]
 *  indices  [B, S, topk] int32, -1 = empty slot
 *  block_table [B, max_blocks] int32 or NULL
 *  actual_q_len / actual_kv_len [B] int32 or NULL (= S / Skv or max_blocks*block_size)
 *  out      [B, S, H, d_v] of `kind`;  lse [B, S, H] fp32 (natural log)
 * d_qk == 576, d_v == 512, H % 16 == 0, indices unique per row.
 */
int dsa_sparse_mla_fwd(int kind, const void* q, const void* kv, const int32_t* indices, const int32_t* block_table,
                       const int32_t* actual_q_len, const int32_t* actual_kv_len, int64_t B, int64_t S,
                       int64_t H, int64_t d_qk, int64_t d_v, int64_t Skv, int64_t block_size, int64_t max_blocks,
                       int64_t topk, float sm_scale, int is_causal, void* out, float* lse, void* workspace,
                       size_t workspace_bytes, void* stream);

/*
 * dsa_sparse_mla_fwd without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.
 * Same arguments (minus the workspace), kernels and results as
 * dsa_sparse_mla_fwd; the split partials of decode-shaped calls go to a
 * library-owned scratch array of dsa_sparse_mla_noalloc_max_workspace() bytes
 * (64 MiB) per GPU, held from the library's first use on that GPU until the
 * process ends.  A shape whose dsa_sparse_mla_workspace_size() exceeds it is
 * rejected (hipErrorInvalidValue).  The call allocates nothing.  Calls that
 * overlap on one GPU (concurrent streams, or host threads) share that array
 * and race: serialise them.  The first call on a GPU looks the array's address
 * up (once); it may run inside HIP-graph capture once any entry of this
 * library has run eagerly on that GPU (the usual graph warm-up).
 */
size_t dsa_sparse_mla_noalloc_max_workspace(void);

int dsa_sparse_mla_fwd_noalloc(int kind, const void* q, const void* kv, const int32_t* indices,
                               const int32_t* block_table, const int32_t* actual_q_len, const int32_t* actual_kv_len,
                               int64_t B, int64_t S, int64_t H, int64_t d_qk, int64_t d_v, int64_t Skv,
                               int64_t block_size, int64_t max_blocks, int64_t topk, float sm_scale, int is_causal,
                               void* out, float* lse, void* stream);

/* Workspace bytes dsa_sparse_attention_fwd needs (0 for d_qk 128, and when no split is used). */
size_t dsa_sparse_attention_workspace_size(int64_t B, int64_t S, int64_t H, int64_t kv_group, int64_t d_qk,
                                           int64_t topk);

/*
 * Sparse attention over kv_group KV heads, with LSE.
 * Replaces the `sparse_attention_fwd` builders with their `kv_group` argument
 * (examples/sparse_flash_attention/example_sparse_flash_attn.py:19-29, kv
 * [B, Skv, kv_group, dim + tail_dim], indices [B, S, kv_group, topk]; paged:
 * example_sparse_flash_attn_mask_pa.py:14-46) and the grouped 128-wide kernel of
 * examples/sparse_flash_attention/example_sparse_flash_attn_gqa.py:13-238.
 * Query heads g * Hg .. (g + 1) * Hg - 1 (Hg = H / kv_group) read KV head g
 * through indices[b, s, g, :] (the goldens' q.view(b, s, g, Hg, d)).
 *
 *  q        [B, S, H, d_qk]
 *  kv       [B, Skv, kv_group, d_qk], or (d_qk 576 only) with block_table a
 *           paged pool [num_blocks, block_size, kv_group, d_qk]; V = kv[..., :d_v]
 *  indices  [B, S, kv_group, topk] int32, -1 = empty slot
 *  out      [B, S, H, d_v] of `kind`;  lse [B, S, H] fp32 (natural log)
 * (d_qk, d_v) = (576, 512): Hg a multiple of 16 (the 576-wide kernels of
 * dsa_sparse_mla_fwd); (128, 128): any Hg <= 1024, topk <= 8192, no block
 * table.  Slot validity, causality and lengths as dsa_sparse_mla_fwd.
 */
int dsa_sparse_attention_fwd(int kind, const void* q, const void* kv, const int32_t* indices,
                             const int32_t* block_table, const int32_t* actual_q_len, const int32_t* actual_kv_len,
                             int64_t B, int64_t S, int64_t H, int64_t kv_group, int64_t d_qk, int64_t d_v, int64_t Skv,
                             int64_t block_size, int64_t max_blocks, int64_t topk, float sm_scale, int is_causal,
                             void* out, float* lse, void* workspace, size_t workspace_bytes, void* stream);

/*
 * DeepSeek V4 sparse flash MLA (D = 512, K = V, paged caches, attention sinks).
 * Replaces `sparse_flash_mla(...)` (examples/deepseek_v4/sparse_flash_mla/
 * sparse_flash_mla_api.py:94-253; semantics of sparse_flash_mla_golden.py:55-160).
 * Query row t of batch b (q_start[b] <= t < q_start[b] + q_len[b]; rows past a
 * batch's length are padding: out = 0, lse = 0) at position
 * s_global = seqused_kv[b] - q_len[b] + (t - q_start[b]) attends to
 *  - the original rows s_global - ori_win_left .. s_global (clipped at 0),
 *  - with cmp_kv and no cmp_sparse_indices ("hca"): compressed rows
 *    0 .. floor((s_global + 1) / cmp_ratio) - 1, at most max_cmp of them,
 *  - with cmp_sparse_indices [T, topk_cmp] ("csa"): the selected compressed
 *    rows among the list's first min(topk_cmp, threshold) entries, up to the
 *    first -1, skipping entries >= threshold,
 * and the sink of each head adds exp(sinks[h]) to the softmax denominator.
 *  q [T, H, 512]; caches [block_num, block_size, 512] with tables
 *  [B, table_len] int32; q_start / q_len / seqused_kv [B] int32 (q_start
 *  non-decreasing); sinks [H] fp32 (natural-log units) or NULL;
 *  out [T, H, 512]; lse [T, H] fp32 (natural log, sink included).
 * H % 16 == 0, H <= 1024 (the reference: H = 64); bf16 or fp16.
 * cmp_slots of the workspace query: 0 (window only), max_cmp ("hca") or
 * topk_cmp ("csa").
 */
size_t dsa_sparse_flash_mla_workspace_size(int64_t T, int64_t H, int64_t ori_win_left, int64_t cmp_slots);

int dsa_sparse_flash_mla(int kind, const void* q, int64_t T, int64_t H, int64_t D, int64_t B, const int32_t* q_start,
                         const int32_t* q_len, const int32_t* seqused_kv, const void* ori_kv, int64_t ori_block_num,
                         int64_t ori_block_size, const int32_t* ori_block_table, int64_t ori_table_len,
                         const void* cmp_kv, int64_t cmp_block_num, int64_t cmp_block_size,
                         const int32_t* cmp_block_table, int64_t cmp_table_len, const int32_t* cmp_sparse_indices,
                         int64_t topk_cmp, int64_t cmp_ratio, int64_t ori_win_left, int64_t max_cmp,
                         const float* sinks, float softmax_scale, void* out, float* lse, void* workspace,
                         size_t workspace_bytes, void* stream);

/*
 * V4 gathered-index attention with sinks: `sparse_attn_kernel(h, d, scale)` /
 * `sparse_attn` (examples/deepseek_v4/sparse_attention.py:28-198).  Query row
 * (b, m) attends to kv[b, topk_idxs[b, m, j]] (-1 = empty slot; duplicates
 * count twice, as in the golden), K = V = the 512-wide row, and the sink of
 * head h adds exp(sinks[h]) to the softmax denominator.
 *  q [B, M, H, 512]; kv [B, N, 512]; topk_idxs [B, M, topk] int32;
 *  sinks [H] fp32 or NULL; out [B, M, H, 512] fp32 (the fp32 accumulator, as the
 *  reference kernel writes it: sparse_attention.py:56); lse [B, M, H] fp32.
 */
size_t dsa_sparse_attn_sink_workspace_size(int64_t B, int64_t M, int64_t H, int64_t topk);

int dsa_sparse_attn_sink(int kind, const void* q, const void* kv, const int32_t* topk_idxs, int64_t B, int64_t M,
                         int64_t H, int64_t N, int64_t D, int64_t topk, const float* sinks, float softmax_scale,
                         void* out, float* lse, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Per-row activation quantiser, the producer of the indexer's low-precision
 * inputs.  Replaces `act_quant_kernel_int8_optimized` / `act_quant_torch`
 * (examples/deepseek_v4/act_quant.py:33-92, :118-142) and extends it to fp8:
 *   amax = max(max |x[r, :]|, 1e-4); scale[r] = amax / QMAX, or with round_scale
 *   2^ceil(log2(amax / QMAX)); y[r, :] = clamp(x / scale, -QMAX, QMAX) converted
 * with QMAX = 127 and round-half-to-even for DSA_KIND_INT8, QMAX = 448 and
 * round-to-nearest-even for DSA_KIND_FP8_E4M3 (OCP e4m3fn).
 *  x [rows, n] of in_kind (bf16, fp16 or fp32); y [rows, n] (1 byte each);
 *  scales [rows] fp32.
 */
int dsa_act_quant(int in_kind, const void* x, int64_t rows, int64_t n, int out_kind, void* y, float* scales,
                  int round_scale, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSA_MI355X_H_ */
