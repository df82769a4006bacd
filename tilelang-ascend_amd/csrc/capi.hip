// C ABI entry points: argument validation, then the kernel launchers.
#include <cstdio>
#include <cstring>

#include "../../include/dsa_mi355x.h"
#include "common.hpp"

namespace dsa {
hipError_t launch_topk(const float* x, int64_t ld, int64_t rows, int64_t n, int64_t k, const int32_t* row_len,
                       int sorted, int32_t* out_idx, float* out_val, void* workspace, hipStream_t stream);
size_t topk_workspace_bytes(int64_t rows, int64_t n, int64_t k);
size_t indexer_topk_fused_bytes(int64_t rows, int64_t B, int64_t S1, int64_t S2, int64_t k);
hipError_t launch_fused_fallback_rows(const void* workspace, int64_t rows, int64_t B, int64_t S1, int64_t S2,
                                      int64_t k, int32_t* count, hipStream_t stream);
hipError_t launch_indexer_topk_fused(int kind, const void* q, const void* k, const float* k_scale, const float* w,
                                     int64_t rows, int64_t B, int64_t S1, int64_t S2, int64_t H, int64_t D,
                                     const int32_t* aq_len, const int32_t* ak_len, const int32_t* cu_q,
                                     const int32_t* cu_k, const int32_t* block_table, int64_t block_size,
                                     int64_t max_blocks, int sparse_mode, int64_t topk, int32_t* out_idx,
                                     float* out_val, void* workspace, hipStream_t stream);
hipError_t launch_indexer_logits(int kind, const void* q, const void* k, const float* k_scale, const float* w,
                                 int64_t B, int64_t S1, int64_t S2, int64_t H, int64_t D, const int32_t* aq_len,
                                 const int32_t* ak_len, const int32_t* cu_q, const int32_t* cu_k,
                                 const int32_t* block_table, int64_t block_size, int64_t max_blocks, int sparse_mode,
                                 float* logits, int64_t ld, hipStream_t stream);
hipError_t launch_sparse_mla(int is_fp16, const void* q, const void* kv, const int32_t* indices, const int32_t* block_table,
                             const int32_t* q_len, const int32_t* kv_len, int64_t B, int64_t S, int64_t G, int64_t H,
                             int64_t Skv, int64_t block_size, int64_t max_blocks, int64_t topk, float sm_scale,
                             int causal, void* out, float* lse, void* workspace, hipStream_t stream);
int64_t sparse_gqa_max_topk();
hipError_t launch_sparse_gqa(int is_fp16, const void* q, const void* kv, const int32_t* indices,
                             const int32_t* q_len, const int32_t* kv_len, int64_t B, int64_t S, int64_t G, int64_t Hg,
                             int64_t Skv, int64_t topk, float sm_scale, int causal, void* out, float* lse,
                             hipStream_t stream);
size_t sparse_mla_workspace_bytes(int64_t tokens, int64_t H, int64_t topk);
size_t mla_scratch_bytes();
hipError_t mla_scratch_ptr(void** out);
size_t v4_workspace_bytes(int64_t T, int64_t H, int64_t cap, bool out_f32);
size_t sparse_attn_sink_workspace_bytes(int64_t T, int64_t H, int64_t K);
hipError_t launch_sparse_attn_sink(int is_fp16, const void* q, const void* kv, const int32_t* idx, int64_t B,
                                   int64_t M, int64_t H, int64_t N, int64_t K, const float* sinks, float sm_scale,
                                   void* out, float* lse, void* workspace, hipStream_t stream);
hipError_t launch_act_quant(int in_kind, const void* x, int64_t rows, int64_t n, int out_kind, void* y,
                            float* scales, int round_scale, hipStream_t stream);
hipError_t launch_sparse_flash_mla(int is_fp16, const void* q, int64_t T, int64_t H, int64_t B,
                                   const int32_t* q_start, const int32_t* q_len, const int32_t* kv_len,
                                   const void* ori_kv, int64_t ori_blocks, int64_t ori_bs, const int32_t* ori_bt,
                                   int64_t ori_tl, const void* cmp_kv, int64_t cmp_blocks, int64_t cmp_bs,
                                   const int32_t* cmp_bt, int64_t cmp_tl, const int32_t* cmp_idx, int64_t K,
                                   int64_t cmp_ratio, int64_t win_left, int64_t max_cmp, int mode, int64_t cap,
                                   const float* sinks, float sm_scale, void* out, float* lse, void* workspace,
                                   hipStream_t stream);
}  // namespace dsa

namespace {
thread_local char g_msg[256] = "";

int reject(const char* what) {
  std::snprintf(g_msg, sizeof(g_msg), "%s", what);
  return (int)hipErrorInvalidValue;
}

int ok(hipError_t e) {
  if (e != hipSuccess) std::snprintf(g_msg, sizeof(g_msg), "launch failed: %s", hipGetErrorString(e));
  return (int)e;
}

constexpr int64_t kMaxInt = 0x7fffffff;
// Physical rows of the V4 caches must stay below the gather kernel's source tag bit.
constexpr int64_t dsa_kSrc2Limit = 0x40000000;
}  // namespace

extern "C" {

int dsa_abi_version(void) { return 106; }

const char* dsa_last_error_message(void) { return g_msg; }

static int check_topk(const float* x, int64_t ld, int64_t rows, int64_t n, int64_t k, const int32_t* out_idx) {
  if (rows < 0 || n < 0 || rows > kMaxInt || n >= kMaxInt) return reject("topk: rows/n out of range");
  if (k < 1 || k > 8192) return reject("topk: k must be in [1, 8192]");
  if (ld < n) return reject("topk: ld < n");
  if (rows > 0 && (!out_idx || (n > 0 && !x))) return reject("topk: null pointer");
  return 0;
}

int dsa_topk_select(const float* x, int64_t ld, int64_t rows, int64_t n, int64_t k, const int32_t* row_len,
                    int sorted, int32_t* out_idx, float* out_val, void* stream) {
  int rc = check_topk(x, ld, rows, n, k, out_idx);
  if (rc) return rc;
  return ok(dsa::launch_topk(x, ld, rows, n, k, row_len, sorted ? 1 : 0, out_idx, out_val, nullptr,
                             static_cast<hipStream_t>(stream)));
}

size_t dsa_topk_select_workspace_size(int64_t rows, int64_t n, int64_t k) {
  if (rows <= 0 || n <= 0 || k < 1) return 0;
  return dsa::topk_workspace_bytes(rows, n, k);
}

int dsa_topk_select_ws(const float* x, int64_t ld, int64_t rows, int64_t n, int64_t k, const int32_t* row_len,
                       int sorted, int32_t* out_idx, float* out_val, void* workspace, size_t workspace_bytes,
                       void* stream) {
  int rc = check_topk(x, ld, rows, n, k, out_idx);
  if (rc) return rc;
  const size_t need = dsa_topk_select_workspace_size(rows, n, k);
  if (workspace_bytes < need) return reject("topk: workspace too small");
  if (need > 0 && !workspace) return reject("topk: null workspace");
  return ok(dsa::launch_topk(x, ld, rows, n, k, row_len, sorted ? 1 : 0, out_idx, out_val,
                             need > 0 ? workspace : nullptr, static_cast<hipStream_t>(stream)));
}

static int check_indexer(int kind, const void* q, const void* k, const float* weights, int64_t B, int64_t S1,
                         int64_t S2, int64_t H, int64_t D, const int32_t* block_table, int64_t block_size,
                         int64_t max_blocks, int sparse_mode) {
  if (kind != DSA_KIND_FP8_E4M3 && kind != DSA_KIND_BF16 && kind != DSA_KIND_FP16) return reject("indexer: bad kind");
  if (D != 128 && D != 64) return reject("indexer: head dim D must be 64 or 128");
  if (H < 1 || H > 64) return reject("indexer: H must be in [1, 64]");
  if (B < 0 || S1 < 0 || S2 < 0 || B > 65535 || S1 > kMaxInt || S2 > kMaxInt) return reject("indexer: bad sizes");
  if (sparse_mode != 0 && sparse_mode != 3) return reject("indexer: sparse_mode must be 0 or 3");
  if (block_table && (block_size <= 0 || max_blocks <= 0 || block_size * max_blocks < S2))
    return reject("indexer: paged key needs block_size > 0 and max_blocks * block_size >= S2");
  if (B * S1 * S2 > 0 && (!q || !k || !weights)) return reject("indexer: null pointer");
  return 0;
}

int dsa_indexer_logits(int kind, const void* q, const void* k, const float* k_scale, const float* weights,
                       int64_t B, int64_t S1, int64_t S2, int64_t H, int64_t D, const int32_t* actual_q_len,
                       const int32_t* actual_k_len, const int32_t* block_table, int64_t block_size,
                       int64_t max_blocks, int sparse_mode, float* logits, int64_t ld, void* stream) {
  int rc = check_indexer(kind, q, k, weights, B, S1, S2, H, D, block_table, block_size, max_blocks, sparse_mode);
  if (rc) return rc;
  if (ld < S2) return reject("indexer: ld < S2");
  if (B * S1 * S2 > 0 && !logits) return reject("indexer: null logits");
  return ok(dsa::launch_indexer_logits(kind, q, k, k_scale, weights, B, S1, S2, H, D, actual_q_len, actual_k_len,
                                       nullptr, nullptr, block_table, block_size, max_blocks, sparse_mode, logits, ld,
                                       static_cast<hipStream_t>(stream)));
}

// Logits of every row, then the top-k candidate buffer for long rows (256-byte aligned).
static size_t indexer_logits_bytes(int64_t B, int64_t S1, int64_t S2) {
  const int64_t ld = (S2 + 3) & ~int64_t(3);
  return ((size_t)(B * S1 * ld) * sizeof(float) + 255) & ~size_t(255);
}

size_t dsa_lightning_indexer_workspace_size(int64_t B, int64_t S1, int64_t S2, int64_t sparse_count) {
  if (B <= 0 || S1 <= 0 || S2 <= 0) return 0;
  const int64_t k = sparse_count < 1 ? 1 : sparse_count;
  return indexer_logits_bytes(B, S1, S2) + dsa::topk_workspace_bytes(B * S1, S2, k);
}

int dsa_lightning_indexer(int kind, const void* q, const void* k, const float* k_scale, const float* weights,
                          int64_t B, int64_t S1, int64_t S2, int64_t H, int64_t D, const int32_t* actual_q_len,
                          const int32_t* actual_k_len, const int32_t* block_table, int64_t block_size,
                          int64_t max_blocks, int sparse_mode, int64_t sparse_count, int32_t* out_idx,
                          float* out_val, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_indexer(kind, q, k, weights, B, S1, S2, H, D, block_table, block_size, max_blocks, sparse_mode);
  if (rc) return rc;
  if (sparse_count < 1 || sparse_count > 8192) return reject("indexer: sparse_count must be in [1, 8192]");
  if (workspace_bytes < dsa_lightning_indexer_workspace_size(B, S1, S2, sparse_count))
    return reject("indexer: workspace too small");
  if (B * S1 > 0 && !out_idx) return reject("indexer: null out_idx");
  if (B * S1 == 0) return 0;
  const int64_t ld = (S2 + 3) & ~int64_t(3);
  float* logits = static_cast<float*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = dsa::launch_indexer_logits(kind, q, k, k_scale, weights, B, S1, S2, H, D, actual_q_len, actual_k_len,
                                            nullptr, nullptr, block_table, block_size, max_blocks, sparse_mode, logits, ld, st);
  if (e != hipSuccess) return ok(e);
  void* cand = dsa::topk_workspace_bytes(B * S1, S2, sparse_count) > 0
                   ? static_cast<void*>(static_cast<uint8_t*>(workspace) + indexer_logits_bytes(B, S1, S2))
                   : nullptr;
  return ok(dsa::launch_topk(logits, ld, B * S1, S2, sparse_count, nullptr, 1, out_idx, out_val, cand, st));
}

int dsa_lightning_indexer_fused_applies(int64_t B, int64_t S1, int64_t S2, int64_t sparse_count) {
  if (B <= 0 || S1 <= 0 || S2 <= 0 || sparse_count < 1) return 0;
  return dsa::indexer_topk_fused_bytes(B * S1, B, S1, S2, sparse_count) > 0;
}

size_t dsa_lightning_indexer_fused_workspace_size(int64_t B, int64_t S1, int64_t S2, int64_t sparse_count) {
  if (B <= 0 || S1 <= 0 || S2 <= 0) return 0;
  const int64_t k = sparse_count < 1 ? 1 : sparse_count;
  const size_t fused = dsa::indexer_topk_fused_bytes(B * S1, B, S1, S2, k);
  return fused ? fused : dsa_lightning_indexer_workspace_size(B, S1, S2, sparse_count);
}

int dsa_lightning_indexer_fused(int kind, const void* q, const void* k, const float* k_scale, const float* weights,
                                int64_t B, int64_t S1, int64_t S2, int64_t H, int64_t D, const int32_t* actual_q_len,
                                const int32_t* actual_k_len, const int32_t* block_table, int64_t block_size,
                                int64_t max_blocks, int sparse_mode, int64_t sparse_count, int32_t* out_idx,
                                float* out_val, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_indexer(kind, q, k, weights, B, S1, S2, H, D, block_table, block_size, max_blocks, sparse_mode);
  if (rc) return rc;
  if (sparse_count < 1 || sparse_count > 8192) return reject("indexer: sparse_count must be in [1, 8192]");
  if (workspace_bytes < dsa_lightning_indexer_fused_workspace_size(B, S1, S2, sparse_count))
    return reject("indexer: workspace too small");
  if (B * S1 > 0 && !out_idx) return reject("indexer: null out_idx");
  if (B * S1 == 0) return 0;
  if (dsa::indexer_topk_fused_bytes(B * S1, B, S1, S2, sparse_count) == 0)
    return dsa_lightning_indexer(kind, q, k, k_scale, weights, B, S1, S2, H, D, actual_q_len, actual_k_len,
                                 block_table, block_size, max_blocks, sparse_mode, sparse_count, out_idx, out_val,
                                 workspace, workspace_bytes, stream);
  return ok(dsa::launch_indexer_topk_fused(kind, q, k, k_scale, weights, B * S1, B, S1, S2, H, D, actual_q_len,
                                           actual_k_len, nullptr, nullptr, block_table, block_size, max_blocks,
                                           sparse_mode, sparse_count, out_idx, out_val, workspace,
                                           static_cast<hipStream_t>(stream)));
}

int dsa_lightning_indexer_fused_fallback_rows(const void* workspace, int64_t B, int64_t S1, int64_t S2,
                                              int64_t sparse_count, int32_t* count, void* stream) {
  if (!dsa_lightning_indexer_fused_applies(B, S1, S2, sparse_count))
    return reject("indexer: the fused path does not apply to this shape");
  if (!workspace || !count) return reject("indexer: null pointer");
  return ok(dsa::launch_fused_fallback_rows(workspace, B * S1, B, S1, S2, sparse_count, count,
                                            static_cast<hipStream_t>(stream)));
}

static int check_indexer_tnd(int kind, const void* q, const void* k, const float* weights, int64_t B, int64_t T,
                             int64_t S1_max, int64_t S2_max, int64_t H, int64_t D, const int32_t* cu_q,
                             const int32_t* cu_k, const int32_t* actual_k_len, const int32_t* block_table,
                             int64_t block_size, int64_t max_blocks, int sparse_mode) {
  int rc = check_indexer(kind, q, k, weights, B, S1_max, S2_max, H, D, block_table, block_size, max_blocks,
                         sparse_mode);
  if (rc) return rc;
  if (T < 0 || T > kMaxInt) return reject("indexer: bad T");
  if (B > 0 && !cu_q) return reject("indexer: TND query needs cu_q");
  if ((cu_k != nullptr) == (block_table != nullptr))
    return reject("indexer: TND keys need exactly one of cu_k (packed) and block_table (paged)");
  if (block_table && !actual_k_len) return reject("indexer: paged keys need actual_k_len");
  return 0;
}

int dsa_indexer_logits_tnd(int kind, const void* q, const void* k, const float* k_scale, const float* weights,
                           int64_t B, int64_t T, int64_t S1_max, int64_t S2_max, int64_t H, int64_t D,
                           const int32_t* cu_q, const int32_t* cu_k, const int32_t* actual_k_len,
                           const int32_t* block_table, int64_t block_size, int64_t max_blocks, int sparse_mode,
                           float* logits, int64_t ld, void* stream) {
  int rc = check_indexer_tnd(kind, q, k, weights, B, T, S1_max, S2_max, H, D, cu_q, cu_k, actual_k_len, block_table,
                             block_size, max_blocks, sparse_mode);
  if (rc) return rc;
  if (ld < S2_max) return reject("indexer: ld < S2_max");
  if (T * S2_max > 0 && !logits) return reject("indexer: null logits");
  if (T == 0) return 0;
  return ok(dsa::launch_indexer_logits(kind, q, k, k_scale, weights, B, S1_max, S2_max, H, D, nullptr,
                                       actual_k_len, cu_q, cu_k, block_table, block_size, max_blocks, sparse_mode,
                                       logits, ld, static_cast<hipStream_t>(stream)));
}

size_t dsa_lightning_indexer_tnd_workspace_size(int64_t T, int64_t S2_max, int64_t sparse_count) {
  return dsa_lightning_indexer_workspace_size(1, T, S2_max, sparse_count);
}

int dsa_lightning_indexer_tnd(int kind, const void* q, const void* k, const float* k_scale, const float* weights,
                              int64_t B, int64_t T, int64_t S1_max, int64_t S2_max, int64_t H, int64_t D,
                              const int32_t* cu_q, const int32_t* cu_k, const int32_t* actual_k_len,
                              const int32_t* block_table, int64_t block_size, int64_t max_blocks, int sparse_mode,
                              int64_t sparse_count, int32_t* out_idx, float* out_val, void* workspace,
                              size_t workspace_bytes, void* stream) {
  int rc = check_indexer_tnd(kind, q, k, weights, B, T, S1_max, S2_max, H, D, cu_q, cu_k, actual_k_len, block_table,
                             block_size, max_blocks, sparse_mode);
  if (rc) return rc;
  if (sparse_count < 1 || sparse_count > 8192) return reject("indexer: sparse_count must be in [1, 8192]");
  if (workspace_bytes < dsa_lightning_indexer_tnd_workspace_size(T, S2_max, sparse_count))
    return reject("indexer: workspace too small");
  if (T > 0 && !out_idx) return reject("indexer: null out_idx");
  if (T == 0 || S2_max == 0 || B == 0) return 0;
  const int64_t ld = (S2_max + 3) & ~int64_t(3);
  float* logits = static_cast<float*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = dsa::launch_indexer_logits(kind, q, k, k_scale, weights, B, S1_max, S2_max, H, D, nullptr,
                                            actual_k_len, cu_q, cu_k, block_table, block_size, max_blocks,
                                            sparse_mode, logits, ld, st);
  if (e != hipSuccess) return ok(e);
  void* cand = dsa::topk_workspace_bytes(T, S2_max, sparse_count) > 0
                   ? static_cast<void*>(static_cast<uint8_t*>(workspace) + indexer_logits_bytes(1, T, S2_max))
                   : nullptr;
  return ok(dsa::launch_topk(logits, ld, T, S2_max, sparse_count, nullptr, 1, out_idx, out_val, cand, st));
}

size_t dsa_lightning_indexer_tnd_fused_workspace_size(int64_t B, int64_t T, int64_t S1_max, int64_t S2_max,
                                                      int64_t sparse_count) {
  if (B <= 0 || T <= 0 || S1_max <= 0 || S2_max <= 0) return 0;
  const int64_t k = sparse_count < 1 ? 1 : sparse_count;
  const size_t fused = dsa::indexer_topk_fused_bytes(T, B, S1_max, S2_max, k);
  return fused ? fused : dsa_lightning_indexer_tnd_workspace_size(T, S2_max, sparse_count);
}

int dsa_lightning_indexer_tnd_fused(int kind, const void* q, const void* k, const float* k_scale,
                                    const float* weights, int64_t B, int64_t T, int64_t S1_max, int64_t S2_max,
                                    int64_t H, int64_t D, const int32_t* cu_q, const int32_t* cu_k,
                                    const int32_t* actual_k_len, const int32_t* block_table, int64_t block_size,
                                    int64_t max_blocks, int sparse_mode, int64_t sparse_count, int32_t* out_idx,
                                    float* out_val, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_indexer_tnd(kind, q, k, weights, B, T, S1_max, S2_max, H, D, cu_q, cu_k, actual_k_len, block_table,
                             block_size, max_blocks, sparse_mode);
  if (rc) return rc;
  if (sparse_count < 1 || sparse_count > 8192) return reject("indexer: sparse_count must be in [1, 8192]");
  if (workspace_bytes < dsa_lightning_indexer_tnd_fused_workspace_size(B, T, S1_max, S2_max, sparse_count))
    return reject("indexer: workspace too small");
  if (T > 0 && !out_idx) return reject("indexer: null out_idx");
  if (T == 0 || S2_max == 0 || B == 0) return 0;
  if (dsa::indexer_topk_fused_bytes(T, B, S1_max, S2_max, sparse_count) == 0)
    return dsa_lightning_indexer_tnd(kind, q, k, k_scale, weights, B, T, S1_max, S2_max, H, D, cu_q, cu_k,
                                     actual_k_len, block_table, block_size, max_blocks, sparse_mode, sparse_count,
                                     out_idx, out_val, workspace, workspace_bytes, stream);
  return ok(dsa::launch_indexer_topk_fused(kind, q, k, k_scale, weights, T, B, S1_max, S2_max, H, D, nullptr,
                                           actual_k_len, cu_q, cu_k, block_table, block_size, max_blocks,
                                           sparse_mode, sparse_count, out_idx, out_val, workspace,
                                           static_cast<hipStream_t>(stream)));
}

size_t dsa_sparse_mla_workspace_size(int64_t B, int64_t S, int64_t H, int64_t topk) {
  if (B <= 0 || S <= 0 || H <= 0 || topk <= 0) return 0;
  return dsa::sparse_mla_workspace_bytes(B * S, H, topk);
}

int dsa_sparse_mla_fwd(int kind, const void* q, const void* kv, const int32_t* indices,
                       const int32_t* block_table, const int32_t* actual_q_len, const int32_t* actual_kv_len,
                       int64_t B, int64_t S, int64_t H, int64_t d_qk, int64_t d_v, int64_t Skv, int64_t block_size,
                       int64_t max_blocks, int64_t topk, float sm_scale, int is_causal, void* out, float* lse,
                       void* workspace, size_t workspace_bytes, void* stream) {
  if (kind != DSA_KIND_BF16 && kind != DSA_KIND_FP16) return reject("sparse_mla: kind must be bf16 or fp16");
  if (d_qk != 576 || d_v != 512) return reject("sparse_mla: d_qk must be 576 and d_v 512");
  if (H < 16 || H % 16 != 0 || H > 1024) return reject("sparse_mla: H must be a multiple of 16 in [16, 1024]");
  if (B < 0 || S < 0 || topk < 1 || B * S > kMaxInt || topk > kMaxInt) return reject("sparse_mla: bad sizes");
  if (block_table) {
    if (block_size <= 0 || max_blocks <= 0 || block_size * max_blocks > kMaxInt)
      return reject("sparse_mla: paged kv needs block_size > 0 and max_blocks > 0");
  } else if (Skv < 0 || Skv > kMaxInt) {
    return reject("sparse_mla: bad Skv");
  }
  if (!(sm_scale > 0.f) || !(sm_scale < 3.0e38f)) return reject("sparse_mla: sm_scale must be positive and finite");
  if (workspace_bytes < dsa_sparse_mla_workspace_size(B, S, H, topk)) return reject("sparse_mla: workspace too small");
  if (B * S > 0 && (!q || !kv || !indices || !out || !lse)) return reject("sparse_mla: null pointer");
  const int64_t skv_eff = block_table ? block_size * max_blocks : Skv;
  return ok(dsa::launch_sparse_mla(kind == DSA_KIND_FP16, q, kv, indices, block_table, actual_q_len, actual_kv_len, B, S, 1, H,
                                   skv_eff, block_size, max_blocks, topk, sm_scale, is_causal ? 1 : 0, out, lse,
                                   workspace, static_cast<hipStream_t>(stream)));
}

size_t dsa_sparse_attention_workspace_size(int64_t B, int64_t S, int64_t H, int64_t kv_group, int64_t d_qk,
                                           int64_t topk) {
  if (B <= 0 || S <= 0 || H <= 0 || topk <= 0 || kv_group <= 0 || H % kv_group != 0) return 0;
  if (d_qk != 576) return 0;  // the 128-wide kernel needs no workspace
  return dsa::sparse_mla_workspace_bytes(B * S * kv_group, H / kv_group, topk);
}

int dsa_sparse_attention_fwd(int kind, const void* q, const void* kv, const int32_t* indices,
                             const int32_t* block_table, const int32_t* actual_q_len, const int32_t* actual_kv_len,
                             int64_t B, int64_t S, int64_t H, int64_t kv_group, int64_t d_qk, int64_t d_v, int64_t Skv,
                             int64_t block_size, int64_t max_blocks, int64_t topk, float sm_scale, int is_causal,
                             void* out, float* lse, void* workspace, size_t workspace_bytes, void* stream) {
  if (kind != DSA_KIND_BF16 && kind != DSA_KIND_FP16) return reject("sparse_attention: kind must be bf16 or fp16");
  if (kv_group < 1 || H < 1 || H % kv_group != 0)
    return reject("sparse_attention: H must be a positive multiple of kv_group >= 1");
  const int64_t Hg = H / kv_group;
  if (B < 0 || S < 0 || topk < 1 || B * S > kMaxInt / kv_group || topk > kMaxInt)
    return reject("sparse_attention: bad sizes");
  if (!(sm_scale > 0.f) || !(sm_scale < 3.0e38f))
    return reject("sparse_attention: sm_scale must be positive and finite");
  const bool mla = d_qk == 576 && d_v == 512;
  if (mla) {
    if (Hg % 16 != 0 || Hg > 1024)
      return reject("sparse_attention: heads per KV group must be a multiple of 16 in [16, 1024] (d_qk 576)");
    if (block_table) {
      if (block_size <= 0 || max_blocks <= 0 || block_size * max_blocks > kMaxInt)
        return reject("sparse_attention: paged kv needs block_size > 0 and max_blocks > 0");
    } else if (Skv < 0 || B * Skv > kMaxInt / kv_group) {
      return reject("sparse_attention: B x Skv x kv_group must stay below 2^31");
    }
  } else if (d_qk == 128 && d_v == 128) {
    if (block_table) return reject("sparse_attention: d_qk 128 takes a contiguous kv (no block table)");
    if (Hg > 1024) return reject("sparse_attention: at most 1024 heads per KV group");
    if (topk > dsa::sparse_gqa_max_topk()) return reject("sparse_attention: topk must be <= 8192 (d_qk 128)");
    if (Skv < 0 || B * Skv > kMaxInt / kv_group) return reject("sparse_attention: B x Skv x kv_group must stay below 2^31");
  } else {
    return reject("sparse_attention: (d_qk, d_v) must be (576, 512) or (128, 128)");
  }
  if (workspace_bytes < dsa_sparse_attention_workspace_size(B, S, H, kv_group, d_qk, topk))
    return reject("sparse_attention: workspace too small");
  if (B * S > 0 && (!q || !kv || !indices || !out || !lse)) return reject("sparse_attention: null pointer");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (mla) {
    const int64_t skv_eff = block_table ? block_size * max_blocks : Skv;
    return ok(dsa::launch_sparse_mla(kind == DSA_KIND_FP16, q, kv, indices, block_table, actual_q_len, actual_kv_len, B,
                                     S, kv_group, Hg, skv_eff, block_size, max_blocks, topk, sm_scale,
                                     is_causal ? 1 : 0, out, lse, workspace, st));
  }
  return ok(dsa::launch_sparse_gqa(kind == DSA_KIND_FP16, q, kv, indices, actual_q_len, actual_kv_len, B, S, kv_group,
                                   Hg, Skv, topk, sm_scale, is_causal ? 1 : 0, out, lse, st));
}

size_t dsa_sparse_mla_noalloc_max_workspace(void) { return dsa::mla_scratch_bytes(); }

int dsa_sparse_mla_fwd_noalloc(int kind, const void* q, const void* kv, const int32_t* indices,
                               const int32_t* block_table, const int32_t* actual_q_len, const int32_t* actual_kv_len,
                               int64_t B, int64_t S, int64_t H, int64_t d_qk, int64_t d_v, int64_t Skv,
                               int64_t block_size, int64_t max_blocks, int64_t topk, float sm_scale, int is_causal,
                               void* out, float* lse, void* stream) {
  const size_t need = dsa_sparse_mla_workspace_size(B, S, H, topk);
  if (need > dsa::mla_scratch_bytes())
    return reject("sparse_mla_noalloc: the split partials of this shape exceed the 64 MiB scratch "
                  "(dsa_sparse_mla_noalloc_max_workspace); use dsa_sparse_mla_fwd with a workspace");
  void* ws = nullptr;
  if (need > 0) {
    const hipError_t e = dsa::mla_scratch_ptr(&ws);
    if (e != hipSuccess) return ok(e);
  }
  return dsa_sparse_mla_fwd(kind, q, kv, indices, block_table, actual_q_len, actual_kv_len, B, S, H, d_qk, d_v, Skv,
                            block_size, max_blocks, topk, sm_scale, is_causal, out, lse, ws, need, stream);
}

// Row-list capacity of a V4 call: the window plus the compressed slots.
static int64_t v4_cap(int64_t ori_win_left, int64_t cmp_slots) { return ori_win_left + 1 + cmp_slots; }

size_t dsa_sparse_flash_mla_workspace_size(int64_t T, int64_t H, int64_t ori_win_left, int64_t cmp_slots) {
  if (T <= 0 || H <= 0 || ori_win_left < 0 || cmp_slots < 0) return 0;
  return dsa::v4_workspace_bytes(T, H, v4_cap(ori_win_left, cmp_slots), false);
}

int dsa_sparse_flash_mla(int kind, const void* q, int64_t T, int64_t H, int64_t D, int64_t B, const int32_t* q_start,
                         const int32_t* q_len, const int32_t* seqused_kv, const void* ori_kv, int64_t ori_block_num,
                         int64_t ori_block_size, const int32_t* ori_block_table, int64_t ori_table_len,
                         const void* cmp_kv, int64_t cmp_block_num, int64_t cmp_block_size,
                         const int32_t* cmp_block_table, int64_t cmp_table_len, const int32_t* cmp_sparse_indices,
                         int64_t topk_cmp, int64_t cmp_ratio, int64_t ori_win_left, int64_t max_cmp,
                         const float* sinks, float softmax_scale, void* out, float* lse, void* workspace,
                         size_t workspace_bytes, void* stream) {
  if (kind != DSA_KIND_BF16 && kind != DSA_KIND_FP16) return reject("sparse_flash_mla: kind must be bf16 or fp16");
  if (D != 512) return reject("sparse_flash_mla: D must be 512");
  if (H < 16 || H % 16 != 0 || H > 1024) return reject("sparse_flash_mla: H must be a multiple of 16 in [16, 1024]");
  if (T < 0 || B < 1 || T > kMaxInt || B > kMaxInt) return reject("sparse_flash_mla: bad T / B");
  if (ori_win_left < 0 || ori_win_left > 65535) return reject("sparse_flash_mla: ori_win_left must be in [0, 65535]");
  if (ori_block_size <= 0 || ori_block_num <= 0 || ori_table_len <= 0 ||
      ori_block_num * ori_block_size >= dsa_kSrc2Limit)
    return reject("sparse_flash_mla: bad original KV pool");
  if (T > 0 && (!q || !ori_kv || !ori_block_table || !q_start || !q_len || !seqused_kv || !out || !lse))
    return reject("sparse_flash_mla: null pointer");
  int mode = 1;
  int64_t cmp_slots = 0;
  if (cmp_kv) {
    if (cmp_ratio < 1) return reject("sparse_flash_mla: cmp_ratio must be >= 1");
    if (cmp_block_size <= 0 || cmp_block_num <= 0 || cmp_table_len <= 0 || !cmp_block_table ||
        cmp_block_num * cmp_block_size >= dsa_kSrc2Limit)
      return reject("sparse_flash_mla: bad compressed KV pool");
    if (cmp_sparse_indices) {
      if (topk_cmp < 1 || topk_cmp > 65536) return reject("sparse_flash_mla: topk_cmp must be in [1, 65536]");
      mode = 3;
      cmp_slots = topk_cmp;
    } else {
      if (max_cmp < 0 || max_cmp > 65536) return reject("sparse_flash_mla: max_cmp must be in [0, 65536]");
      mode = 2;
      cmp_slots = max_cmp;
    }
  }
  const int64_t cap = v4_cap(ori_win_left, cmp_slots);
  if (T * (cap + 1) > kMaxInt) return reject("sparse_flash_mla: T x slots too large");
  if (workspace_bytes < dsa_sparse_flash_mla_workspace_size(T, H, ori_win_left, cmp_slots))
    return reject("sparse_flash_mla: workspace too small");
  if (T > 0 && !workspace) return reject("sparse_flash_mla: null workspace");
  return ok(dsa::launch_sparse_flash_mla(kind == DSA_KIND_FP16, q, T, H, B, q_start, q_len, seqused_kv, ori_kv,
                                         ori_block_num, ori_block_size, ori_block_table, ori_table_len, cmp_kv,
                                         cmp_block_num, cmp_block_size, cmp_block_table, cmp_table_len,
                                         cmp_sparse_indices, topk_cmp, cmp_ratio, ori_win_left, max_cmp, mode, cap,
                                         sinks, softmax_scale, out, lse, workspace, static_cast<hipStream_t>(stream)));
}

int dsa_act_quant(int in_kind, const void* x, int64_t rows, int64_t n, int out_kind, void* y, float* scales,
                  int round_scale, void* stream) {
  if (in_kind != DSA_KIND_BF16 && in_kind != DSA_KIND_FP16 && in_kind != DSA_KIND_FP32)
    return reject("act_quant: input kind must be bf16, fp16 or fp32");
  if (out_kind != DSA_KIND_FP8_E4M3 && out_kind != DSA_KIND_INT8) return reject("act_quant: output kind must be fp8 or int8");
  if (rows < 0 || n < 0 || n > kMaxInt || (n > 0 && rows > ((int64_t)1 << 62) / n)) return reject("act_quant: bad sizes");
  if (rows * n > 0 && (!x || !y || !scales)) return reject("act_quant: null pointer");
  return ok(dsa::launch_act_quant(in_kind, x, rows, n, out_kind, y, scales, round_scale ? 1 : 0,
                                  static_cast<hipStream_t>(stream)));
}

size_t dsa_sparse_attn_sink_workspace_size(int64_t B, int64_t M, int64_t H, int64_t topk) {
  if (B <= 0 || M <= 0 || H <= 0 || topk <= 0) return 0;
  return dsa::sparse_attn_sink_workspace_bytes(B * M, H, topk);
}

int dsa_sparse_attn_sink(int kind, const void* q, const void* kv, const int32_t* topk_idxs, int64_t B, int64_t M,
                         int64_t H, int64_t N, int64_t D, int64_t topk, const float* sinks, float softmax_scale,
                         void* out, float* lse, void* workspace, size_t workspace_bytes, void* stream) {
  if (kind != DSA_KIND_BF16 && kind != DSA_KIND_FP16) return reject("sparse_attn: kind must be bf16 or fp16");
  if (D != 512) return reject("sparse_attn: D must be 512");
  if (H < 16 || H % 16 != 0 || H > 1024) return reject("sparse_attn: H must be a multiple of 16 in [16, 1024]");
  if (B < 0 || M < 0 || N < 0 || topk < 1 || B * N >= dsa_kSrc2Limit || (topk + 1) * B * M > kMaxInt)
    return reject("sparse_attn: bad sizes");
  if (B * M > 0 && (!q || !kv || !topk_idxs || !out || !lse)) return reject("sparse_attn: null pointer");
  const size_t need = dsa_sparse_attn_sink_workspace_size(B, M, H, topk);
  if (workspace_bytes < need) return reject("sparse_attn: workspace too small");
  if (need > 0 && !workspace) return reject("sparse_attn: null workspace");
  return ok(dsa::launch_sparse_attn_sink(kind == DSA_KIND_FP16, q, kv, topk_idxs, B, M, H, N, topk, sinks,
                                         softmax_scale, out, lse, workspace, static_cast<hipStream_t>(stream)));
}

}  // extern "C"
