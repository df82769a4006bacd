// PyTorch operator registration of the DSA kernels: torch.ops.dsa.*.
//
// The pattern of examples/torch_tl_ascend/src/_inner.cpp:17-68 (a wrapper that
// allocates outputs and workspaces with ATen, fetches the current stream and
// calls the C entry point; TORCH_LIBRARY schemas; device and Meta
// implementations), for a HIP device: the device implementations call the C
// ABI of include/dsa_mi355x.h on the current HIP stream; the Meta
// implementations only compute output shapes, so the ops trace under
// torch.compile / FakeTensor.  No implementation synchronises with the host or
// allocates outside ATen's caching allocator, so the calls can be captured in a
// HIP graph.  Sizes that the Python wrappers read from device tensors (the
// longest paged key length, the compressed-row bound of V4 "hca") are explicit
// arguments here.
//
// Every tensor argument, optional ones included, is checked before anything is
// launched: on the main tensor's device, of the expected element count / shape,
// and made contiguous in the dtype the kernel reads (a host tensor or a short
// buffer raises here instead of reaching a kernel).
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include "../../include/dsa_mi355x.h"

namespace {

void* ptr(const at::Tensor& t) { return t.data_ptr(); }
template <typename T>
T* ptr_or_null(const c10::optional<at::Tensor>& t) {
  return t.has_value() ? static_cast<T*>(t->data_ptr()) : nullptr;
}

void* stream_of(const at::Tensor& t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

void check_rc(int rc, const char* what) {
  TORCH_CHECK(rc == 0, "dsa.", what, ": ", dsa_last_error_message(), " (hipError ", rc, ")");
}

int kind_of(const at::Tensor& t) {
  switch (t.scalar_type()) {
    case at::kFloat8_e4m3fn: return DSA_KIND_FP8_E4M3;
    case at::kBFloat16: return DSA_KIND_BF16;
    case at::kHalf: return DSA_KIND_FP16;
    case at::kFloat: return DSA_KIND_FP32;
    case at::kChar: return DSA_KIND_INT8;
    default: TORCH_CHECK(false, "dsa: unsupported dtype ", t.scalar_type());
  }
  return -1;
}

void require(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda(), "dsa: ", name, " must be on a HIP device");
  TORCH_CHECK(t.is_contiguous(), "dsa: ", name, " must be contiguous");
}

// A tensor a kernel reads lives on the main tensor's device: a host tensor (the
// torch_npu convention for actual_seq_lengths) or one on another GPU would hand
// the kernel an address it cannot read.
void require_on(const at::Tensor& t, const at::Tensor& main, const char* name) {
  TORCH_CHECK(t.is_cuda() && t.device() == main.device(), "dsa: ", name, " must be on ", main.device(), " (got ",
              t.device(), ")");
}

void require_numel(const at::Tensor& t, int64_t n, const char* name) {
  TORCH_CHECK(t.numel() == n, "dsa: ", name, " must have ", n, " elements (got ", t.numel(), ")");
}

bool is_int(const at::Tensor& t) {
  return at::isIntegralType(t.scalar_type(), /*includeBool=*/false);
}

// An int32 argument: on main's device, integral, `n` elements (n < 0: any), made contiguous int32.
at::Tensor aux_i32(const at::Tensor& t, const at::Tensor& main, int64_t n, const char* name) {
  require_on(t, main, name);
  TORCH_CHECK(is_int(t), "dsa: ", name, " must be an integer tensor (got ", t.scalar_type(), ")");
  if (n >= 0) require_numel(t, n, name);
  return t.to(at::kInt).contiguous();
}

c10::optional<at::Tensor> aux_i32(const c10::optional<at::Tensor>& t, const at::Tensor& main, int64_t n,
                                  const char* name) {
  if (!t.has_value()) return t;
  return aux_i32(*t, main, n, name);
}

// A float argument: on main's device, `n` elements, made contiguous fp32.
at::Tensor aux_f32(const at::Tensor& t, const at::Tensor& main, int64_t n, const char* name) {
  require_on(t, main, name);
  TORCH_CHECK(at::isFloatingType(t.scalar_type()), "dsa: ", name, " must be a floating-point tensor");
  require_numel(t, n, name);
  return t.to(at::kFloat).contiguous();
}

c10::optional<at::Tensor> aux_f32(const c10::optional<at::Tensor>& t, const at::Tensor& main, int64_t n,
                                  const char* name) {
  if (!t.has_value()) return t;
  return aux_f32(*t, main, n, name);
}

// A block table [B, max_blocks] (max_blocks >= 1) on main's device, made contiguous int32.
at::Tensor aux_table(const at::Tensor& t, const at::Tensor& main, int64_t B, const char* name) {
  TORCH_CHECK(t.dim() == 2 && t.size(0) == B && t.size(1) > 0, "dsa: ", name, " must be [", B,
              ", max_blocks] (got ", t.sizes(), ")");
  return aux_i32(t, main, -1, name);
}

c10::optional<at::Tensor> aux_table(const c10::optional<at::Tensor>& t, const at::Tensor& main, int64_t B,
                                    const char* name) {
  if (!t.has_value()) return t;
  return aux_table(*t, main, B, name);
}

// ---------------------------------------------------------------- top-k
std::tuple<at::Tensor, at::Tensor> topk_select(const at::Tensor& x, int64_t k, bool sorted) {
  require(x, "x");
  TORCH_CHECK(x.dim() == 2 && x.scalar_type() == at::kFloat, "dsa.topk_select: x must be [rows, n] fp32");
  TORCH_CHECK(k >= 1 && k <= 8192, "dsa.topk_select: k must be in [1, 8192]");
  c10::OptionalDeviceGuard guard(x.device());
  const int64_t rows = x.size(0), n = x.size(1);
  auto idx = at::empty({rows, k}, x.options().dtype(at::kInt));
  auto val = at::empty({rows, k}, x.options());
  const size_t ws_bytes = dsa_topk_select_workspace_size(rows, n, k);
  auto ws = at::empty({(int64_t)(ws_bytes > 0 ? ws_bytes : 1)}, x.options().dtype(at::kByte));
  check_rc(dsa_topk_select_ws(static_cast<const float*>(ptr(x)), n, rows, n, k, nullptr, sorted ? 1 : 0,
                              static_cast<int32_t*>(ptr(idx)), static_cast<float*>(ptr(val)), ptr(ws), ws_bytes,
                              stream_of(x)),
           "topk_select");
  return {idx, val};
}

std::tuple<at::Tensor, at::Tensor> topk_select_meta(const at::Tensor& x, int64_t k, bool) {
  return {at::empty({x.size(0), k}, x.options().dtype(at::kInt)), at::empty({x.size(0), k}, x.options())};
}

// ---------------------------------------------------------------- lightning indexer (BSND query)
// query [B, S1, H, D]; key [B, S2, 1, D] or paged [blocks, block_size, 1, D] with block_table, in
// which case s2 (the longest key length) is required.
std::tuple<at::Tensor, at::Tensor> lightning_indexer(const at::Tensor& query, const at::Tensor& key,
                                                     const at::Tensor& weights,
                                                     const c10::optional<at::Tensor>& key_scale,
                                                     const c10::optional<at::Tensor>& actual_seq_lengths_query,
                                                     const c10::optional<at::Tensor>& actual_seq_lengths_key,
                                                     const c10::optional<at::Tensor>& block_table,
                                                     int64_t sparse_count, int64_t sparse_mode, bool return_value,
                                                     int64_t s2) {
  require(query, "query");
  require(key, "key");
  require_on(key, query, "key");
  TORCH_CHECK(query.dim() == 4 && key.dim() == 4, "dsa.lightning_indexer: query and key must be 4-D");
  TORCH_CHECK(key.scalar_type() == query.scalar_type(), "dsa.lightning_indexer: key dtype must equal query dtype");
  TORCH_CHECK(sparse_count >= 1 && sparse_count <= 8192, "dsa.lightning_indexer: sparse_count must be in [1, 8192]");
  c10::OptionalDeviceGuard guard(query.device());
  const int64_t B = query.size(0), S1 = query.size(1), H = query.size(2), D = query.size(3);
  const bool paged = block_table.has_value();
  TORCH_CHECK(key.size(2) == 1 && key.size(3) == D, "dsa.lightning_indexer: key must be [.., .., 1, ", D, "] (got ",
              key.sizes(), ")");
  TORCH_CHECK(paged || key.size(0) == B, "dsa.lightning_indexer: key batch ", key.size(0), " != query batch ", B);
  TORCH_CHECK(!paged || s2 > 0, "dsa.lightning_indexer: paged keys need s2 (the longest key length)");
  const int64_t S2 = paged ? s2 : key.size(1);
  auto w = aux_f32(weights, query, B * S1 * H, "weights");
  // One scale per key row of `key` (contiguous [B, S2] or paged [blocks, block_size]).
  auto ks = aux_f32(key_scale, query, key.size(0) * key.size(1), "key_scale");
  auto aq = aux_i32(actual_seq_lengths_query, query, B, "actual_seq_lengths_query");
  auto ak = aux_i32(actual_seq_lengths_key, query, B, "actual_seq_lengths_key");
  auto bt = aux_table(block_table, query, B, "block_table");
  TORCH_CHECK(!paged || bt->size(1) * key.size(1) >= S2,
              "dsa.lightning_indexer: block_table covers fewer than s2 keys");
  auto idx = at::empty({B, S1, 1, sparse_count}, query.options().dtype(at::kInt));
  auto val = return_value ? at::empty({B, S1, 1, sparse_count}, query.options().dtype(at::kFloat))
                          : at::empty({0}, query.options().dtype(at::kFloat));
  if (B * S1 == 0) return {idx, val};
  // At least 2048 rows past 32768 keys stream the top-k out of the indexer (same output, no full logits).
  const bool fused = S2 > 32768 && B * S1 >= 2048;
  const size_t ws_bytes = fused ? dsa_lightning_indexer_fused_workspace_size(B, S1, S2, sparse_count)
                                : dsa_lightning_indexer_workspace_size(B, S1, S2, sparse_count);
  auto ws = at::empty({(int64_t)(ws_bytes > 0 ? ws_bytes : 1)}, query.options().dtype(at::kByte));
  check_rc((fused ? dsa_lightning_indexer_fused : dsa_lightning_indexer)(kind_of(query), ptr(query), ptr(key), ptr_or_null<float>(ks),
                                 static_cast<float*>(ptr(w)), B, S1, S2, H, D, ptr_or_null<int32_t>(aq),
                                 ptr_or_null<int32_t>(ak), ptr_or_null<int32_t>(bt), paged ? key.size(1) : 0,
                                 paged ? bt->size(1) : 0, (int)sparse_mode, sparse_count,
                                 static_cast<int32_t*>(ptr(idx)), return_value ? static_cast<float*>(ptr(val)) : nullptr,
                                 ptr(ws), ws_bytes, stream_of(query)),
           "lightning_indexer");
  return {idx, val};
}

std::tuple<at::Tensor, at::Tensor> lightning_indexer_meta(const at::Tensor& query, const at::Tensor&,
                                                          const at::Tensor&, const c10::optional<at::Tensor>&,
                                                          const c10::optional<at::Tensor>&,
                                                          const c10::optional<at::Tensor>&,
                                                          const c10::optional<at::Tensor>&, int64_t sparse_count,
                                                          int64_t, bool return_value, int64_t) {
  const int64_t B = query.size(0), S1 = query.size(1);
  auto idx = at::empty({B, S1, 1, sparse_count}, query.options().dtype(at::kInt));
  auto val = return_value ? at::empty({B, S1, 1, sparse_count}, query.options().dtype(at::kFloat))
                          : at::empty({0}, query.options().dtype(at::kFloat));
  return {idx, val};
}

// ---------------------------------------------------------------- sparse MLA (d_qk 576, d_v 512)
// q [B, S, H, 576]; kv [B, Skv, 1, 576] or paged [blocks, block_size, 1, 576]; indices [B, S, 1, topk].
std::tuple<at::Tensor, at::Tensor> sparse_mla_fwd(const at::Tensor& q, const at::Tensor& kv,
                                                  const at::Tensor& indices, double sm_scale,
                                                  const c10::optional<at::Tensor>& block_table,
                                                  const c10::optional<at::Tensor>& actual_seq_lengths_query,
                                                  const c10::optional<at::Tensor>& actual_seq_lengths_kv,
                                                  bool is_causal) {
  require(q, "q");
  require(kv, "kv");
  require(indices, "indices");
  require_on(kv, q, "kv");
  require_on(indices, q, "indices");
  TORCH_CHECK(q.dim() == 4 && q.size(3) == 576, "dsa.sparse_mla_fwd: q must be [B, S, H, 576] (got ", q.sizes(), ")");
  TORCH_CHECK(kv.dim() == 4 && kv.size(2) == 1 && kv.size(3) == 576,
              "dsa.sparse_mla_fwd: kv must be [B, Skv, 1, 576] or [blocks, block_size, 1, 576] (got ", kv.sizes(), ")");
  TORCH_CHECK(kv.scalar_type() == q.scalar_type(), "dsa.sparse_mla_fwd: kv dtype must equal q dtype");
  TORCH_CHECK(indices.scalar_type() == at::kInt, "dsa.sparse_mla_fwd: indices must be int32");
  c10::OptionalDeviceGuard guard(q.device());
  const int64_t B = q.size(0), S = q.size(1), H = q.size(2);
  TORCH_CHECK(indices.dim() == 4 && indices.size(0) == B && indices.size(1) == S && indices.size(2) == 1 &&
                  indices.size(3) >= 1,
              "dsa.sparse_mla_fwd: indices must be [", B, ", ", S, ", 1, topk] (got ", indices.sizes(), ")");
  const int64_t topk = indices.size(3);
  const bool paged = block_table.has_value();
  TORCH_CHECK(paged || kv.size(0) == B, "dsa.sparse_mla_fwd: kv batch ", kv.size(0), " != q batch ", B);
  auto bt = aux_table(block_table, q, B, "block_table");
  auto aq = aux_i32(actual_seq_lengths_query, q, B, "actual_seq_lengths_query");
  auto ak = aux_i32(actual_seq_lengths_kv, q, B, "actual_seq_lengths_kv");
  auto out = at::empty({B, S, H, 512}, q.options());
  auto lse = at::empty({B, S, H}, q.options().dtype(at::kFloat));
  const size_t ws_bytes = dsa_sparse_mla_workspace_size(B, S, H, topk);
  auto ws = at::empty({(int64_t)(ws_bytes > 0 ? ws_bytes : 1)}, q.options().dtype(at::kByte));
  const int64_t nblk = paged ? bt->size(1) : 0, bs = paged ? kv.size(1) : 0;
  check_rc(dsa_sparse_mla_fwd(kind_of(q), ptr(q), ptr(kv), static_cast<const int32_t*>(ptr(indices)),
                              ptr_or_null<int32_t>(bt), ptr_or_null<int32_t>(aq), ptr_or_null<int32_t>(ak), B, S, H,
                              576, 512, paged ? nblk * bs : kv.size(1), bs, nblk, topk, (float)sm_scale,
                              is_causal ? 1 : 0, ptr(out), static_cast<float*>(ptr(lse)), ptr(ws), ws_bytes,
                              stream_of(q)),
           "sparse_mla_fwd");
  return {out, lse};
}

std::tuple<at::Tensor, at::Tensor> sparse_mla_fwd_meta(const at::Tensor& q, const at::Tensor&, const at::Tensor&,
                                                       double, const c10::optional<at::Tensor>&,
                                                       const c10::optional<at::Tensor>&,
                                                       const c10::optional<at::Tensor>&, bool) {
  return {at::empty({q.size(0), q.size(1), q.size(2), 512}, q.options()),
          at::empty({q.size(0), q.size(1), q.size(2)}, q.options().dtype(at::kFloat))};
}

// ---------------------------------------------------------------- V4 sparse flash MLA (TND rows)
// q [T, H, 512]; q_start / q_len / seqused_kv [B]; caches [blocks, block_size, 1, 512] (or 3-D).
// "hca" (cmp_kv without cmp_sparse_indices) needs max_cmp, the compressed-row bound
// seqused_kv.max() // cmp_ratio that the reference API derives on the host
// (sparse_flash_mla_api.py:177): rows past it would be dropped, so it has no default.
std::tuple<at::Tensor, at::Tensor> sparse_flash_mla(
    const at::Tensor& q, const at::Tensor& ori_kv, const at::Tensor& ori_block_table, const at::Tensor& q_start,
    const at::Tensor& q_len, const at::Tensor& seqused_kv, const c10::optional<at::Tensor>& sinks,
    double softmax_scale, const c10::optional<at::Tensor>& cmp_kv, const c10::optional<at::Tensor>& cmp_block_table,
    const c10::optional<at::Tensor>& cmp_sparse_indices, int64_t cmp_ratio, int64_t ori_win_left, int64_t max_cmp) {
  require(q, "q");
  require(ori_kv, "ori_kv");
  require_on(ori_kv, q, "ori_kv");
  TORCH_CHECK(q.dim() == 3 && q.size(2) == 512, "dsa.sparse_flash_mla: q must be [T, H, 512] (got ", q.sizes(), ")");
  auto check_cache = [&](const at::Tensor& c, const char* name) {
    TORCH_CHECK((c.dim() == 4 && c.size(2) == 1 && c.size(3) == 512) || (c.dim() == 3 && c.size(2) == 512),
                "dsa.sparse_flash_mla: ", name, " must be [blocks, block_size, 1, 512] (got ", c.sizes(), ")");
    TORCH_CHECK(c.scalar_type() == q.scalar_type(), "dsa.sparse_flash_mla: ", name, " dtype must equal q dtype");
  };
  check_cache(ori_kv, "ori_kv");
  c10::OptionalDeviceGuard guard(q.device());
  const int64_t T = q.size(0), H = q.size(1), B = q_start.numel();
  TORCH_CHECK(B >= 1, "dsa.sparse_flash_mla: q_start must have one entry per batch");
  auto obt = aux_table(ori_block_table, q, B, "ori_block_table");
  auto qs = aux_i32(q_start, q, B, "q_start");
  auto ql = aux_i32(q_len, q, B, "q_len");
  auto kl = aux_i32(seqused_kv, q, B, "seqused_kv");
  auto sk = aux_f32(sinks, q, H, "sinks");
  c10::optional<at::Tensor> cbt, idx;
  int64_t K = 0, cmp_slots = 0;
  if (cmp_kv.has_value()) {
    require(*cmp_kv, "cmp_kv");
    require_on(*cmp_kv, q, "cmp_kv");
    check_cache(*cmp_kv, "cmp_kv");
    TORCH_CHECK(cmp_block_table.has_value(), "dsa.sparse_flash_mla: cmp_kv needs cmp_block_table");
    cbt = aux_table(cmp_block_table, q, B, "cmp_block_table");
    if (cmp_sparse_indices.has_value()) {
      const auto& ci = *cmp_sparse_indices;
      TORCH_CHECK(ci.dim() >= 2 && ci.size(0) == T && ci.size(-1) >= 1 && ci.numel() == T * ci.size(-1),
                  "dsa.sparse_flash_mla: cmp_sparse_indices must be [T, (1,) topk_cmp] (got ", ci.sizes(), ")");
      idx = aux_i32(cmp_sparse_indices, q, -1, "cmp_sparse_indices");
      K = ci.size(-1);
      cmp_slots = K;
    } else {
      TORCH_CHECK(max_cmp >= 0, "dsa.sparse_flash_mla: cmp_kv without cmp_sparse_indices needs max_cmp "
                  "(seqused_kv.max() // cmp_ratio)");
      cmp_slots = max_cmp;
    }
  } else {
    TORCH_CHECK(!cmp_sparse_indices.has_value(), "dsa.sparse_flash_mla: cmp_sparse_indices without cmp_kv");
  }
  auto out = at::empty({T, H, 512}, q.options());
  auto lse = at::empty({T, H}, q.options().dtype(at::kFloat));
  const size_t ws_bytes = dsa_sparse_flash_mla_workspace_size(T, H, ori_win_left, cmp_slots);
  auto ws = at::empty({(int64_t)(ws_bytes > 0 ? ws_bytes : 1)}, q.options().dtype(at::kByte));
  const at::Tensor* c = cmp_kv.has_value() ? &*cmp_kv : nullptr;
  check_rc(dsa_sparse_flash_mla(kind_of(q), ptr(q), T, H, 512, B, static_cast<int32_t*>(ptr(qs)),
                                static_cast<int32_t*>(ptr(ql)), static_cast<int32_t*>(ptr(kl)), ptr(ori_kv),
                                ori_kv.size(0), ori_kv.size(1), static_cast<int32_t*>(ptr(obt)), obt.size(1),
                                c ? ptr(*c) : nullptr, c ? c->size(0) : 0, c ? c->size(1) : 0,
                                ptr_or_null<int32_t>(cbt), cbt.has_value() ? cbt->size(1) : 0,
                                ptr_or_null<int32_t>(idx), K, cmp_ratio, ori_win_left, c ? cmp_slots : 0,
                                ptr_or_null<float>(sk), (float)softmax_scale, ptr(out), static_cast<float*>(ptr(lse)),
                                ptr(ws), ws_bytes, stream_of(q)),
           "sparse_flash_mla");
  return {out, lse};
}

std::tuple<at::Tensor, at::Tensor> sparse_flash_mla_meta(
    const at::Tensor& q, const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
    const c10::optional<at::Tensor>&, double, const c10::optional<at::Tensor>&, const c10::optional<at::Tensor>&,
    const c10::optional<at::Tensor>&, int64_t, int64_t, int64_t) {
  return {at::empty({q.size(0), q.size(1), 512}, q.options()),
          at::empty({q.size(0), q.size(1)}, q.options().dtype(at::kFloat))};
}

// ---------------------------------------------------------------- producer
std::tuple<at::Tensor, at::Tensor> act_quant(const at::Tensor& x, bool round_scale,
                                             c10::optional<at::ScalarType> dtype_opt) {
  require(x, "x");
  TORCH_CHECK(x.dim() >= 1, "dsa.act_quant: x must have at least one dimension");
  const at::ScalarType dtype = dtype_opt.value_or(at::kChar);
  TORCH_CHECK(dtype == at::kChar || dtype == at::kFloat8_e4m3fn, "dsa.act_quant: dtype must be int8 or float8_e4m3fn");
  c10::OptionalDeviceGuard guard(x.device());
  const int64_t n = x.size(-1), rows = n ? x.numel() / n : 0;
  auto y = at::empty(x.sizes(), x.options().dtype(dtype));
  auto sizes = x.sizes().vec();
  sizes.back() = 1;
  auto s = at::empty(sizes, x.options().dtype(at::kFloat));
  if (rows * n > 0)
    check_rc(dsa_act_quant(kind_of(x), ptr(x), rows, n, dtype == at::kChar ? DSA_KIND_INT8 : DSA_KIND_FP8_E4M3,
                           ptr(y), static_cast<float*>(ptr(s)), round_scale ? 1 : 0, stream_of(x)),
             "act_quant");
  return {y, s};
}

std::tuple<at::Tensor, at::Tensor> act_quant_meta(const at::Tensor& x, bool, c10::optional<at::ScalarType> dtype_opt) {
  const at::ScalarType dtype = dtype_opt.value_or(at::kChar);
  auto sizes = x.sizes().vec();
  sizes.back() = 1;
  return {at::empty(x.sizes(), x.options().dtype(dtype)), at::empty(sizes, x.options().dtype(at::kFloat))};
}

// V4 gathered-index attention with sinks (examples/deepseek_v4/sparse_attention.py:171-198):
// q [b, m, h, 512], kv [b, n, 512], attn_sink [h] fp32, topk_idxs [b, m, topk] -> (out fp32, lse fp32);
// the kernel writes its fp32 accumulator, as the reference's does.
std::tuple<at::Tensor, at::Tensor> sparse_attn(const at::Tensor& q, const at::Tensor& kv,
                                               const c10::optional<at::Tensor>& attn_sink, const at::Tensor& topk_idxs,
                                               double softmax_scale) {
  require(q, "q");
  require(kv, "kv");
  require_on(kv, q, "kv");
  TORCH_CHECK(q.dim() == 4 && kv.dim() == 3 && topk_idxs.dim() == 3, "dsa.sparse_attn: q [b,m,h,d], kv [b,n,d], "
              "topk_idxs [b,m,topk]");
  TORCH_CHECK(kv.scalar_type() == q.scalar_type(), "dsa.sparse_attn: kv dtype must equal q dtype");
  c10::OptionalDeviceGuard guard(q.device());
  const int64_t B = q.size(0), M = q.size(1), H = q.size(2), D = q.size(3), N = kv.size(1), K = topk_idxs.size(2);
  TORCH_CHECK(kv.size(0) == B && kv.size(2) == D, "dsa.sparse_attn: kv must be [", B, ", n, ", D, "] (got ",
              kv.sizes(), ")");
  TORCH_CHECK(topk_idxs.size(0) == B && topk_idxs.size(1) == M && K >= 1, "dsa.sparse_attn: topk_idxs must be [", B,
              ", ", M, ", topk] (got ", topk_idxs.sizes(), ")");
  auto idx = aux_i32(topk_idxs, q, -1, "topk_idxs");
  auto sk = aux_f32(attn_sink, q, H, "attn_sink");
  auto out = at::empty({B, M, H, D}, q.options().dtype(at::kFloat));
  auto lse = at::empty({B, M, H}, q.options().dtype(at::kFloat));
  if (B * M > 0) {
    const size_t ws_bytes = dsa_sparse_attn_sink_workspace_size(B, M, H, K);
    auto ws = at::empty({(int64_t)(ws_bytes > 0 ? ws_bytes : 1)}, q.options().dtype(at::kByte));
    check_rc(dsa_sparse_attn_sink(kind_of(q), ptr(q), ptr(kv), static_cast<int32_t*>(ptr(idx)), B, M, H, N, D, K,
                                  ptr_or_null<float>(sk), (float)softmax_scale, ptr(out),
                                  static_cast<float*>(ptr(lse)), ptr(ws), ws_bytes, stream_of(q)),
             "sparse_attn");
  }
  return {out, lse};
}

std::tuple<at::Tensor, at::Tensor> sparse_attn_meta(const at::Tensor& q, const at::Tensor&,
                                                    const c10::optional<at::Tensor>&, const at::Tensor&, double) {
  return {at::empty(q.sizes(), q.options().dtype(at::kFloat)),
          at::empty({q.size(0), q.size(1), q.size(2)}, q.options().dtype(at::kFloat))};
}

}  // namespace

TORCH_LIBRARY(dsa, m) {
  m.def("topk_select(Tensor x, int k, bool sorted=True) -> (Tensor, Tensor)");
  m.def(
      "lightning_indexer(Tensor query, Tensor key, Tensor weights, Tensor? key_scale=None, "
      "Tensor? actual_seq_lengths_query=None, Tensor? actual_seq_lengths_key=None, Tensor? block_table=None, "
      "int sparse_count=2048, int sparse_mode=3, bool return_value=False, int s2=-1) -> (Tensor, Tensor)");
  m.def(
      "sparse_mla_fwd(Tensor q, Tensor kv, Tensor indices, float sm_scale, Tensor? block_table=None, "
      "Tensor? actual_seq_lengths_query=None, Tensor? actual_seq_lengths_kv=None, bool is_causal=True) "
      "-> (Tensor, Tensor)");
  m.def(
      "sparse_flash_mla(Tensor q, Tensor ori_kv, Tensor ori_block_table, Tensor q_start, Tensor q_len, "
      "Tensor seqused_kv, Tensor? sinks, float softmax_scale, Tensor? cmp_kv=None, Tensor? cmp_block_table=None, "
      "Tensor? cmp_sparse_indices=None, int cmp_ratio=4, int ori_win_left=127, int max_cmp=-1) -> (Tensor, Tensor)");
  m.def("act_quant(Tensor x, bool round_scale=False, ScalarType? dtype=None) -> (Tensor, Tensor)");
  m.def("sparse_attn(Tensor q, Tensor kv, Tensor? attn_sink, Tensor topk_idxs, float softmax_scale) -> (Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(dsa, CUDA, m) {
  m.impl("topk_select", &topk_select);
  m.impl("lightning_indexer", &lightning_indexer);
  m.impl("sparse_mla_fwd", &sparse_mla_fwd);
  m.impl("sparse_flash_mla", &sparse_flash_mla);
  m.impl("act_quant", &act_quant);
  m.impl("sparse_attn", &sparse_attn);
}

TORCH_LIBRARY_IMPL(dsa, Meta, m) {
  m.impl("topk_select", &topk_select_meta);
  m.impl("lightning_indexer", &lightning_indexer_meta);
  m.impl("sparse_mla_fwd", &sparse_mla_fwd_meta);
  m.impl("sparse_flash_mla", &sparse_flash_mla_meta);
  m.impl("act_quant", &act_quant_meta);
  m.impl("sparse_attn", &sparse_attn_meta);
}
