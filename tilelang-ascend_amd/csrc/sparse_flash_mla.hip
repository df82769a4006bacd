// DeepSeek V4 sparse flash MLA on gfx950: the per-query-row KV row lists.
//
// V4 attention reads one paged cache of original KV rows and one of
// compressed rows (D = 512, K = V) through three access patterns
// (examples/deepseek_v4/sparse_flash_mla/sparse_flash_mla_golden.py:55-160):
//   swa  a left window over the original rows:   s_global - win_left .. s_global
//   hca  the window, then every compressed row below the row's threshold
//   csa  the window, then the top-k compressed rows it selected
// with s_global = kv_len - q_len + s and threshold = floor((s_global + 1) / cmp_ratio)
// (cmp_mask_mode 3).  csa follows the golden's walk over the selection list
// (:15-52): only its first min(K, threshold) entries are read, the first -1
// ends the list, and entries at or above the threshold are skipped.
//
// This kernel turns each query row's pattern into a list of physical rows --
// original rows as block_table[b][pos / bs] * bs + pos % bs, compressed rows
// the same through their own table and tagged kSrc2Bit -- and its length.
// The attention itself is the gather kernel of sparse_mla.hip in its 512-wide
// row-list form, with the per-head sinks in the softmax denominator.  One
// wave per query row; lists are written densely (window first), so the gather
// kernel never visits an empty tile.  A row past its batch's query length
// (padded BSND rows) gets length -1: the gather kernel writes out = 0, lse = 0
// there, as the golden leaves them.
#include "common.hpp"

namespace dsa {

hipError_t launch_sparse_mla_rows(int is_fp16, const void* q, const void* kv, const void* kv2, const int32_t* rows,
                                  const int32_t* count, int64_t T, int64_t H, int64_t cap, const float* sinks,
                                  float sm_scale, void* out, float* lse, void* workspace, hipStream_t stream);
size_t mla_workspace_bytes(int64_t tokens, int64_t H, int64_t topk);

constexpr int32_t kCmpTag = 0x40000000;  // the gather kernel's second-source bit

struct V4Args {
  const int32_t* q_start;     // [B] first query row of each batch (TND prefix or b * S)
  const int32_t* q_len;       // [B] query rows of each batch
  const int32_t* kv_len;      // [B] seqused_kv
  const int32_t* ori_bt;      // [B, ori_tl]
  const int32_t* cmp_bt;      // [B, cmp_tl] or null
  const int32_t* cmp_idx;     // [T, K] or null
  int32_t* rows;              // [T, cap]
  int32_t* count;             // [T]
  int B, T, cap;
  int ori_bs, ori_tl, ori_blocks;
  int cmp_bs, cmp_tl, cmp_blocks;
  int K, cmp_ratio, win_left, max_cmp;
  int mode;                   // 1 swa, 2 hca, 3 csa
};

// Physical row of logical position pos through a block table of tl entries;
// -1 when the table has no block there (or names one outside the pool).
__device__ __forceinline__ int32_t table_row(const int32_t* bt, int tl, int bs, int nblocks, int pos) {
  const int e = pos / bs;
  const int blk = e < tl ? bt[e] : -1;
  return (blk >= 0 && blk < nblocks) ? blk * bs + pos % bs : -1;
}

__global__ __launch_bounds__(256) void v4_row_lists_kernel(V4Args a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int t = blockIdx.x * (256 / kWave) + (int)(threadIdx.x / kWave);
  if (t >= a.T) return;
  // Batch of row t: the last b with q_start[b] <= t (q_start is non-decreasing).
  int lo = 0, hi = a.B - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a.q_start[mid] <= t) lo = mid; else hi = mid - 1;
  }
  const int b = lo;
  const int s = t - a.q_start[b];
  const int ql = a.q_len[b];
  int32_t* out = a.rows + (int64_t)t * a.cap;
  if (s < 0 || s >= ql) {
    if (lane == 0) a.count[t] = -1;
    return;
  }
  const int sg = a.kv_len[b] - ql + s;  // position of this row in its sequence
  // Window: sg - win_left .. sg, clipped at 0 (none if the row precedes the cache).
  const int nw = sg >= 0 ? min(a.win_left, sg) + 1 : 0;
  const int w0 = sg - nw + 1;
  const int32_t* obt = a.ori_bt + (int64_t)b * a.ori_tl;
  for (int i = lane; i < nw; i += kWave) out[i] = table_row(obt, a.ori_tl, a.ori_bs, a.ori_blocks, w0 + i);
  int n = nw;
  if (a.mode >= 2) {
    const int thr = sg >= 0 ? (sg + 1) / a.cmp_ratio : 0;
    const int32_t* cbt = a.cmp_bt + (int64_t)b * a.cmp_tl;
    if (a.mode == 2) {
      const int nc = min(thr, a.max_cmp);
      for (int j = lane; j < nc; j += kWave) {
        const int32_t r = table_row(cbt, a.cmp_tl, a.cmp_bs, a.cmp_blocks, j);
        out[nw + j] = r >= 0 ? (r | kCmpTag) : -1;
      }
      n += nc;
    } else {
      const int32_t* sel = a.cmp_idx + (int64_t)t * a.K;
      const int nread = min(a.K, thr);
      for (int i0 = 0; i0 < nread; i0 += kWave) {
        const int i = i0 + lane;
        const int id = i < nread ? sel[i] : -1;
        const uint64_t end = __ballot(i < nread && id == -1);
        // Entries before the first -1 of this chunk; none after it count.
        const int stop = end ? (int)__builtin_ctzll(end) : kWave;
        const bool take = lane < stop && i < nread && id >= 0 && id < thr;
        const uint64_t m = __ballot(take);
        if (take) {
          const int at = n + (int)__builtin_popcountll(m & ((1ull << lane) - 1));
          const int32_t r = table_row(cbt, a.cmp_tl, a.cmp_bs, a.cmp_blocks, id);
          out[at] = r >= 0 ? (r | kCmpTag) : -1;
        }
        n += (int)__builtin_popcountll(m);
        if (end) break;
      }
    }
  }
  if (lane == 0) a.count[t] = n;
}

// Gathered-index lists of V4's sparse_attn (examples/deepseek_v4/sparse_attention.py:171-198):
// query row t (batch t / M) attends to kv rows b * N + idx[t][j]; -1 (or an index outside
// [0, N)) is an empty slot.  One wave per row.
__global__ __launch_bounds__(256) void index_row_lists_kernel(const int32_t* __restrict__ idx, int T, int M, int N,
                                                             int K, int32_t* __restrict__ rows,
                                                             int32_t* __restrict__ count) {
  const int lane = threadIdx.x & (kWave - 1);
  const int t = blockIdx.x * (256 / kWave) + (int)(threadIdx.x / kWave);
  if (t >= T) return;
  const int64_t base = (int64_t)(t / M) * N;
  for (int j = lane; j < K; j += kWave) {
    const int id = idx[(int64_t)t * K + j];
    rows[(int64_t)t * K + j] = (id >= 0 && id < N) ? (int32_t)(base + id) : -1;
  }
  if (lane == 0) count[t] = K;
}

static size_t v4_lists_bytes(int64_t T, int64_t cap) {
  return ((size_t)T * (cap + 1) * sizeof(int32_t) + 255) & ~size_t(255);
}

size_t v4_workspace_bytes(int64_t T, int64_t H, int64_t cap) {
  return v4_lists_bytes(T, cap) + mla_workspace_bytes(T, H, cap);
}

// Caller validated shapes; cap = win_left + 1 + (hca: max_cmp, csa: K).
hipError_t launch_sparse_flash_mla(int is_fp16, const void* q, int64_t T, int64_t H, int64_t B,
                                   const int32_t* q_start, const int32_t* q_len, const int32_t* kv_len,
                                   const void* ori_kv, int64_t ori_blocks, int64_t ori_bs, const int32_t* ori_bt,
                                   int64_t ori_tl, const void* cmp_kv, int64_t cmp_blocks, int64_t cmp_bs,
                                   const int32_t* cmp_bt, int64_t cmp_tl, const int32_t* cmp_idx, int64_t K,
                                   int64_t cmp_ratio, int64_t win_left, int64_t max_cmp, int mode, int64_t cap,
                                   const float* sinks, float sm_scale, void* out, float* lse, void* workspace,
                                   hipStream_t stream) {
  if (T == 0 || H == 0) return hipSuccess;
  V4Args a;
  a.q_start = q_start;
  a.q_len = q_len;
  a.kv_len = kv_len;
  a.ori_bt = ori_bt;
  a.cmp_bt = cmp_bt;
  a.cmp_idx = cmp_idx;
  a.count = static_cast<int32_t*>(workspace);
  a.rows = a.count + T;
  a.B = (int)B;
  a.T = (int)T;
  a.cap = (int)cap;
  a.ori_bs = (int)ori_bs;
  a.ori_tl = (int)ori_tl;
  a.ori_blocks = (int)ori_blocks;
  a.cmp_bs = (int)cmp_bs;
  a.cmp_tl = (int)cmp_tl;
  a.cmp_blocks = (int)cmp_blocks;
  a.K = (int)K;
  a.cmp_ratio = (int)cmp_ratio;
  a.win_left = (int)win_left;
  a.max_cmp = (int)max_cmp;
  a.mode = mode;
  const int per_block = 256 / kWave;
  hipLaunchKernelGGL(v4_row_lists_kernel, dim3((unsigned)((T + per_block - 1) / per_block)), dim3(256), 0, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  void* mla_ws = static_cast<uint8_t*>(workspace) + v4_lists_bytes(T, cap);
  return launch_sparse_mla_rows(is_fp16, q, ori_kv, cmp_kv, a.rows, a.count, T, H, cap, sinks, sm_scale, out, lse,
                                mla_ws, stream);
}

size_t sparse_attn_sink_workspace_bytes(int64_t T, int64_t H, int64_t K) { return v4_workspace_bytes(T, H, K); }

// Caller validated: D = 512, H % 16 == 0, B * N < 2^30, T = B * M < 2^31 / (K + 1).
hipError_t launch_sparse_attn_sink(int is_fp16, const void* q, const void* kv, const int32_t* idx, int64_t B,
                                   int64_t M, int64_t H, int64_t N, int64_t K, const float* sinks, float sm_scale,
                                   void* out, float* lse, void* workspace, hipStream_t stream) {
  const int64_t T = B * M;
  if (T == 0 || H == 0) return hipSuccess;
  int32_t* count = static_cast<int32_t*>(workspace);
  int32_t* rows = count + T;
  const int per_block = 256 / kWave;
  hipLaunchKernelGGL(index_row_lists_kernel, dim3((unsigned)((T + per_block - 1) / per_block)), dim3(256), 0, stream,
                     idx, (int)T, (int)M, (int)N, (int)K, rows, count);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  void* mla_ws = static_cast<uint8_t*>(workspace) + v4_lists_bytes(T, K);
  return launch_sparse_mla_rows(is_fp16, q, kv, nullptr, rows, count, T, H, K, sinks, sm_scale, out, lse, mla_ws,
                                stream);
}

}  // namespace dsa
