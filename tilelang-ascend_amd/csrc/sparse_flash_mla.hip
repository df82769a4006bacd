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
                                  float sm_scale, void* out, float* lse, void* workspace, hipStream_t stream,
                                  int out_f32);
size_t mla_workspace_bytes(int64_t tokens, int64_t H, int64_t topk, bool f32);

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

// ---------------------------------------------------------------------------
// Decode-shaped row lists (at most kDecodeRows query rows, at most
// kDecodeMaxSlots slots): one workgroup per (query row, 16 heads, chunk of
// slots), its four waves splitting the chunk into 16-slot blocks (wave w takes
// blocks w, w + 4, ...), each with its own online softmax and O, merged in LDS
// at the end.  A list of at most kDecSingle slots is one chunk, and the
// workgroup writes the output: no partials and no combine launch, since such a
// call is a chain of latencies.  Longer lists are cut into kDecChunk-slot
// chunks (more CUs, fewer blocks per wave) whose partials a small combine
// kernel merges.  For V4 rows the kernel also derives the row lists itself
// (the window, then the compressed rows: hca every one below the row's
// threshold, csa the selection's entries before its first -1 that lie below
// the threshold), so no list kernel runs.  csa slots are not compacted: a
// skipped entry is a masked slot, which changes only the order of the softmax
// sums.
//
// A wave looks up the rows of four of its blocks at once (lane 16 j + u: slot
// u of its j-th block of the group) and keeps two blocks in LDS: the DMA of
// block i + 1 is issued before block i is waited for and multiplied.  A
// block's 16 rows (1 KB each, K = V) go to 16 KB of LDS, one row per DMA
// instruction, lane l carrying 16-byte chunk l ^ 2u of row u (so the Q K^T
// operand reads, 16 rows at one chunk, fall on distinct banks).
// S^T = K Q^T by 16x16x32 MFMAs (lane (g, r): keys 4g + i of head r), then
// O^T += V^T P^T by 16x16x16 MFMAs whose V^T operand comes from
// ds_read_b64_tr_b16 and whose P operand is the lane's own four scores.  As in
// the gather kernel, O is normalised by the sum of the 16-bit-rounded P, the
// LSE by the exact sum, and the sinks join the denominator.
constexpr int kDecBlk = 16;
constexpr int64_t kDecodeRows = 8;
// ... and at most this many slots per row.  Longer lists go through the split
// gather kernel.
constexpr int64_t kDecodeMaxSlots = 1024;
// Up to kDecSingle slots one workgroup per (row, 16 heads) takes them all and
// writes the output; longer lists are cut into chunks of kDecChunk slots, one
// workgroup each (grid z), whose fp32 partials (O unnormalised, its max, exact
// and rounded sums) v4_decode_combine_kernel merges.
constexpr int kDecSingle = 256;
constexpr int kDecChunk = 128;
static_assert(kDecSingle % 64 == 0 && kDecChunk % 64 == 0, "whole blocks per wave");
constexpr float kDecSlack = 8.f;
constexpr int kDecPart = 516;  // floats per (row, head, chunk): O[512], max, sum, rounded sum, pad
// Row-lookup groups per wave: four of its blocks each.
constexpr int kDecGroups = ((kDecSingle > kDecChunk ? kDecSingle : kDecChunk) / 64 + 3) / 4;
// One block of rows in LDS: 16 rows x 1 KB (K = V), then for 576-wide rows
// (sparse MLA: 512 latent + 64 rope) their 128-byte tails, 16 x 128 B.
template <int kD>
constexpr int dec_blk_lds() { return kDecBlk * 1024 + (kD == 576 ? kDecBlk * 128 : 0); }
constexpr int kDecOBytes = 4 * 512 * 16 * 4;  // the four waves' O^T, fp32 (aliases the 4 x 2 blocks)
// LDS of the kernel: the 4 waves' two blocks, or the merge's O^T + m, l, rounded l per wave and head.
template <int kD>
constexpr int dec_lds() {
  return 8 * dec_blk_lds<kD>() > kDecOBytes + 3 * 4 * 16 * 4 ? 8 * dec_blk_lds<kD>() : kDecOBytes + 3 * 4 * 16 * 4;
}

struct DecArgs {
  const uint16_t* q;      // [T, H, 512]
  const uint8_t* kv;      // rows of 1 KB
  const uint8_t* kv2;     // rows tagged kCmpTag, or null
  const int32_t* rows;    // [T, cap]
  const int32_t* count;   // [T]; -1: padded row
  const float* sinks;     // [H] or null
  uint16_t* out;          // [T, H, 512]
  float* out32;           // [T, H, 512] fp32 instead of out, or null
  float* lse;             // [T, H]
  int T, H, cap;
  int chunk, nsplit;      // slots per workgroup, workgroups per (row, 16 heads)
  float* part;            // [T, H, nsplit, kDecPart] when nsplit > 1
  float scale_log2;
  // V4 rows whose lists the kernel derives (kMode 1..3): the row's batch, window
  // and compressed rows, as v4_row_lists_kernel computes them.
  V4Args v4;
  // Sparse MLA decode rows (kMode 4): query row t = b * S + s attends to the KV
  // rows of indices[t][j] (paged through the block table, or b * Skv + idx).
  struct {
    const int32_t* idx;          // [T, cap]
    const int32_t* block_table;  // [B, max_blocks] or null
    const int32_t* q_len;        // [B] or null (S)
    const int32_t* kv_len;       // [B] or null (Skv)
    // KV groups: row t = (b * S + s) * G + g reads KV column g, physical row
    // (pool row) * G + g.
    int S, G, Skv, block_size, max_blocks, causal;
  } mla;
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void dec_lds_void;
typedef const __attribute__((address_space(1))) void dec_gbl_void;

template <bool kF16>
__device__ __forceinline__ f32x4 dec_mfma_qk(const u32x4& a, const u32x4& b, const f32x4& c) {
  if constexpr (kF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <bool kF16>
__device__ __forceinline__ f32x4 dec_mfma_pv(const s16x4& a, const s16x4& b, const f32x4& c) {
  if constexpr (kF16)
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// s_waitcnt with only vmcnt constrained (expcnt, lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void dec_wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ uint32_t dec_lds_u32(const void* p) {
  return (uint32_t)(uintptr_t)(const dec_lds_void*)p;
}

// ds_read_b64_tr_b16 as inline asm: through the builtin the compiler waits for
// every outstanding DMA (the next block's included) before each read.
// Completion is tracked explicitly with dec_lgkm_wait.
__device__ __forceinline__ void dec_tr_read(u32x2& out, uint32_t lds_addr) {
  __asm__ __volatile__("ds_read_b64_tr_b16 %0, %1" : "=v"(out) : "v"(lds_addr));
}

__device__ __forceinline__ void dec_b128_read(u32x4& out, uint32_t lds_addr) {
  __asm__ __volatile__("ds_read_b128 %0, %1" : "=v"(out) : "v"(lds_addr));
}

// Wait until at most N LDS operations are outstanding; the eight values pass
// through the asm so no use of them can be scheduled before the wait.
template <int N, typename V>
__device__ __forceinline__ void dec_lgkm_wait(V (&v)[8]) {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  __asm__ __volatile__("s_waitcnt lgkmcnt(%8)"
                       : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7])
                       : "i"(N));
}

template <int N, typename V>
__device__ __forceinline__ void dec_lgkm_wait(V (&v)[2]) {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  __asm__ __volatile__("s_waitcnt lgkmcnt(%2)" : "+v"(v[0]), "+v"(v[1]) : "i"(N));
}

// Max and sum over the four lane groups of 16 (lanes r, r + 16, r + 32, r + 48),
// by lane swaps rather than LDS permutes (which would wait for the pending LDS reads).
__device__ __forceinline__ float dec_max_across_groups(float x) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
  const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}

__device__ __forceinline__ float dec_sum_across_groups(float x) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// One 16-bit value of p (round to nearest even) and its value back in fp32.
template <bool kF16>
__device__ __forceinline__ short dec_round(float p, float& back) {
  if constexpr (kF16) {
    const _Float16 h = (_Float16)p;
    back = (float)h;
    return __builtin_bit_cast(short, h);
  } else {
    const __bf16 h = (__bf16)p;
    back = (float)h;
    return __builtin_bit_cast(short, h);
  }
}

// kMode: 0 row lists given (rows / count), 1 swa, 2 hca, 3 csa (lists derived
// here), 4 sparse MLA index rows (kD = 576: K is the whole row, V its first 512).
template <bool kF16, int kMode, int kD = 512>
__global__ __launch_bounds__(256) void v4_decode_rows_kernel(DecArgs a) {
  static_assert(kD == 512 || (kD == 576 && kMode == 4), "576-wide rows: sparse MLA index rows");
  constexpr int kBlkLds = dec_blk_lds<kD>();
  constexpr int kSteps = kD / 32;                      // Q K^T steps of 32 dims
  constexpr int kDmaPerBlk = kD == 576 ? kDecBlk + 2 : kDecBlk;  // DMA instructions per block
  extern __shared__ __align__(16) uint8_t lds[];
  const int t = blockIdx.x;
  const int h0 = blockIdx.y * 16;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int r = lane & 15, g = lane >> 4;
  const int s_lo = blockIdx.z * a.chunk;  // this workgroup's slots: s_lo .. s_lo + chunk - 1
  // Q^T operands: head h0 + r, dims 32 st + 8g .. +7 (loaded first: they need no row list).
  u32x4 qb[kSteps];
  const uint16_t* qp = a.q + ((int64_t)t * a.H + h0 + r) * kD + 8 * g;
#pragma unroll
  for (int st = 0; st < kSteps; ++st) qb[st] = *reinterpret_cast<const u32x4*>(qp + 32 * st);
  int cnt_raw, vb = 0, vnw = 0, vw0 = 0, thr = 0, nread = 0;
  const V4Args& v = a.v4;
  int mb = 0, mg = 0, mkl = 0, mlim = 0;  // kMode 4: batch, KV group, kv length, causal bound of the row
  if constexpr (kMode == 4) {
    // A row past its batch's query length has no valid slot (out 0, lse -inf, as
    // the gather kernel gives it); a slot is valid iff 0 <= idx < kv_len and, when
    // causal, idx <= kv_len - q_len + s.
    const int bs_row = t / a.mla.G;
    mg = t - bs_row * a.mla.G;
    mb = bs_row / a.mla.S;
    const int sq = bs_row - mb * a.mla.S;
    const int ql = min(max(a.mla.q_len ? a.mla.q_len[mb] : a.mla.S, 0), a.mla.S);
    mkl = min(max(a.mla.kv_len ? a.mla.kv_len[mb] : a.mla.Skv, 0), a.mla.Skv);
    mlim = a.mla.causal ? mkl - ql + sq : 0x7fffffff;
    cnt_raw = sq < ql ? a.cap : 0;
  } else if constexpr (kMode != 0) {
    // Batch of row t: the last b with q_start[b] <= t (0 if none).  Past one batch,
    // 64 batches per step, each lane loading its batch's start, query length and
    // kv length at once.
    int qsb = 0, qlb = 0, klb = 0;
    if (v.B == 1) {
      qsb = v.q_start[0];
      qlb = v.q_len[0];
      klb = v.kv_len[0];
    }
    for (int b0 = 0; v.B > 1 && b0 < v.B; b0 += kWave) {
      const int b = b0 + lane;
      const bool in = b < v.B;
      const int qs = in ? v.q_start[b] : 0, ql = in ? v.q_len[b] : 0, kl = in ? v.kv_len[b] : 0;
      const uint64_t le = __builtin_amdgcn_ballot_w64(in && qs <= t);
      if (b0 == 0 || le) {
        const int j = le ? 63 - __builtin_clzll(le) : 0;
        vb = b0 + j;
        qsb = __builtin_amdgcn_readlane(qs, j);
        qlb = __builtin_amdgcn_readlane(ql, j);
        klb = __builtin_amdgcn_readlane(kl, j);
      }
    }
    const int sq = t - qsb;
    if (sq < 0 || sq >= qlb) {
      cnt_raw = -1;
    } else {
      const int sg = klb - qlb + sq;  // position of this row in its sequence
      vnw = sg >= 0 ? min(v.win_left, sg) + 1 : 0;
      vw0 = sg - vnw + 1;
      thr = (kMode >= 2 && sg >= 0) ? (sg + 1) / v.cmp_ratio : 0;
      // csa: min(K, thr) entries of the selection are read (fewer if one is -1, found below).
      nread = kMode == 3 ? min(v.K, thr) : 0;
      cnt_raw = vnw + (kMode == 2 ? min(thr, v.max_cmp) : nread);
    }
  } else {
    cnt_raw = a.count[t];
  }
  if (cnt_raw < 0) {  // padded query row: out 0, lse 0 (workgroup-uniform)
    if (a.nsplit > 1) {  // chunk 0 marks it (sum -1) for the combine
      if (blockIdx.z == 0 && tid < 16) a.part[((int64_t)t * a.H + h0 + tid) * a.nsplit * kDecPart + 513] = -1.f;
      return;
    }
    for (int e = tid; e < 16 * 64; e += 256) {
      const int64_t at = ((int64_t)t * a.H + h0 + e / 64) * 512 + 8 * (e % 64);
      if (a.out32) {
        *reinterpret_cast<f32x4*>(a.out32 + at) = f32x4{0.f, 0.f, 0.f, 0.f};
        *reinterpret_cast<f32x4*>(a.out32 + at + 4) = f32x4{0.f, 0.f, 0.f, 0.f};
      } else {
        *reinterpret_cast<u32x4*>(a.out + at) = u32x4{0, 0, 0, 0};
      }
    }
    if (tid < 16) a.lse[(int64_t)t * a.H + h0 + tid] = 0.f;
    return;
  }
  int cnt = min(cnt_raw, a.cap);
  const int32_t* rowl = a.rows + (int64_t)t * a.cap;
  // Physical row of slot i < cnt (kCmpTag on compressed rows), -1 for an empty slot.
  auto row_of = [&](int i) -> int32_t {
    if constexpr (kMode == 0) {
      return rowl[i];
    } else if constexpr (kMode == 4) {
      const int idx = a.mla.idx[(int64_t)t * a.cap + i];
      const bool ok = idx >= 0 && idx < mkl && idx <= mlim;
      if (a.mla.block_table) {
        const int blk = a.mla.block_table[(int64_t)mb * a.mla.max_blocks + (ok ? idx / a.mla.block_size : 0)];
        return ok ? (blk * a.mla.block_size + idx % a.mla.block_size) * a.mla.G + mg : -1;
      }
      return ok ? (mb * a.mla.Skv + idx) * a.mla.G + mg : -1;
    } else {
      // Window position vw0 + i, then compressed entry i - vnw: the lookups of both
      // go out (from clamped entries) and the slot picks one.
      const int pw = max(vw0 + i, 0), ew = pw / v.ori_bs;
      const int bw = v.ori_bt[(int64_t)vb * v.ori_tl + min(ew, v.ori_tl - 1)];
      int pc = max(i - vnw, 0);
      bool ok = true;
      if constexpr (kMode == 3) {
        const int id = v.cmp_idx[(int64_t)t * v.K + min(pc, v.K - 1)];
        ok = id >= 0 && id < thr;
        pc = ok ? id : 0;
      }
      int32_t rc = -1;
      if constexpr (kMode >= 2) {
        const int ec = pc / v.cmp_bs;
        const int bc = v.cmp_bt[(int64_t)vb * v.cmp_tl + min(ec, v.cmp_tl - 1)];
        rc = (ok && ec < v.cmp_tl && bc >= 0 && bc < v.cmp_blocks) ? ((bc * v.cmp_bs + pc % v.cmp_bs) | kCmpTag) : -1;
      }
      const int32_t rw = (ew < v.ori_tl && bw >= 0 && bw < v.ori_blocks) ? bw * v.ori_bs + pw % v.ori_bs : -1;
      return i < vnw ? rw : rc;
    }
  };
  // The wave's blocks are wave, wave + 4, ...; its block i sits in group i / 4, whose
  // rows are looked up together (lane 16 j + u: slot u of the group's block j), all
  // groups before the first DMA.
  auto slot_of = [&](int grp) { return s_lo + (wave + 4 * (4 * grp + (lane >> 4))) * kDecBlk + (lane & 15); };
  // csa: the first 512 entries of the selection go out with the lookups.
  constexpr bool csa = kMode == 3;
  const int32_t* sel = csa ? v.cmp_idx + (int64_t)t * v.K : nullptr;
  int32_t e0[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (csa && nread > 0) {  // loads from clamped entries, so none waits on a lane branch
#pragma unroll
    for (int j = 0; j < 8; ++j) e0[j] = sel[min(j * kWave + lane, nread - 1)];
  }
  int32_t rowg[kDecGroups];
#pragma unroll
  for (int k = 0; k < kDecGroups; ++k) {
    const int slot = slot_of(k);
    rowg[k] = -1;
    if (s_lo + (wave + 16 * k) * kDecBlk < cnt) rowg[k] = row_of(min(slot, cnt - 1));  // wave-uniform test
  }
  if constexpr (csa) {
    // The selection's first -1 among its first nread entries ends it.
    int f = nread;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint64_t end = __builtin_amdgcn_ballot_w64(e0[j] == -1 && j * kWave + lane < nread);
      if (end && f == nread) f = j * kWave + (int)__builtin_ctzll(end);
    }
    for (int i0 = 8 * kWave; i0 < nread && f == nread; i0 += 8 * kWave) {
      int32_t e[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = i0 + j * kWave + lane;
        e[j] = i < nread ? sel[i] : 0;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint64_t end = __builtin_amdgcn_ballot_w64(e[j] == -1);
        if (end && f == nread) f = i0 + j * kWave + (int)__builtin_ctzll(end);
      }
    }
    cnt = min(vnw + f, cnt);
  }
  f32x4 o[32];
#pragma unroll
  for (int c = 0; c < 32; ++c) o[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -__builtin_huge_valf(), l = 0.f, lr = 0.f;
  uint8_t* wbuf = lds + wave * (2 * kBlkLds);
  const int s_hi = min(cnt, s_lo + a.chunk);
  const int nblk = s_hi > s_lo ? (s_hi - s_lo + kDecBlk - 1) / kDecBlk : 0;
  // DMA of the wave's block i to bp; returns its valid-slot mask.  rowg[0] holds
  // block i's group: the groups shift down when block i starts one.
  auto load = [&](int i, uint8_t* bp) -> uint32_t {
    const int k = i >> 2, j = i & 3;
    if (j == 0 && k > 0) {
#pragma unroll
      for (int kk = 0; kk + 1 < kDecGroups; ++kk) rowg[kk] = rowg[kk + 1];
    }
    const int32_t rows = rowg[0];
    const bool valid = rows >= 0 && slot_of(k) < cnt;
    const uint32_t vmask = (uint32_t)(__builtin_amdgcn_ballot_w64(valid) >> (16 * j)) & 0xffffu;
    const int32_t rz = valid ? rows : 0;  // empty slots read row 0 (their scores are masked)
    constexpr int kRowBytes = kD * 2;
#pragma unroll
    for (int u = 0; u < kDecBlk; ++u) {
      const int ru = __builtin_amdgcn_readlane(rz, 16 * j + u);
      // Index rows (kMode 4) use all 31 bits; V4 lists tag compressed rows.
      const uint8_t* base = (kMode != 4 && (ru & kCmpTag)) ? a.kv2 : a.kv;
      const int64_t pr = kMode == 4 ? (int64_t)ru : (int64_t)(ru & ~kCmpTag);
      const uint8_t* src = base + pr * kRowBytes + 16 * (lane ^ (2 * u));
      __builtin_amdgcn_global_load_lds((dec_gbl_void*)src, (dec_lds_void*)(bp + u * 1024), 16, 0, 0);
    }
    if constexpr (kD == 576) {
      // The rows' 128-byte tails: instruction q carries rows 8q .. 8q + 7, lane l chunk
      // (l % 8) ^ f(u) of row u = 8q + l / 8 to slot l % 8, f(u) = 2 ((u / 4) % 4), so the
      // Q K^T reads of a half-wave (16 rows, two chunks each) fall on distinct banks.
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int ruq = __shfl(rz, 16 * j + 8 * q + (lane >> 3), kWave);
        const int u = 8 * q + (lane >> 3);
        const int c = (lane & 7) ^ (2 * ((u >> 2) & 3));
        const uint8_t* src = a.kv + (int64_t)ruq * kRowBytes + 1024 + 16 * c;
        __builtin_amdgcn_global_load_lds((dec_gbl_void*)src, (dec_lds_void*)(bp + kDecBlk * 1024 + q * 1024), 16, 0, 0);
      }
    }
    return vmask;
  };
  const int vrow = 4 * g + (r >> 2);
  auto process = [&](const uint8_t* bp, uint32_t vmask) {
    // S^T = K Q^T: A = K rows r (chunk 4 st + g), B = Q^T; the first two groups of V^T
    // reads (below) go out behind the K reads.
    const uint32_t kb0 = dec_lds_u32(bp) + r * 1024;
    u32x4 kr[2][8];
#pragma unroll
    for (int st = 0; st < 16; ++st) dec_b128_read(kr[st >> 3][st & 7], kb0 + 16 * ((4 * st + g) ^ (2 * r)));
    // 576-wide rows: steps 16 and 17 from the tails (row r, chunk 4 (st - 16) + g, stored at slot chunk ^ f(r)).
    u32x4 krt[2];
    const uint32_t kt0 = dec_lds_u32(bp) + kDecBlk * 1024 + r * 128;
    // O^T += V^T P^T: lane (g, L) feeds row 4g + L / 4, columns 16 c + 4 (L % 4) .. +3,
    // i.e. chunk (2c + (L % 4) / 2) ^ 2 vrow of the row, at bytes vb0 + 32 (c ^ vrow).
    const uint32_t vb0 = dec_lds_u32(bp) + vrow * 1024 + 16 * ((r & 3) >> 1) + 8 * (r & 1);
    u32x2 va[4][8];
    auto reads = [&](int grp) {
#pragma unroll
      for (int k = 0; k < 8; ++k) dec_tr_read(va[grp][k], vb0 + 32 * ((8 * grp + k) ^ vrow));
    };
    f32x4 sc = {0.f, 0.f, 0.f, 0.f};
    dec_lgkm_wait<8>(kr[0]);
#pragma unroll
    for (int st = 0; st < 8; ++st) sc = dec_mfma_qk<kF16>(kr[0][st], qb[st], sc);
    // LDS reads retire in issue order: the wait for kr[1] must count the reads
    // issued after it (the two tails, or the first eight V^T reads), since with
    // nothing behind kr[1] a count of 8 would not wait for it at all.
    if constexpr (kD == 576) {
#pragma unroll
      for (int q = 0; q < 2; ++q) dec_b128_read(krt[q], kt0 + 16 * ((4 * q + g) ^ (2 * ((r >> 2) & 3))));
      dec_lgkm_wait<2>(kr[1]);
    } else {
      reads(0);
      dec_lgkm_wait<8>(kr[1]);
    }
#pragma unroll
    for (int st = 0; st < 8; ++st) sc = dec_mfma_qk<kF16>(kr[1][st], qb[8 + st], sc);
    if constexpr (kD == 576) {
      reads(0);
      dec_lgkm_wait<8>(krt);
#pragma unroll
      for (int q = 0; q < 2; ++q) sc = dec_mfma_qk<kF16>(krt[q], qb[16 + q], sc);
    }
    reads(1);
    float s2[4], bm = -__builtin_huge_valf();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s2[i] = ((vmask >> (4 * g + i)) & 1u) ? sc[i] * a.scale_log2 : -__builtin_huge_valf();
      bm = fmaxf(bm, s2[i]);
    }
    bm = dec_max_across_groups(bm);
    // The reference max moves only when a score passes it by more than kDecSlack
    // (p <= 2^kDecSlack then), so O is seldom rescaled.  Both -inf (nothing valid
    // yet): alpha 1 and every p 0, with no inf - inf.
    const float mn = (m == -__builtin_huge_valf() || bm > m + kDecSlack) ? fmaxf(m, bm) : m;
    const float alpha = m == mn ? 1.f : fast_exp2(m - mn);
    // O is still 0 while m is -inf; otherwise it is rescaled when some head's max moved.
    if (__builtin_amdgcn_ballot_w64(m != mn && m != -__builtin_huge_valf())) {
#pragma unroll
      for (int c = 0; c < 32; ++c) o[c] *= alpha;
    }
    m = mn;
    l *= alpha;
    lr *= alpha;
    s16x4 pb;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = s2[i] == -__builtin_huge_valf() ? 0.f : fast_exp2(s2[i] - mn);
      float back;
      pb[i] = dec_round<kF16>(p, back);
      l += p;
      lr += back;
    }
    auto mfmas = [&](int grp) {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        o[8 * grp + k] = dec_mfma_pv<kF16>(__builtin_bit_cast(s16x4, va[grp][k]), pb, o[8 * grp + k]);
    };
    dec_lgkm_wait<8>(va[0]);
    mfmas(0);
    reads(2);
    dec_lgkm_wait<8>(va[1]);
    mfmas(1);
    reads(3);
    dec_lgkm_wait<8>(va[2]);
    mfmas(2);
    dec_lgkm_wait<0>(va[3]);
    mfmas(3);
  };
  // Block i of the wave goes to buffer i % 2; the DMA of block i + 1 is issued
  // before block i is waited for.
  const int nmine = nblk > wave ? (nblk - 1 - wave) / 4 + 1 : 0;
  // Q and the lookups have landed before the first DMA (the lookups are needed for
  // it): waiting here once keeps the compiler from waiting, inside the loop, for a
  // Q register it loaded -- a wait that would also drain the next block's DMA.
  dec_wait_vmcnt<0>();
  uint32_t vm = nmine > 0 ? load(0, wbuf) : 0u;
  for (int i = 0; i < nmine; ++i) {
    uint32_t vn = 0;
    if (i + 1 < nmine) {
      vn = load(i + 1, wbuf + ((i + 1) & 1) * kBlkLds);
      dec_wait_vmcnt<kDmaPerBlk>();  // block i is in LDS, block i + 1 in flight
    } else {
      dec_wait_vmcnt<0>();
    }
    process(wbuf + (i & 1) * kBlkLds, vm);
    vm = vn;
  }
  l = dec_sum_across_groups(l);
  lr = dec_sum_across_groups(lr);
  __syncthreads();  // every wave is done with its block buffers
  // Wave w's O^T: f32x4 (c * 64 + lane) of its area holds head r, columns 16 c + 4 g .. +3.
  f32x4* ow = reinterpret_cast<f32x4*>(lds) + wave * (32 * 64);
#pragma unroll
  for (int c = 0; c < 32; ++c) ow[c * 64 + lane] = o[c];
  float* stats = reinterpret_cast<float*>(lds + kDecOBytes);  // [3][4 waves][16 heads]
  if (g == 0) {
    stats[wave * 16 + r] = m;
    stats[64 + wave * 16 + r] = l;
    stats[128 + wave * 16 + r] = lr;
  }
  __syncthreads();
  // Merge: thread tid takes head h = tid % 16 and the f32x4 items tid + 256 j (j < 8)
  // of every wave's area: columns 4 q .. 4 q + 3, q = tid / 16 + 16 j.  A chunk's
  // workgroup leaves the sinks to the combine and writes its partial instead.
  const f32x4* of = reinterpret_cast<const f32x4*>(lds);
  const bool split = a.nsplit > 1;
  const int h = tid & 15;
  float mw[4], mx = -__builtin_huge_valf();
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    mw[w] = stats[w * 16 + h];
    mx = fmaxf(mx, mw[w]);
  }
  const float sink2 = a.sinks && !split ? a.sinks[h0 + h] * 1.4426950408889634f : -__builtin_huge_valf();
  const float mm = fmaxf(mx, sink2);
  float den = 0.f, den_r = 0.f, wgt[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    wgt[w] = mm == -__builtin_huge_valf() ? 0.f : fast_exp2(mw[w] - mm);
    den += stats[64 + w * 16 + h] * wgt[w];
    den_r += stats[128 + w * 16 + h] * wgt[w];
  }
  const int64_t th = (int64_t)t * a.H + h0 + h;
  // sum_w wgt[w] O_w for item j.
  auto merged = [&](int j) -> f32x4 {
    const int item = tid + 256 * j;
    f32x4 acc = of[item] * wgt[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) acc += of[w * (32 * 64) + item] * wgt[w];
    return acc;
  };
  if (split) {
    float* pp = a.part + (th * a.nsplit + blockIdx.z) * kDecPart;
#pragma unroll
    for (int j = 0; j < 8; ++j) *reinterpret_cast<f32x4*>(pp + 4 * ((tid + 256 * j) >> 4)) = merged(j);
    if (tid < 16) {
      pp[512] = mm;
      pp[513] = den;
      pp[514] = den_r;
    }
    return;
  }
  const float es = a.sinks && mm != -__builtin_huge_valf() ? fast_exp2(sink2 - mm) : 0.f;
  den += es;
  den_r += es;
  const float inv = den_r > 0.f ? 1.f / den_r : 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int item = tid + 256 * j;
    const f32x4 acc = merged(j) * inv;
    if (a.out32) {
      *reinterpret_cast<f32x4*>(a.out32 + th * 512 + 4 * (item >> 4)) = acc;
      continue;
    }
    uint32_t pk[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      if constexpr (kF16) {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        const h2 hv = {(_Float16)acc[2 * k], (_Float16)acc[2 * k + 1]};
        pk[k] = __builtin_bit_cast(uint32_t, hv);
      } else {
        pk[k] = pack_bf16x2(acc[2 * k], acc[2 * k + 1]);
      }
    }
    *reinterpret_cast<u32x2*>(a.out + th * 512 + 4 * (item >> 4)) = u32x2{pk[0], pk[1]};
  }
  if (tid < 16) a.lse[th] = den > 0.f ? (mm + fast_log2(den)) * 0.69314718055994531f : -__builtin_huge_valf();
}

// Merge of the chunk partials: thread = (row, head, 8 columns); the sinks join
// the denominator here.  A row whose chunk 0 carries sum -1 is padded: out 0, lse 0.
template <bool kF16>
__global__ __launch_bounds__(256) void v4_decode_combine_kernel(const float* __restrict__ part,
                                                                const float* __restrict__ sinks, int TH, int H,
                                                                int nsplit, uint16_t* __restrict__ out,
                                                                float* __restrict__ out32, float* __restrict__ lse) {
  const int hh = blockIdx.x * 4 + (int)(threadIdx.x / 64);  // row * H + head
  if (hh >= TH) return;
  const int c8 = 8 * (threadIdx.x % 64);
  const float* base = part + (int64_t)hh * nsplit * kDecPart;
  uint16_t* op = out + (int64_t)hh * 512 + c8;
  float* op32 = out32 ? out32 + (int64_t)hh * 512 + c8 : nullptr;
  if (base[513] < 0.f) {
    if (op32) {
      *reinterpret_cast<f32x4*>(op32) = f32x4{0.f, 0.f, 0.f, 0.f};
      *reinterpret_cast<f32x4*>(op32 + 4) = f32x4{0.f, 0.f, 0.f, 0.f};
    } else {
      *reinterpret_cast<u32x4*>(op) = u32x4{0, 0, 0, 0};
    }
    if (c8 == 0) lse[hh] = 0.f;
    return;
  }
  // Chunks kU at a time, every load of a group issued before any is used.
  constexpr int kU = 4;
  const float sink2 = sinks ? sinks[hh % H] * 1.4426950408889634f : -__builtin_huge_valf();
  float mm = sink2;
  for (int z0 = 0; z0 < nsplit; z0 += kU) {
    float mz[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) mz[u] = z0 + u < nsplit ? base[(z0 + u) * kDecPart + 512] : -__builtin_huge_valf();
#pragma unroll
    for (int u = 0; u < kU; ++u) mm = fmaxf(mm, mz[u]);
  }
  float den = 0.f, den_r = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int z0 = 0; z0 < nsplit; z0 += kU) {
    f32x4 st[kU], lo[kU], hi[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const float* pz = base + min(z0 + u, nsplit - 1) * kDecPart;  // clamped: a real partial, unused past nsplit
      st[u] = *reinterpret_cast<const f32x4*>(pz + 512);          // max, sum, rounded sum, pad
      lo[u] = *reinterpret_cast<const f32x4*>(pz + c8);
      hi[u] = *reinterpret_cast<const f32x4*>(pz + c8 + 4);
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (z0 + u >= nsplit || st[u][0] == -__builtin_huge_valf()) continue;  // past the chunks / no valid slot
      const float w = fast_exp2(st[u][0] - mm);
      den += st[u][1] * w;
      den_r += st[u][2] * w;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc[k] += lo[u][k] * w;
        acc[4 + k] += hi[u][k] * w;
      }
    }
  }
  const float es = sinks && mm != -__builtin_huge_valf() ? fast_exp2(sink2 - mm) : 0.f;
  den += es;
  den_r += es;
  const float inv = den_r > 0.f ? 1.f / den_r : 0.f;
  if (c8 == 0) lse[hh] = den > 0.f ? (mm + fast_log2(den)) * 0.69314718055994531f : -__builtin_huge_valf();
  if (op32) {
    *reinterpret_cast<f32x4*>(op32) = f32x4{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
    *reinterpret_cast<f32x4*>(op32 + 4) = f32x4{acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv};
    return;
  }
  uint32_t pk[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (kF16) {
      typedef _Float16 h2 __attribute__((ext_vector_type(2)));
      const h2 hv = {(_Float16)(acc[2 * j] * inv), (_Float16)(acc[2 * j + 1] * inv)};
      pk[j] = __builtin_bit_cast(uint32_t, hv);
    } else {
      pk[j] = pack_bf16x2(acc[2 * j] * inv, acc[2 * j + 1] * inv);
    }
  }
  *reinterpret_cast<u32x4*>(op) = u32x4{pk[0], pk[1], pk[2], pk[3]};
}

template <bool kF16, int kMode, int kD = 512>
static hipError_t dec_launch_mode(dim3 grid, hipStream_t stream, const DecArgs& a) {
  constexpr int kLds = dec_lds<kD>();
  const hipError_t e = set_dynamic_lds_once<v4_decode_rows_kernel<kF16, kMode, kD>>(kLds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((v4_decode_rows_kernel<kF16, kMode, kD>), grid, dim3(256), kLds, stream, a);
  return hipSuccess;
}

template <bool kF16>
static hipError_t dec_launch(int mode, dim3 grid, hipStream_t stream, const DecArgs& a) {
  switch (mode) {
    case 1: return dec_launch_mode<kF16, 1>(grid, stream, a);
    case 2: return dec_launch_mode<kF16, 2>(grid, stream, a);
    case 3: return dec_launch_mode<kF16, 3>(grid, stream, a);
    case 4: return dec_launch_mode<kF16, 4, 576>(grid, stream, a);
    default: return dec_launch_mode<kF16, 0>(grid, stream, a);
  }
}

// Workgroups per (row, 16 heads) of the decode kernel for `cap` slots.
static int dec_splits(int64_t cap) { return cap <= kDecSingle ? 1 : (int)((cap + kDecChunk - 1) / kDecChunk); }

static size_t dec_part_bytes(int64_t T, int64_t H, int64_t cap) {
  if (T > kDecodeRows || cap > kDecodeMaxSlots || dec_splits(cap) == 1) return 0;
  return (size_t)T * H * dec_splits(cap) * kDecPart * sizeof(float);
}

// Caller: T <= kDecodeRows, cap <= kDecodeMaxSlots, H % 16 == 0; rows / count from
// a row-list kernel on `stream` (or v4 set: the kernel derives them); `part`
// holds dec_part_bytes(T, H, cap).
// The decode kernel (and, past kDecSingle slots, its combine) for kernel mode
// `mode`; `a` holds the mode's own arguments.
// out_f32: out is fp32 (else q's dtype).
static hipError_t dec_run(int is_fp16, int mode, DecArgs& a, const void* q, const void* kv, const void* kv2,
                          int64_t T, int64_t H, int64_t cap, const float* sinks, float sm_scale, void* out, float* lse,
                          void* part, hipStream_t stream, int out_f32 = 0) {
  a.q = static_cast<const uint16_t*>(q);
  a.kv = static_cast<const uint8_t*>(kv);
  a.kv2 = static_cast<const uint8_t*>(kv2);
  a.sinks = sinks;
  a.out = out_f32 ? nullptr : static_cast<uint16_t*>(out);
  a.out32 = out_f32 ? static_cast<float*>(out) : nullptr;
  a.lse = lse;
  a.T = (int)T;
  a.H = (int)H;
  a.cap = (int)cap;
  a.nsplit = dec_splits(cap);
  a.chunk = a.nsplit == 1 ? (int)cap : kDecChunk;
  a.part = static_cast<float*>(part);
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  const dim3 grid((unsigned)T, (unsigned)(H / 16), (unsigned)a.nsplit);
  const int TH = (int)(T * H);
  const dim3 cgrid((unsigned)((TH + 3) / 4));
  const hipError_t e = is_fp16 ? dec_launch<true>(mode, grid, stream, a) : dec_launch<false>(mode, grid, stream, a);
  if (e != hipSuccess) return e;
  if (a.nsplit > 1) {
    if (is_fp16)
      hipLaunchKernelGGL(v4_decode_combine_kernel<true>, cgrid, dim3(256), 0, stream, a.part, sinks, TH, (int)H,
                         a.nsplit, a.out, a.out32, lse);
    else
      hipLaunchKernelGGL(v4_decode_combine_kernel<false>, cgrid, dim3(256), 0, stream, a.part, sinks, TH, (int)H,
                         a.nsplit, a.out, a.out32, lse);
  }
  return hipGetLastError();
}

static hipError_t launch_v4_decode_rows(int is_fp16, const void* q, const void* kv, const void* kv2,
                                        const int32_t* rows, const int32_t* count, int64_t T, int64_t H, int64_t cap,
                                        const float* sinks, float sm_scale, void* out, float* lse, void* part,
                                        hipStream_t stream, const V4Args* v4 = nullptr, int out_f32 = 0) {
  DecArgs a = {};
  a.v4 = v4 ? *v4 : V4Args{};
  a.rows = rows;
  a.count = count;
  return dec_run(is_fp16, v4 ? v4->mode : 0, a, q, kv, kv2, T, H, cap, sinks, sm_scale, out, lse, part, stream,
                 out_f32);
}

// Sparse MLA (576-wide rows, V = the first 512) decode rows through the decode
// kernel: at most kDecodeRows query rows, at most 1024 (row, head) pairs (so the
// partials stay within the allocation-free entry's scratch), at most
// kMlaDecodeMaxSlots index slots.
constexpr int64_t kMlaDecodeMaxSlots = 2048;

bool mla_decode_applies(int64_t T, int64_t H, int64_t topk) {
  return T <= kDecodeRows && T * H <= 1024 && topk <= kMlaDecodeMaxSlots;
}

size_t mla_decode_part_bytes(int64_t T, int64_t H, int64_t topk) {
  if (!mla_decode_applies(T, H, topk) || dec_splits(topk) == 1) return 0;
  return (size_t)T * H * dec_splits(topk) * kDecPart * sizeof(float);
}

// Caller: mla_decode_applies(B * S * G, H, topk), H (heads per KV group) % 16 == 0,
// workspace >= mla_decode_part_bytes.
hipError_t launch_mla_decode_rows(int is_fp16, const void* q, const void* kv, const int32_t* indices,
                                  const int32_t* block_table, const int32_t* q_len, const int32_t* kv_len, int64_t B,
                                  int64_t S, int64_t G, int64_t H, int64_t Skv, int64_t block_size,
                                  int64_t max_blocks, int64_t topk, float sm_scale, int causal, void* out, float* lse,
                                  void* workspace, hipStream_t stream) {
  DecArgs a = {};
  a.mla.idx = indices;
  a.mla.block_table = block_table;
  a.mla.q_len = q_len;
  a.mla.kv_len = kv_len;
  a.mla.S = (int)S;
  a.mla.G = (int)G;
  a.mla.Skv = (int)Skv;
  a.mla.block_size = (int)block_size;
  a.mla.max_blocks = (int)max_blocks;
  a.mla.causal = causal;
  return dec_run(is_fp16, 4, a, q, kv, nullptr, B * S * G, H, topk, nullptr, sm_scale, out, lse, workspace, stream);
}

static size_t v4_lists_bytes(int64_t T, int64_t cap) {
  return ((size_t)T * (cap + 1) * sizeof(int32_t) + 255) & ~size_t(255);
}

// Row lists, then the split partials of the gather kernel or of the decode kernel.
size_t v4_workspace_bytes(int64_t T, int64_t H, int64_t cap, bool out_f32) {
  const size_t a = mla_workspace_bytes(T, H, cap, out_f32), b = dec_part_bytes(T, H, cap);
  return v4_lists_bytes(T, cap) + (a > b ? a : b);
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
  // Decode rows: the decode kernel derives the lists itself (one launch).
  void* part = static_cast<uint8_t*>(workspace) + v4_lists_bytes(T, cap);
  if (T <= kDecodeRows && cap <= kDecodeMaxSlots)
    return launch_v4_decode_rows(is_fp16, q, ori_kv, cmp_kv, nullptr, nullptr, T, H, cap, sinks, sm_scale, out, lse,
                                 part, stream, &a);
  const int per_block = 256 / kWave;
  hipLaunchKernelGGL(v4_row_lists_kernel, dim3((unsigned)((T + per_block - 1) / per_block)), dim3(256), 0, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_sparse_mla_rows(is_fp16, q, ori_kv, cmp_kv, a.rows, a.count, T, H, cap, sinks, sm_scale, out, lse,
                                part, stream, 0);
}

// The output is fp32 (as the reference kernel's), so are the split partials.
size_t sparse_attn_sink_workspace_bytes(int64_t T, int64_t H, int64_t K) { return v4_workspace_bytes(T, H, K, true); }

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
  if (T <= kDecodeRows && K <= kDecodeMaxSlots)
    return launch_v4_decode_rows(is_fp16, q, kv, nullptr, rows, count, T, H, K, sinks, sm_scale, out, lse, mla_ws,
                                 stream, nullptr, 1);
  return launch_sparse_mla_rows(is_fp16, q, kv, nullptr, rows, count, T, H, K, sinks, sm_scale, out, lse, mla_ws,
                                stream, 1);
}

}  // namespace dsa
