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

// ---------------------------------------------------------------------------
// Decode-shaped row lists (at most kDecodeRows query rows): one workgroup per
// (query row, 16 heads), its four waves splitting the row's slots into
// 16-slot blocks (wave w takes blocks w, w + 4, ...), each with its own online
// softmax and O, merged in LDS at the end.  No split partials and no combine
// launch: such a call is a chain of latencies, and this removes a launch and
// a global round trip from it.  For swa and hca rows the kernel also derives
// the row lists itself (the window, then the compressed rows below the row's
// threshold, through the block tables), so the call is this one launch.
//
// A block's 16 rows (1 KB each, K = V) go to the wave's 16 KB of LDS by DMA,
// one row per instruction, lane l carrying 16-byte chunk l ^ 2u of row u (so
// the Q K^T operand reads, 16 rows at one chunk, fall on distinct banks).
// S^T = K Q^T by 16x16x32 MFMAs (lane (g, r): keys 4g + i of head r), then
// O^T += V^T P^T by 16x16x16 MFMAs whose V^T operand comes from
// ds_read_b64_tr_b16 and whose P operand is the lane's own four scores.  As in
// the gather kernel, O is normalised by the sum of the 16-bit-rounded P, the
// LSE by the exact sum, and the sinks join the denominator.
constexpr int kDecBlk = 16;
constexpr int64_t kDecodeRows = 8;
// ... and at most this many slots per row: three blocks per wave.  Longer lists
// (a csa selection) go through the split gather kernel, which keeps several
// tiles in flight per workgroup where this kernel loads one block at a time.
constexpr int64_t kDecodeMaxSlots = 12 * kDecBlk;
constexpr int kDecWaveLds = kDecBlk * 1024;          // a wave's block of rows
constexpr int kDecOBytes = 4 * 512 * 16 * 4;          // the four waves' O^T, fp32
constexpr int kDecLds = kDecOBytes + 3 * 4 * 16 * 4;  // + m, l, rounded l per wave and head

struct DecArgs {
  const uint16_t* q;      // [T, H, 512]
  const uint8_t* kv;      // rows of 1 KB
  const uint8_t* kv2;     // rows tagged kCmpTag, or null
  const int32_t* rows;    // [T, cap]
  const int32_t* count;   // [T]; -1: padded row
  const float* sinks;     // [H] or null
  uint16_t* out;          // [T, H, 512]
  float* lse;             // [T, H]
  int T, H, cap;
  float scale_log2;
  // swa / hca lists derived here instead (inl): the row's batch, window and
  // compressed rows, as v4_row_lists_kernel computes them.
  int inl;
  V4Args v4;
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
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

template <bool kF16>
__global__ __launch_bounds__(256) void v4_decode_rows_kernel(DecArgs a) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int t = blockIdx.x;
  const int h0 = blockIdx.y * 16;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int r = lane & 15, g = lane >> 4;
  int cnt_raw, vb = 0, vnw = 0, vw0 = 0;
  const V4Args& v = a.v4;
  if (a.inl) {  // workgroup-uniform
    for (int i = 1; i < v.B; ++i) vb = v.q_start[i] <= t ? i : vb;
    const int sq = t - v.q_start[vb];
    const int qlb = v.q_len[vb];
    if (sq < 0 || sq >= qlb) {
      cnt_raw = -1;
    } else {
      const int sg = v.kv_len[vb] - qlb + sq;  // position of this row in its sequence
      vnw = sg >= 0 ? min(v.win_left, sg) + 1 : 0;
      vw0 = sg - vnw + 1;
      cnt_raw = vnw + ((v.mode == 2 && sg >= 0) ? min((sg + 1) / v.cmp_ratio, v.max_cmp) : 0);
    }
  } else {
    cnt_raw = a.count[t];
  }
  if (cnt_raw < 0) {  // padded query row: out 0, lse 0 (workgroup-uniform)
    for (int e = tid; e < 16 * 64; e += 256)
      *reinterpret_cast<u32x4*>(a.out + ((int64_t)t * a.H + h0 + e / 64) * 512 + 8 * (e % 64)) = u32x4{0, 0, 0, 0};
    if (tid < 16) a.lse[(int64_t)t * a.H + h0 + tid] = 0.f;
    return;
  }
  const int cnt = min(cnt_raw, a.cap);
  // Q^T operands: head h0 + r, dims 32 st + 8g .. +7.
  u32x4 qb[16];
  const uint16_t* qp = a.q + ((int64_t)t * a.H + h0 + r) * 512 + 8 * g;
#pragma unroll
  for (int st = 0; st < 16; ++st) qb[st] = *reinterpret_cast<const u32x4*>(qp + 32 * st);
  f32x4 o[32];
#pragma unroll
  for (int c = 0; c < 32; ++c) o[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -__builtin_huge_valf(), l = 0.f, lr = 0.f;
  uint8_t* buf = lds + wave * kDecWaveLds;
  const int32_t* rowl = a.rows + (int64_t)t * a.cap;
  const int nblk = (cnt + kDecBlk - 1) / kDecBlk;
  auto load = [&](int blk, uint8_t* bp) -> uint32_t {
    const int s0 = blk * kDecBlk;
    // Lane u < 16 holds slot s0 + u's row; invalid slots read row 0 (their scores are masked).
    const int slot = s0 + (lane & 15);
    int32_t rr;
    if (a.inl) {
      // Window position vw0 + i, then compressed row i - vnw; both lookups go out
      // (from clamped entries), the slot picks one.
      const int i = min(slot, cnt - 1);
      const int pw = max(vw0 + i, 0), ew = pw / v.ori_bs;
      const int bw = v.ori_bt[(int64_t)vb * v.ori_tl + min(ew, v.ori_tl - 1)];
      const int32_t rw = (ew < v.ori_tl && bw >= 0 && bw < v.ori_blocks) ? bw * v.ori_bs + pw % v.ori_bs : -1;
      int32_t rc = -1;
      if (v.mode == 2) {
        const int pc = max(i - vnw, 0), ec = pc / v.cmp_bs;
        const int bc = v.cmp_bt[(int64_t)vb * v.cmp_tl + min(ec, v.cmp_tl - 1)];
        rc = (ec < v.cmp_tl && bc >= 0 && bc < v.cmp_blocks) ? ((bc * v.cmp_bs + pc % v.cmp_bs) | kCmpTag) : -1;
      }
      rr = i < vnw ? rw : rc;
    } else {
      rr = rowl[min(slot, cnt - 1)];
    }
    const bool valid = slot < cnt && rr >= 0;
    const uint32_t vmask = (uint32_t)__builtin_amdgcn_ballot_w64(valid && lane < 16);
#pragma unroll
    for (int u = 0; u < kDecBlk; ++u) {
      const int ru = __builtin_amdgcn_readlane(valid ? rr : 0, u);
      const uint8_t* base = (ru & kCmpTag) ? a.kv2 : a.kv;
      const uint8_t* src = base + (int64_t)(ru & ~kCmpTag) * 1024 + 16 * (lane ^ (2 * u));
      __builtin_amdgcn_global_load_lds((dec_gbl_void*)src, (dec_lds_void*)(bp + u * 1024), 16, 0, 0);
    }
    return vmask;
  };
  auto process = [&](const uint8_t* bp, uint32_t vmask) {
    // S^T = K Q^T: A = K rows r (chunk 4 st + g), B = Q^T.
    f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 16; ++st) {
      const u32x4 kr = *reinterpret_cast<const u32x4*>(bp + r * 1024 + 16 * ((4 * st + g) ^ (2 * r)));
      sc = dec_mfma_qk<kF16>(kr, qb[st], sc);
    }
    float s2[4], bm = -__builtin_huge_valf();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s2[i] = ((vmask >> (4 * g + i)) & 1u) ? sc[i] * a.scale_log2 : -__builtin_huge_valf();
      bm = fmaxf(bm, s2[i]);
    }
    bm = fmaxf(bm, __shfl_xor(bm, 16, kWave));
    bm = fmaxf(bm, __shfl_xor(bm, 32, kWave));
    const float mn = fmaxf(m, bm);
    // Both -inf (nothing valid yet): alpha 1 and every p 0, with no inf - inf.
    const float alpha = m == mn ? 1.f : fast_exp2(m - mn);
    m = mn;
    l *= alpha;
    lr *= alpha;
#pragma unroll
    for (int c = 0; c < 32; ++c) o[c] *= alpha;
    s16x4 pb;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = s2[i] == -__builtin_huge_valf() ? 0.f : fast_exp2(s2[i] - mn);
      float back;
      pb[i] = dec_round<kF16>(p, back);
      l += p;
      lr += back;
    }
    // O^T += V^T P^T: lane (g, L) feeds row 4g + L / 4, columns 16 c + 4 (L % 4) .. +3.
    const int vrow = 4 * g + (r >> 2);
#pragma unroll
    for (int c = 0; c < 32; ++c) {
      const int chunk = 2 * c + ((r & 3) >> 1);
      const s16x4 va = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_s16x4*)(bp + vrow * 1024 + 16 * (chunk ^ (2 * vrow)) + 8 * (r & 1)));
      o[c] = dec_mfma_pv<kF16>(va, pb, o[c]);
    }
  };
  for (int blk = wave; blk < nblk; blk += 4) {
    const uint32_t vm = load(blk, buf);
    __builtin_amdgcn_s_waitcnt(0);  // the block is in LDS
    process(buf, vm);
  }
  l += __shfl_xor(l, 16, kWave);
  l += __shfl_xor(l, 32, kWave);
  lr += __shfl_xor(lr, 16, kWave);
  lr += __shfl_xor(lr, 32, kWave);
  __syncthreads();  // every wave is done with its block buffer
  float* ow = reinterpret_cast<float*>(lds) + wave * (512 * 16);
#pragma unroll
  for (int c = 0; c < 32; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i) ow[(16 * c + 4 * g + i) * 16 + r] = o[c][i];
  float* stats = reinterpret_cast<float*>(lds + kDecOBytes);  // [3][4 waves][16 heads]
  if (g == 0) {
    stats[wave * 16 + r] = m;
    stats[64 + wave * 16 + r] = l;
    stats[128 + wave * 16 + r] = lr;
  }
  __syncthreads();
  // Merge: thread handles head e % 16, columns 8 (e / 16) .. +7.
  const float* of = reinterpret_cast<const float*>(lds);
  for (int e = tid; e < 16 * 64; e += 256) {
    const int h = e & 15, c8 = 8 * (e >> 4);
    float mw[4], mx = -__builtin_huge_valf();
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      mw[w] = stats[w * 16 + h];
      mx = fmaxf(mx, mw[w]);
    }
    const float sink2 = a.sinks ? a.sinks[h0 + h] * 1.4426950408889634f : -__builtin_huge_valf();
    const float mm = fmaxf(mx, sink2);
    float den = 0.f, den_r = 0.f, wgt[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      wgt[w] = mm == -__builtin_huge_valf() ? 0.f : fast_exp2(mw[w] - mm);
      den += stats[64 + w * 16 + h] * wgt[w];
      den_r += stats[128 + w * 16 + h] * wgt[w];
    }
    const float es = a.sinks && mm != -__builtin_huge_valf() ? fast_exp2(sink2 - mm) : 0.f;
    den += es;
    den_r += es;
    const float inv = den_r > 0.f ? 1.f / den_r : 0.f;
    uint32_t pk[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v2[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int col = c8 + 2 * j + k;
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) acc += of[w * (512 * 16) + col * 16 + h] * wgt[w];
        v2[k] = acc * inv;
      }
      if constexpr (kF16) {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        const h2 hv = {(_Float16)v2[0], (_Float16)v2[1]};
        pk[j] = __builtin_bit_cast(uint32_t, hv);
      } else {
        pk[j] = pack_bf16x2(v2[0], v2[1]);
      }
    }
    *reinterpret_cast<u32x4*>(a.out + ((int64_t)t * a.H + h0 + h) * 512 + c8) = u32x4{pk[0], pk[1], pk[2], pk[3]};
    if (c8 == 0)
      a.lse[(int64_t)t * a.H + h0 + h] = den > 0.f ? (mm + fast_log2(den)) * 0.69314718055994531f : -__builtin_huge_valf();
  }
}

// Caller: T <= kDecodeRows, H % 16 == 0, rows / count from a row-list kernel on `stream`.
static hipError_t launch_v4_decode_rows(int is_fp16, const void* q, const void* kv, const void* kv2,
                                        const int32_t* rows, const int32_t* count, int64_t T, int64_t H, int64_t cap,
                                        const float* sinks, float sm_scale, void* out, float* lse,
                                        hipStream_t stream, const V4Args* v4 = nullptr) {
  DecArgs a;
  a.inl = v4 != nullptr;
  a.v4 = v4 ? *v4 : V4Args{};
  a.q = static_cast<const uint16_t*>(q);
  a.kv = static_cast<const uint8_t*>(kv);
  a.kv2 = static_cast<const uint8_t*>(kv2);
  a.rows = rows;
  a.count = count;
  a.sinks = sinks;
  a.out = static_cast<uint16_t*>(out);
  a.lse = lse;
  a.T = (int)T;
  a.H = (int)H;
  a.cap = (int)cap;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  const dim3 grid((unsigned)T, (unsigned)(H / 16));
  if (is_fp16) {
    const hipError_t e = set_dynamic_lds_once<v4_decode_rows_kernel<true>>(kDecLds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(v4_decode_rows_kernel<true>, grid, dim3(256), kDecLds, stream, a);
  } else {
    const hipError_t e = set_dynamic_lds_once<v4_decode_rows_kernel<false>>(kDecLds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(v4_decode_rows_kernel<false>, grid, dim3(256), kDecLds, stream, a);
  }
  return hipGetLastError();
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
  // swa / hca decode rows: the decode kernel derives the lists itself (one launch fewer).
  if (mode != 3 && T <= kDecodeRows && cap <= kDecodeMaxSlots)
    return launch_v4_decode_rows(is_fp16, q, ori_kv, cmp_kv, nullptr, nullptr, T, H, cap, sinks, sm_scale, out, lse,
                                 stream, &a);
  const int per_block = 256 / kWave;
  hipLaunchKernelGGL(v4_row_lists_kernel, dim3((unsigned)((T + per_block - 1) / per_block)), dim3(256), 0, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (T <= kDecodeRows && cap <= kDecodeMaxSlots)
    return launch_v4_decode_rows(is_fp16, q, ori_kv, cmp_kv, a.rows, a.count, T, H, cap, sinks, sm_scale, out, lse,
                                 stream);
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
  if (T <= kDecodeRows && K <= kDecodeMaxSlots)
    return launch_v4_decode_rows(is_fp16, q, kv, nullptr, rows, count, T, H, K, sinks, sm_scale, out, lse, stream);
  void* mla_ws = static_cast<uint8_t*>(workspace) + v4_lists_bytes(T, K);
  return launch_sparse_mla_rows(is_fp16, q, kv, nullptr, rows, count, T, H, K, sinks, sm_scale, out, lse, mla_ws,
                                stream);
}

}  // namespace dsa
