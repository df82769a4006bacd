// Sparse MLA forward (DeepSeek sparse attention over the shared latent KV) on gfx950.
//
// For query row (b, s) and head h, over the topk index slots j of that row:
//   score_j = sm_scale * q[b,s,h,:576] . kv[row(idx_j), :576]       (valid slots only)
//   out[b,s,h,:] = softmax_j(score) @ kv[row(idx_j), :512]
//   lse[b,s,h]   = max_j score_j + ln(sum_j exp(score_j - max))      (natural log)
// A slot is valid iff idx >= 0, idx < kv_len[b] and, when causal,
// idx <= kv_len[b] - q_len[b] + s (examples/sparse_flash_attention/
// example_sparse_flash_attn_mask_pa.py:221-224; sfa_golden.py:64-199).
// row(idx) is b*Skv + idx for a contiguous cache, or the paged address
// block_table[b][idx / block_size] * block_size + idx % block_size
// (example_sparse_flash_attn_mask_pa.py:226-233).  LSE convention:
// examples/deepseek_v4/sparse_flash_mla/sparse_flash_mla_golden.py:149.
//
// Work split.  One workgroup per (query row, split of the index list, group
// of up to 128 heads); a wave owns 16 heads.  Per 32-slot tile the workgroup
// gathers the selected KV rows from HBM with 16-byte loads into LDS twice: a
// row-major copy (the A operand of S^T = K Q^T, K = 576 over 18 MFMAs
// 16x16x32 bf16) and a column-major copy of the first 512 dims (the B operand
// of O += P V).  Q stays in VGPRs for the whole row.  Because S^T puts the
// keys on the MFMA M axis, each lane's 8 softmax probabilities are exactly the
// 8 K-values its lane must feed the PV MFMA, so P goes to bf16 and into the
// MFMA with no cross-lane shuffle.  Online softmax in base 2 (scale folded
// with log2 e), fp32 row max / row sum, P rounded to bf16 only as the MFMA
// operand (as the V4 golden does, sparse_flash_mla_golden.py:143).  The two
// LDS buffers alternate so the next tile's gather (staged in VGPRs) overlaps
// this tile's MFMAs.  With more than one split the workgroup writes a
// normalised bf16 partial and its LSE; a combine kernel merges them.
#include "common.hpp"

namespace dsa {

constexpr int kMlaD = 576;
constexpr int kMlaDV = 512;
constexpr int kMlaTile = 32;
constexpr int kKPitch = kMlaD * 2 + 16;       // bytes per key row, row-major copy
constexpr int kVtPitch = kMlaTile * 2 + 8;    // bytes per value column, column-major copy
constexpr int kKBytes = kMlaTile * kKPitch;   // 37376
constexpr int kVtBytes = kMlaDV * kVtPitch;   // 36864
constexpr int kBufBytes = kKBytes + kVtBytes + kMlaTile * 4;
constexpr int kMlaLds = 2 * kBufBytes;        // 148736 bytes

struct MlaArgs {
  const uint16_t* q;          // [B, S, H, 576] bf16
  const uint16_t* kv;         // [B, Skv, 576] or paged [blocks, block_size, 576] bf16
  const int32_t* indices;     // [B, S, topk]
  const int32_t* block_table; // [B, max_blocks] or null
  const int32_t* q_len;       // [B] or null
  const int32_t* kv_len;      // [B] or null
  uint16_t* out;              // [B, S, H, 512] bf16
  float* lse;                 // [B, S, H]
  uint16_t* part_o;           // [splits, B*S, H, 512] bf16 (splits > 1)
  float* part_lse;            // [splits, B*S, H]
  int B, S, H, Skv, topk;
  int block_size, max_blocks;
  int causal;
  int splits, keys_per_split;
  float scale_log2;           // sm_scale * log2(e)
};

__device__ __forceinline__ const uint16_t* kv_row(const MlaArgs& a, int b, int idx) {
  int64_t r;
  if (a.block_table) {
    const int blk = a.block_table[(int64_t)b * a.max_blocks + idx / a.block_size];
    r = (int64_t)blk * a.block_size + idx % a.block_size;
  } else {
    r = (int64_t)b * a.Skv + idx;
  }
  return a.kv + r * kMlaD;
}

// Interleave the bf16 halves of two words: lo16(x), lo16(y) and hi16(x), hi16(y).
__device__ __forceinline__ uint32_t pair_lo(uint32_t x, uint32_t y) { return (x & 0xffffu) | (y << 16); }
__device__ __forceinline__ uint32_t pair_hi(uint32_t x, uint32_t y) { return (x >> 16) | (y & 0xffff0000u); }

__device__ __forceinline__ bool slot_valid(int idx, int kl, int lim) { return idx >= 0 && idx < kl && idx <= lim; }

// One gather task of the value part: key pair kp (keys 2kp, 2kp+1 of the tile),
// 16-byte column chunk c (value dims 8c .. 8c+7).
__device__ __forceinline__ void vtask_load(const MlaArgs& a, const int32_t* irow, int slot0, int slot_end, int b,
                                           int kl, int lim, int e, u32x4& x, u32x4& y) {
  const int kp = e & 15;
  const int c = e >> 4;
  u32x4 v[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int slot = slot0 + 2 * kp + h;
    const int idx = slot < slot_end ? irow[slot] : -1;
    v[h] = u32x4{0, 0, 0, 0};
    if (slot < slot_end && slot_valid(idx, kl, lim)) v[h] = *reinterpret_cast<const u32x4*>(kv_row(a, b, idx) + c * 8);
  }
  x = v[0];
  y = v[1];
}

__device__ __forceinline__ void vtask_store(uint8_t* buf, int e, const u32x4& x, const u32x4& y) {
  const int kp = e & 15;
  const int c = e >> 4;
  uint8_t* krow = buf;
  *reinterpret_cast<u32x4*>(krow + (2 * kp) * kKPitch + c * 16) = x;
  *reinterpret_cast<u32x4*>(krow + (2 * kp + 1) * kKPitch + c * 16) = y;
  // Columns 8c .. 8c+7 of the column-major copy, keys 2kp and 2kp+1 packed per word.
  uint8_t* col = buf + kKBytes + (8 * c) * kVtPitch + 4 * kp;
  *reinterpret_cast<uint32_t*>(col + 0 * kVtPitch) = pair_lo(x.x, y.x);
  *reinterpret_cast<uint32_t*>(col + 1 * kVtPitch) = pair_hi(x.x, y.x);
  *reinterpret_cast<uint32_t*>(col + 2 * kVtPitch) = pair_lo(x.y, y.y);
  *reinterpret_cast<uint32_t*>(col + 3 * kVtPitch) = pair_hi(x.y, y.y);
  *reinterpret_cast<uint32_t*>(col + 4 * kVtPitch) = pair_lo(x.z, y.z);
  *reinterpret_cast<uint32_t*>(col + 5 * kVtPitch) = pair_hi(x.z, y.z);
  *reinterpret_cast<uint32_t*>(col + 6 * kVtPitch) = pair_lo(x.w, y.w);
  *reinterpret_cast<uint32_t*>(col + 7 * kVtPitch) = pair_hi(x.w, y.w);
}

// One gather task of the rope tail (dims 512..575): key e/8, chunk 64 + e%8.
__device__ __forceinline__ u32x4 ttask_load(const MlaArgs& a, const int32_t* irow, int slot0, int slot_end, int b,
                                            int kl, int lim, int e) {
  const int key = e >> 3;
  const int c = 64 + (e & 7);
  const int slot = slot0 + key;
  const int idx = slot < slot_end ? irow[slot] : -1;
  if (slot < slot_end && slot_valid(idx, kl, lim)) return *reinterpret_cast<const u32x4*>(kv_row(a, b, idx) + c * 8);
  return u32x4{0, 0, 0, 0};
}

__device__ __forceinline__ void ttask_store(uint8_t* buf, int e, const u32x4& v) {
  *reinterpret_cast<u32x4*>(buf + (e >> 3) * kKPitch + (64 + (e & 7)) * 16) = v;
}

__device__ __forceinline__ void bias_store(uint8_t* buf, const int32_t* irow, int slot0, int slot_end, int kl,
                                           int lim) {
  const int t = threadIdx.x;
  if (t < kMlaTile) {
    const int slot = slot0 + t;
    const int idx = slot < slot_end ? irow[slot] : -1;
    reinterpret_cast<float*>(buf + kKBytes + kVtBytes)[t] =
        (slot < slot_end && slot_valid(idx, kl, lim)) ? 0.f : -__builtin_huge_valf();
  }
}

// Register-staged gather (8-wave workgroups): loads for the next tile are in
// flight while the current tile computes.
template <int kNW>
struct Staged {
  static constexpr int kThreads = kNW * kWave;
  static constexpr int kV = 1024 / kThreads;                     // value tasks per thread
  static constexpr int kT = (kMlaTile * 8 + kThreads - 1) / kThreads;  // tail tasks per thread
  u32x4 x[kV], y[kV], t[kT];

  __device__ __forceinline__ void load(const MlaArgs& a, const int32_t* irow, int slot0, int slot_end, int b, int kl,
                                       int lim) {
#pragma unroll
    for (int i = 0; i < kV; ++i) vtask_load(a, irow, slot0, slot_end, b, kl, lim, threadIdx.x + i * kThreads, x[i], y[i]);
#pragma unroll
    for (int i = 0; i < kT; ++i) {
      const int e = threadIdx.x + i * kThreads;
      t[i] = e < kMlaTile * 8 ? ttask_load(a, irow, slot0, slot_end, b, kl, lim, e) : u32x4{0, 0, 0, 0};
    }
  }
  __device__ __forceinline__ void store(uint8_t* buf, const int32_t* irow, int slot0, int slot_end, int kl,
                                        int lim) const {
#pragma unroll
    for (int i = 0; i < kV; ++i) vtask_store(buf, threadIdx.x + i * kThreads, x[i], y[i]);
#pragma unroll
    for (int i = 0; i < kT; ++i) {
      const int e = threadIdx.x + i * kThreads;
      if (e < kMlaTile * 8) ttask_store(buf, e, t[i]);
    }
    bias_store(buf, irow, slot0, slot_end, kl, lim);
  }
};

// Direct gather (smaller workgroups): load and store task by task.
template <int kNW>
__device__ __forceinline__ void gather_direct(const MlaArgs& a, uint8_t* buf, const int32_t* irow, int slot0,
                                              int slot_end, int b, int kl, int lim) {
  constexpr int kThreads = kNW * kWave;
  for (int e = threadIdx.x; e < 1024; e += kThreads) {
    u32x4 x, y;
    vtask_load(a, irow, slot0, slot_end, b, kl, lim, e, x, y);
    vtask_store(buf, e, x, y);
  }
  for (int e = threadIdx.x; e < kMlaTile * 8; e += kThreads) ttask_store(buf, e, ttask_load(a, irow, slot0, slot_end, b, kl, lim, e));
  bias_store(buf, irow, slot0, slot_end, kl, lim);
}

template <bool kF16>
__device__ __forceinline__ f32x4 mfma16(const u32x4& av, const u32x4& bv, const f32x4& c) {
  if constexpr (kF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av), __builtin_bit_cast(f16x8, bv), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, bv), c, 0, 0, 0);
  }
}

template <bool kF16>
__device__ __forceinline__ uint32_t pack2(float x, float y) {
  if constexpr (kF16) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    h2 r;
    r.x = (_Float16)x;
    r.y = (_Float16)y;
    return __builtin_bit_cast(uint32_t, r);
  } else {
    return pack_bf16x2(x, y);
  }
}

template <bool kF16>
__device__ __forceinline__ uint16_t cvt1(float x) {
  if constexpr (kF16) return __builtin_bit_cast(uint16_t, (_Float16)x);
  else return __builtin_bit_cast(uint16_t, (__bf16)x);
}

template <bool kF16>
__device__ __forceinline__ float unpack_lo(uint32_t v) {
  if constexpr (kF16) return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xffffu));
  else return __uint_as_float(v << 16);
}
template <bool kF16>
__device__ __forceinline__ float unpack_hi(uint32_t v) {
  if constexpr (kF16) return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
  else return __uint_as_float(v & 0xffff0000u);
}

template <int kNW, bool kF16>
__global__ __launch_bounds__(kNW * kWave) void sparse_mla_kernel(MlaArgs a) {
  constexpr bool kStaged = (kNW == 8);
  extern __shared__ __align__(16) uint8_t lds[];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int r = lane & 15;
  const int g = lane >> 4;

  const int T = a.B * a.S;
  const int token = blockIdx.x % T;
  const int split = blockIdx.x / T;
  const int b = token / a.S;
  const int s = token % a.S;
  const int head0 = blockIdx.y * (kNW * 16) + wave * 16;
  const bool wave_active = head0 < a.H;

  const int ql = a.q_len ? a.q_len[b] : a.S;
  const int kl = a.kv_len ? a.kv_len[b] : a.Skv;
  const bool row_active = s < ql;
  const int lim = a.causal ? (kl - ql + s) : 0x7fffffff;
  const int32_t* irow = a.indices + (int64_t)token * a.topk;
  const int slot_begin = split * a.keys_per_split;
  const int slot_end = min(a.topk, slot_begin + a.keys_per_split);
  const int ntiles = row_active && slot_end > slot_begin ? (slot_end - slot_begin + kMlaTile - 1) / kMlaTile : 0;

  // Q operand (B of S^T = K Q^T): head head0 + r, dims 32*st + 8*g .. +8.
  u32x4 qb[kMlaD / 32];
  {
    const uint16_t* qp = a.q + ((int64_t)token * a.H + head0 + r) * kMlaD + 8 * g;
#pragma unroll
    for (int st = 0; st < kMlaD / 32; ++st) {
      qb[st] = (wave_active && row_active) ? *reinterpret_cast<const u32x4*>(qp + 32 * st) : u32x4{0, 0, 0, 0};
    }
  }

  f32x4 o[kMlaDV / 16];
#pragma unroll
  for (int i = 0; i < kMlaDV / 16; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m2 = -__builtin_huge_valf();  // running max (base-2 units) of head head0 + r
  float lsum = 0.f;                   // this lane's share of the running sum

  Staged<kNW> gs;
  if (ntiles > 0) {
    if constexpr (kStaged) {
      gs.load(a, irow, slot_begin, slot_end, b, kl, lim);
      gs.store(lds, irow, slot_begin, slot_end, kl, lim);
    } else {
      gather_direct<kNW>(a, lds, irow, slot_begin, slot_end, b, kl, lim);
    }
  }
  __syncthreads();

  for (int tile = 0; tile < ntiles; ++tile) {
    uint8_t* buf = lds + (tile & 1) * kBufBytes;
    const int next0 = slot_begin + (tile + 1) * kMlaTile;
    if constexpr (kStaged) {
      if (tile + 1 < ntiles) gs.load(a, irow, next0, slot_end, b, kl, lim);
    }

    if (wave_active) {
      const uint8_t* krow = buf;
      const uint8_t* vt = buf + kKBytes;
      const float* bias = reinterpret_cast<const float*>(buf + kKBytes + kVtBytes);
      // S^T[key][head] for keys 0-15 (c0) and 16-31 (c1).
      f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < kMlaD / 32; ++st) {
        const u32x4 k0 = *reinterpret_cast<const u32x4*>(krow + r * kKPitch + (32 * st + 8 * g) * 2);
        const u32x4 k1 = *reinterpret_cast<const u32x4*>(krow + (16 + r) * kKPitch + (32 * st + 8 * g) * 2);
        c0 = mfma16<kF16>(k0, qb[st], c0);
        c1 = mfma16<kF16>(k1, qb[st], c1);
      }
      // Lane (g, r) holds keys 4g+i and 16+4g+i of head head0 + r.
      float t[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        t[i] = c0[i] * a.scale_log2 + bias[4 * g + i];
        t[4 + i] = c1[i] * a.scale_log2 + bias[16 + 4 * g + i];
      }
      float tmax = t[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) tmax = fmaxf(tmax, t[i]);
      tmax = fmaxf(tmax, __shfl_xor(tmax, 16, kWave));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
      const float m_new = fmaxf(m2, tmax);
      const float m_use = (m_new == -__builtin_huge_valf()) ? 0.f : m_new;
      const float alpha = fast_exp2(m2 - m_use);
      float p[8];
      float psum = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        p[i] = fast_exp2(t[i] - m_use);
        psum += p[i];
      }
      lsum = lsum * alpha + psum;
      m2 = m_new;
      // Rows of the PV accumulator are heads 4g+i: fetch their alpha.
      float al[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * g + i, kWave);
      const u32x4 pa = {pack2<kF16>(p[0], p[1]), pack2<kF16>(p[2], p[3]), pack2<kF16>(p[4], p[5]), pack2<kF16>(p[6], p[7])};
#pragma unroll
      for (int cb = 0; cb < kMlaDV / 16; ++cb) {
        const uint8_t* col = vt + (16 * cb + r) * kVtPitch;
        const u32x2 lo = *reinterpret_cast<const u32x2*>(col + 8 * g);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(col + 32 + 8 * g);
        const u32x4 vb = {lo.x, lo.y, hi.x, hi.y};
        f32x4 acc = o[cb];
        acc[0] *= al[0]; acc[1] *= al[1]; acc[2] *= al[2]; acc[3] *= al[3];
        o[cb] = mfma16<kF16>(pa, vb, acc);
      }
    }
    if (tile + 1 < ntiles) {
      __syncthreads();  // everyone is done reading the other buffer (tile - 1)
      uint8_t* nbuf = lds + ((tile + 1) & 1) * kBufBytes;
      if constexpr (kStaged) {
        gs.store(nbuf, irow, next0, slot_end, kl, lim);
      } else {
        gather_direct<kNW>(a, nbuf, irow, next0, slot_end, b, kl, lim);
      }
    }
    __syncthreads();
  }

  // Epilogue: normalise, write out (or the split partial) and the LSE.
  float l_tot = lsum;
  l_tot += __shfl_xor(l_tot, 16, kWave);
  l_tot += __shfl_xor(l_tot, 32, kWave);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  float inv_i[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) inv_i[i] = __shfl(inv, 4 * g + i, kWave);

  const bool final_out = (a.splits == 1);
  uint16_t* obase = final_out ? a.out : a.part_o + (int64_t)split * T * a.H * kMlaDV;
  float* lbase = final_out ? a.lse : a.part_lse + (int64_t)split * T * a.H;
  // Stage the wave's 16 x 512 tile in LDS, then store 16-byte row chunks.
  uint16_t* stage = reinterpret_cast<uint16_t*>(lds) + wave * 16 * (kMlaDV + 8);
#pragma unroll
  for (int cb = 0; cb < kMlaDV / 16; ++cb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) stage[(4 * g + i) * (kMlaDV + 8) + 16 * cb + r] = cvt1<kF16>(o[cb][i] * inv_i[i]);
  }
  __syncthreads();
  if (wave_active) {
    uint16_t* orow = obase + ((int64_t)token * a.H + head0) * kMlaDV;
#pragma unroll
    for (int it = 0; it < 16 * kMlaDV / 8 / kWave; ++it) {
      const int e = lane + it * kWave;  // 16-byte chunk: head e / 64, cols 8*(e % 64)
      const int h = e >> 6;
      const int c = (e & 63) * 8;
      *reinterpret_cast<u32x4*>(orow + h * kMlaDV + c) = *reinterpret_cast<const u32x4*>(stage + h * (kMlaDV + 8) + c);
    }
    if (g == 0) {
      const float lse = l_tot > 0.f ? (m2 + fast_log2(l_tot)) * 0.69314718055994531f : -__builtin_huge_valf();
      lbase[(int64_t)token * a.H + head0 + r] = lse;
    }
  }
}

// Merge split partials: lse = log(sum_i exp(lse_i)), out = sum_i exp(lse_i - lse) * o_i.
template <bool kF16>
__global__ __launch_bounds__(256) void sparse_mla_combine_kernel(const uint16_t* __restrict__ part_o,
                                                                 const float* __restrict__ part_lse, int splits,
                                                                 int64_t rows, uint16_t* __restrict__ out,
                                                                 float* __restrict__ lse) {
  // One thread per (row = token*H + head, 8 columns).
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = gid >> 6;
  const int c = (int)(gid & 63) * 8;
  if (row >= rows) return;
  float mx = -__builtin_huge_valf();
  for (int i = 0; i < splits; ++i) mx = fmaxf(mx, part_lse[(int64_t)i * rows + row]);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float wsum = 0.f;
  if (mx != -__builtin_huge_valf()) {
    for (int i = 0; i < splits; ++i) {
      const float li = part_lse[(int64_t)i * rows + row];
      if (li == -__builtin_huge_valf()) continue;
      const float w = __expf(li - mx);
      wsum += w;
      const u32x4 v = *reinterpret_cast<const u32x4*>(part_o + ((int64_t)i * rows + row) * kMlaDV + c);
      const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] += w * unpack_lo<kF16>(vv[j]);
        acc[2 * j + 1] += w * unpack_hi<kF16>(vv[j]);
      }
    }
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  u32x4 o;
  o.x = pack2<kF16>(acc[0] * inv, acc[1] * inv);
  o.y = pack2<kF16>(acc[2] * inv, acc[3] * inv);
  o.z = pack2<kF16>(acc[4] * inv, acc[5] * inv);
  o.w = pack2<kF16>(acc[6] * inv, acc[7] * inv);
  *reinterpret_cast<u32x4*>(out + row * kMlaDV + c) = o;
  if (c == 0) lse[row] = wsum > 0.f ? mx + __logf(wsum) : -__builtin_huge_valf();
}

int mla_choose_splits(int64_t tokens, int64_t head_groups, int64_t topk) {
  const int64_t wgs = tokens * head_groups;
  int splits = 1;
  const int max_splits = (int)((topk + kMlaTile - 1) / kMlaTile);
  while (wgs * splits < 256 && splits * 2 <= max_splits) splits *= 2;
  return splits;
}

size_t mla_workspace_bytes(int64_t tokens, int64_t H, int64_t topk) {
  const int64_t hg = (H + 127) / 128;
  const int splits = mla_choose_splits(tokens, hg, topk);
  if (splits == 1) return 0;
  return (size_t)splits * tokens * H * (kMlaDV * 2 + 4) + 256;
}

template <int kNW, bool kF16>
static hipError_t launch_mla_nw(const MlaArgs& a, int head_groups, hipStream_t stream) {
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute((const void*)sparse_mla_kernel<kNW, kF16>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              kMlaLds);
    attr = true;
  }
  const dim3 grid((unsigned)((int64_t)a.B * a.S * a.splits), (unsigned)head_groups);
  hipLaunchKernelGGL((sparse_mla_kernel<kNW, kF16>), grid, dim3(kNW * kWave), kMlaLds, stream, a);
  return hipGetLastError();
}

template <bool kF16>
static hipError_t launch_mla_dtype(const MlaArgs& a, int head_groups, int hpg, hipStream_t stream) {
  hipError_t e;
  if (hpg > 64) e = launch_mla_nw<8, kF16>(a, head_groups, stream);
  else if (hpg > 32) e = launch_mla_nw<4, kF16>(a, head_groups, stream);
  else if (hpg > 16) e = launch_mla_nw<2, kF16>(a, head_groups, stream);
  else e = launch_mla_nw<1, kF16>(a, head_groups, stream);
  if (e != hipSuccess || a.splits == 1) return e;
  const int64_t rows = (int64_t)a.B * a.S * a.H;
  const int64_t threads = rows * (kMlaDV / 8);
  hipLaunchKernelGGL((sparse_mla_combine_kernel<kF16>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream,
                     a.part_o, a.part_lse, a.splits, rows, a.out, a.lse);
  return hipGetLastError();
}

// Caller validated: d_qk 576, d_v 512, H % 16 == 0, 16-bit inputs, workspace >= mla_workspace_bytes.
hipError_t launch_sparse_mla(int is_fp16, const void* q, const void* kv, const int32_t* indices,
                             const int32_t* block_table, const int32_t* q_len, const int32_t* kv_len, int64_t B,
                             int64_t S, int64_t H, int64_t Skv, int64_t block_size, int64_t max_blocks, int64_t topk,
                             float sm_scale, int causal, void* out, float* lse, void* workspace, hipStream_t stream) {
  const int64_t T = B * S;
  if (T == 0 || H == 0) return hipSuccess;
  MlaArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.kv = static_cast<const uint16_t*>(kv);
  a.indices = indices;
  a.block_table = block_table;
  a.q_len = q_len;
  a.kv_len = kv_len;
  a.out = static_cast<uint16_t*>(out);
  a.lse = lse;
  a.B = (int)B;
  a.S = (int)S;
  a.H = (int)H;
  a.Skv = (int)Skv;
  a.topk = (int)topk;
  a.block_size = (int)block_size;
  a.max_blocks = (int)max_blocks;
  a.causal = causal;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  const int head_groups = (int)((H + 127) / 128);
  a.splits = mla_choose_splits(T, head_groups, topk);
  const int64_t per = (topk + a.splits - 1) / a.splits;
  a.keys_per_split = (int)(((per + kMlaTile - 1) / kMlaTile) * kMlaTile);
  a.part_o = nullptr;
  a.part_lse = nullptr;
  if (a.splits > 1) {
    a.part_o = static_cast<uint16_t*>(workspace);
    a.part_lse = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + (size_t)a.splits * T * H * kMlaDV * 2);
  }
  const int hpg = H >= 128 ? 128 : (int)H;  // heads per workgroup
  return is_fp16 ? launch_mla_dtype<true>(a, head_groups, hpg, stream)
                 : launch_mla_dtype<false>(a, head_groups, hpg, stream);
}

}  // namespace dsa
