// Sparse GQA attention (grouped 128-wide KV heads) on gfx950.
//
// The grouped sparse attention of
// examples/sparse_flash_attention/example_sparse_flash_attn_gqa.py:13-238 (golden
// :241-295): kv [B, Skv, G, 128] holds G KV heads; query heads g*Hg .. (g+1)*Hg - 1
// (Hg = H / G) read, through their own index row indices[b, s, g, :], rows of KV
// head g, with K = V = the whole 128-wide row:
//   score_j = sm_scale * q[b,s,h,:] . kv[b, idx_j, g, :]     (valid slots only)
//   out[b,s,h,:] = softmax_j(score) @ kv[b, idx_j, g, :]
//   lse[b,s,h]   = max_j score_j + ln(sum_j exp(score_j - max))  (natural log)
// A slot is valid iff 0 <= idx < kv_len[b] and, when causal,
// idx <= kv_len[b] - q_len[b] + s (the convention of sparse_mla.hip); a row with
// no valid slot gets out = 0, lse = -inf.
//
// Work split.  One workgroup of four waves per query row (b, s, g) and group of
// up to 32 heads.  The workgroup first turns the index row into KV row numbers
// in LDS (one pass, all loads in flight at once) and lists the tiles of 32 slots
// that hold a valid slot; wave w then walks entries w, w + 4, ... of that list
// on its own -- its own LDS ring, no workgroup barrier in the loop -- with an
// online softmax; the four waves' (max, sum, O) merge through LDS at the end.
//
// Per tile and wave: the DMA (global_load_lds_dwordx4; one instruction moves
// 4 rows = 1 KB, each row's 16-byte chunks permuted by gqa_swz so that the
// operand reads below are bank-conflict free but for the 2-way sharing every
// transposed read has), S^T = K Q^T (2 key blocks x 4 steps of
// v_mfma_f32_16x16x32 per 16-head block, keys on the M axis), the softmax
// (each lane holds 8 scores of one head), and O^T += V^T P^T (8 blocks of 16
// output columns, V^T through ds_read_b64_tr_b16).  Each slot brings 256 bytes
// for 16 x 2 x 2 x 128 flops per 16 heads: the loop is bound by the gather.
#include "common.hpp"

namespace dsa {

constexpr int kGqaD = 128;
constexpr int kGqaRowBytes = kGqaD * 2;                 // 256
constexpr int kGqaTile = 32;                            // slots per tile
constexpr int kGqaTileBytes = kGqaTile * kGqaRowBytes;  // 8 KB
constexpr int kGqaWaves = 4;
constexpr int kGqaThreads = kGqaWaves * kWave;
constexpr int kGqaMaxTopk = 8192;
constexpr int kGqaMaxTiles = kGqaMaxTopk / kGqaTile;    // 256: a wave holds <= 64 list entries
constexpr int kGqaIdxBatch = 2048;                      // index slots loaded per prologue pass

typedef __attribute__((address_space(3))) void gqa_lds_void;
typedef const __attribute__((address_space(1))) void gqa_gbl_void;

struct GqaArgs {
  const uint16_t* q;       // [B, S, G * Hg, 128]
  const uint16_t* kv;      // [B, Skv, G, 128]
  const int32_t* indices;  // [B, S, G, topk]
  const int32_t* q_len;    // [B] or null (S)
  const int32_t* kv_len;   // [B] or null (Skv)
  uint16_t* out;           // [B, S, G * Hg, 128]
  float* lse;              // [B, S, G * Hg]
  int B, S, G, Hg, Skv, topk, causal;
  float scale_log2;        // sm_scale * log2(e)
};

// LDS position of 16-byte chunk c of tile key k (0..31) is c ^ gqa_swz(k).  A
// ds_read_b128 is served per 32-lane half-wave and is conflict-free when its
// 32 chunks fall on distinct positions modulo 512 bytes (two 256-byte rows).
// K operand reads (half-wave: keys r = 0..15, chunks 4 st + g for two g):
// position 16 (r & 1) + (4 st + g) ^ swz(r), and swz maps (r >> 1) & 3 onto
// bits 2-3 and (r >> 3) & 1 onto bit 1: all 32 distinct.  Transposed V reads
// (keys 4g + (r >> 2), chunks 4p + (r & 3), 8 bytes a lane): each position is
// read by the two lanes of keys k and k ^ 8, the sharing such reads always have.
__host__ __device__ constexpr int gqa_swz(int k) { return 4 * ((k >> 1) & 3) + 2 * ((k >> 3) & 1); }

__device__ __forceinline__ uint32_t gqa_lds_u32(const void* p) {
  return (uint32_t)(uintptr_t)(const gqa_lds_void*)p;
}

// LDS reads as inline asm: through the builtins the compiler would wait for
// every outstanding DMA before each read.  Completion is waited for explicitly.
template <int kOff>
__device__ __forceinline__ void gqa_b128(u32x4& out, uint32_t addr) {
  __asm__ __volatile__("ds_read_b128 %0, %1 offset:%2" : "=v"(out) : "v"(addr), "i"(kOff));
}
template <int kOff>
__device__ __forceinline__ void gqa_tr(u32x2& out, uint32_t addr) {
  __asm__ __volatile__("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(out) : "v"(addr), "i"(kOff));
}
template <int N, typename V>
__device__ __forceinline__ void gqa_lgkm_wait(V (&v)[N]) {
  // All LDS operations retired; the values pass through the asm so that no use
  // is scheduled above the wait.
#pragma unroll
  for (int i = 0; i < N; ++i) __asm__ __volatile__("" : "+v"(v[i]));
  __asm__ __volatile__("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < N; ++i) __asm__ __volatile__("" : "+v"(v[i]));
}

// s_waitcnt with only vmcnt constrained.
template <int N>
__device__ __forceinline__ void gqa_wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

template <bool kF16>
__device__ __forceinline__ f32x4 gqa_mfma(const u32x4& a, const u32x4& b, const f32x4& c) {
  if constexpr (kF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

template <bool kF16>
__device__ __forceinline__ uint32_t gqa_pack(float lo, float hi) {
  if constexpr (kF16) {
    const _Float16 a = (_Float16)lo, b = (_Float16)hi;
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
  } else {
    return pack_bf16x2(lo, hi);
  }
}

// LDS layout of a workgroup: the four waves' rings (kStg stages of one tile),
// then the slot -> KV row table (per tile, key k at (k & 3) * 8 + (k >> 2), so
// that DMA lane group q reads its eight rows 8q .. 8q + 7 with two b128
// reads), the tiles' valid-slot masks, the list of tiles holding a valid slot
// and its length, and the waves' (max, sum) per head for the merge.
__host__ __device__ constexpr int gqa_ring_bytes(int stg) { return kGqaWaves * stg * kGqaTileBytes; }
__host__ __device__ constexpr int gqa_lds_bytes(int stg, int hb, int ntiles) {
  return gqa_ring_bytes(stg) + ntiles * kGqaTile * 4 + ntiles * 4 + (ntiles + 1) * 4 + kGqaWaves * 16 * hb * 2 * 4;
}

template <bool kF16, int kHB, int kStg>
__global__ __launch_bounds__(kGqaThreads, 2) void sparse_gqa_kernel(GqaArgs a) {
  static_assert(kStg >= 2 && kStg <= 3, "ring depth: the merge reuses a wave's ring (16 KB per 16 heads x 2)");
  static_assert(kHB * 16 * kGqaD * 4 <= kStg * kGqaTileBytes, "a wave's O fits its ring");
  extern __shared__ __align__(16) uint8_t lds[];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int r = lane & 15, g = lane >> 4;

  const int row = blockIdx.x;  // (b * S + s) * G + kvg
  const int bs_row = row / a.G;
  const int kvg = row - bs_row * a.G;
  const int b = bs_row / a.S;
  const int s = bs_row - b * a.S;
  const int h0 = blockIdx.y * (16 * kHB);  // first head of this workgroup within its group

  const int ntiles = (a.topk + kGqaTile - 1) / kGqaTile;
  int32_t* rows = reinterpret_cast<int32_t*>(lds + gqa_ring_bytes(kStg));
  uint32_t* tmask = reinterpret_cast<uint32_t*>(rows + ntiles * kGqaTile);
  int32_t* tlist = reinterpret_cast<int32_t*>(tmask + ntiles);  // [ntiles] then the count
  float* mlbuf = reinterpret_cast<float*>(tlist + ntiles + 1);  // [wave][16 kHB heads][max, sum]

  typedef const __attribute__((address_space(4))) int32_t const_i32;
  const int ql = a.q_len ? min(max(*(const_i32*)(a.q_len + b), 0), a.S) : a.S;
  const int kl = a.kv_len ? min(max(*(const_i32*)(a.kv_len + b), 0), a.Skv) : a.Skv;
  const bool active = s < ql;
  const int lim = a.causal ? kl - ql + s : 0x7fffffff;
  const int32_t* irow = a.indices + (int64_t)row * a.topk;
  const int row0 = b * a.Skv * a.G + kvg;  // KV row of (b, idx 0, kvg); idx adds idx * G

  // Slot table.  Pass p covers slots p .. p + 2047: lane l of wave w loads slot
  // 64 (w + 4 j) + l for j < 8 (all loads first, from clamped addresses).
  u32x4 qb[kHB][kGqaD / 32];
  const int npad = ntiles * kGqaTile;
  for (int p = 0; p < npad; p += kGqaIdxBatch) {
    int idx[kGqaIdxBatch / kGqaThreads];
#pragma unroll
    for (int j = 0; j < kGqaIdxBatch / kGqaThreads; ++j) {
      const int i = p + kWave * (wave + kGqaWaves * j) + lane;
      idx[j] = irow[min(i, a.topk - 1)];
    }
    if (p == 0) {
      // Q operands (B of S^T = K Q^T): head h0 + 16 hb + r, dims 32 st + 8 g .. +7;
      // heads past Hg repeat head Hg - 1 and are not stored.  Issued behind the
      // index loads, so the first tile's DMA wait covers them.
      __asm__ __volatile__("" ::: "memory");
#pragma unroll
      for (int hb = 0; hb < kHB; ++hb) {
        const int h = min(h0 + 16 * hb + r, a.Hg - 1);
        const uint16_t* qp = a.q + ((int64_t)row * a.Hg + h) * kGqaD + 8 * g;
#pragma unroll
        for (int st = 0; st < kGqaD / 32; ++st) qb[hb][st] = *reinterpret_cast<const u32x4*>(qp + 32 * st);
      }
    }
#pragma unroll
    for (int j = 0; j < kGqaIdxBatch / kGqaThreads; ++j) {
      const int i0 = p + kWave * (wave + kGqaWaves * j);
      if (i0 >= npad) break;
      const int i = i0 + lane;
      const bool ok = active && i < a.topk && idx[j] >= 0 && idx[j] < kl && idx[j] <= lim;
      const int k = i & (kGqaTile - 1);
      // With an odd tile count the last group's upper half lies past the table.
      if (i < npad) rows[(i & ~(kGqaTile - 1)) + (k & 3) * 8 + (k >> 2)] = ok ? row0 + idx[j] * a.G : -1;
      const uint64_t vm = __ballot(ok);
      if (lane == 0) {
        tmask[i0 / kGqaTile] = (uint32_t)vm;
        if (i0 / kGqaTile + 1 < ntiles) tmask[i0 / kGqaTile + 1] = (uint32_t)(vm >> 32);
      }
    }
  }
  __syncthreads();
  // The tiles with a valid slot, in order (wave 0).
  if (wave == 0) {
    int n = 0;
    for (int t0 = 0; t0 < ntiles; t0 += kWave) {
      const int t = t0 + lane;
      const bool ne = t < ntiles && tmask[t] != 0u;
      const uint64_t bal = __ballot(ne);
      const int pos = n + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
      if (ne) tlist[pos] = t;
      n += __builtin_popcountll(bal);
    }
    if (lane == 0) tlist[ntiles] = n;
  }
  __syncthreads();
  const int nlist = tlist[ntiles];
  const int nmy = nlist > wave ? (nlist - wave + kGqaWaves - 1) / kGqaWaves : 0;  // <= 64
  // Lane j holds this wave's entry j: its tile and valid-slot mask.
  const int my_tile = wave + kGqaWaves * lane < nlist ? tlist[wave + kGqaWaves * lane] : 0;
  const uint32_t my_mask = tmask[my_tile];

  uint8_t* ring = lds + wave * kStg * kGqaTileBytes;
  const uint8_t* kvb = reinterpret_cast<const uint8_t*>(a.kv);
  const int q4 = lane >> 4;
  // DMA of entry e into stage st: instruction n moves keys 4n .. 4n + 3; lane l
  // fetches chunk (l & 15) ^ gqa_swz(4n + q4) of key 4n + q4.  Tiles in the list
  // hold a valid slot, so kv_len >= 1 and row0 (idx 0) is a row of the cache:
  // empty slots load it and get probability 0.
  auto dma = [&](int e, int st) {
    const int tile = __builtin_amdgcn_readlane(my_tile, e);
    const uint32_t taddr = gqa_lds_u32(rows + tile * kGqaTile + 8 * q4);
    u32x4 rv[2];
    gqa_b128<0>(rv[0], taddr);
    gqa_b128<16>(rv[1], taddr);
    gqa_lgkm_wait(rv);
    uint8_t* dst = ring + st * kGqaTileBytes;
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      int rw = (int)rv[n / 4][n % 4];
      rw = rw >= 0 ? rw : row0;
      const uint8_t* src = kvb + (int64_t)rw * kGqaRowBytes + 16 * ((lane & 15) ^ gqa_swz(4 * n + q4));
      __builtin_amdgcn_global_load_lds((gqa_gbl_void*)src, (gqa_lds_void*)(dst + n * 1024), 16, 0, 0);
    }
  };

  // Operand offsets in a stage.  K (A of S^T = K Q^T, step st, key block kb):
  // key 16 kb + r, chunk 4 st + g.  V^T (A of O^T = V^T P^T, block 2p + h): lane
  // (g, r) addresses key 4g + (r >> 2) (+16), columns 32p + 8 (r & 3) + 4h .. +3,
  // and receives V[keys 4g .. 4g+3 (16+..)][column 32p + 8 (r >> 2) + 4h + (r & 3)].
  uint32_t k_off[kGqaD / 32], v_off[kGqaD / 32];
#pragma unroll
  for (int st = 0; st < kGqaD / 32; ++st) k_off[st] = r * kGqaRowBytes + 16 * ((4 * st + g) ^ gqa_swz(r));
  {
    const int kk = 4 * g + (r >> 2);
#pragma unroll
    for (int p = 0; p < kGqaD / 32; ++p) v_off[p] = kk * kGqaRowBytes + 16 * ((4 * p + (r & 3)) ^ gqa_swz(kk));
  }

  f32x4 o[kHB][kGqaD / 16];
#pragma unroll
  for (int hb = 0; hb < kHB; ++hb)
#pragma unroll
    for (int i = 0; i < kGqaD / 16; ++i) o[hb][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[kHB], l_run[kHB];
#pragma unroll
  for (int hb = 0; hb < kHB; ++hb) {
    m_run[hb] = -__builtin_huge_valf();
    l_run[hb] = 0.f;
  }
  const float scale_log2 = a.scale_log2;

#pragma unroll
  for (int e = 0; e < kStg - 1; ++e)
    if (e < nmy) dma(e, e);
  for (int e = 0; e < nmy; ++e) {
    // The stage of entry e - 1 is free: its reads retired before its MFMAs.
    if (e + kStg - 1 < nmy) dma(e + kStg - 1, (e + kStg - 1) % kStg);
    const int ahead = min(kStg - 1, nmy - 1 - e);  // entries issued after e
    if (ahead >= 2) gqa_wait_vmcnt<16>();
    else if (ahead == 1) gqa_wait_vmcnt<8>();
    else gqa_wait_vmcnt<0>();
    const uint32_t base = gqa_lds_u32(ring + (e % kStg) * kGqaTileBytes);

    u32x4 kop[2 * (kGqaD / 32)];
    gqa_b128<0>(kop[0], base + k_off[0]);
    gqa_b128<0>(kop[1], base + k_off[1]);
    gqa_b128<0>(kop[2], base + k_off[2]);
    gqa_b128<0>(kop[3], base + k_off[3]);
    gqa_b128<16 * kGqaRowBytes>(kop[4], base + k_off[0]);
    gqa_b128<16 * kGqaRowBytes>(kop[5], base + k_off[1]);
    gqa_b128<16 * kGqaRowBytes>(kop[6], base + k_off[2]);
    gqa_b128<16 * kGqaRowBytes>(kop[7], base + k_off[3]);
    u32x2 vop[kGqaD / 16][2];
#pragma unroll
    for (int p = 0; p < kGqaD / 32; ++p) {
      // Offsets: h = 0 / 1 at +0 / +8 bytes; keys 16.. at +4096.
      gqa_tr<0>(vop[2 * p][0], base + v_off[p]);
      gqa_tr<16 * kGqaRowBytes>(vop[2 * p][1], base + v_off[p]);
      gqa_tr<8>(vop[2 * p + 1][0], base + v_off[p]);
      gqa_tr<16 * kGqaRowBytes + 8>(vop[2 * p + 1][1], base + v_off[p]);
    }
    gqa_lgkm_wait(kop);
#pragma unroll
    for (int i = 0; i < kGqaD / 16; ++i) __asm__ __volatile__("" : "+v"(vop[i][0]), "+v"(vop[i][1]));

    // S^T: lane (g, r) holds keys 4g + i (c[.][0]) and 16 + 4g + i (c[.][1]) of head r.
    f32x4 c[kHB][2];
#pragma unroll
    for (int hb = 0; hb < kHB; ++hb)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < kGqaD / 32; ++st) acc = gqa_mfma<kF16>(kop[4 * kb + st], qb[hb][st], acc);
        c[hb][kb] = acc;
      }
    const uint32_t m = (uint32_t)__builtin_amdgcn_readlane((int)my_mask, e);
    if (m != 0xffffffffu) {
      const uint32_t lo = (m >> (4 * g)) & 15u, hi = (m >> (16 + 4 * g)) & 15u;
#pragma unroll
      for (int hb = 0; hb < kHB; ++hb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          c[hb][0][i] = ((lo >> i) & 1u) ? c[hb][0][i] : -__builtin_huge_valf();
          c[hb][1][i] = ((hi >> i) & 1u) ? c[hb][1][i] : -__builtin_huge_valf();
        }
    }
    // Online softmax in base 2; the lane keeps its share of the sum.
    u32x4 pb[kHB];
#pragma unroll
    for (int hb = 0; hb < kHB; ++hb) {
      float mx = -__builtin_huge_valf();
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = fmaxf(mx, fmaxf(c[hb][0][i], c[hb][1][i]));
      mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
      mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
      const float m_new = fmaxf(m_run[hb], mx * scale_log2);  // sm_scale > 0
      const float m_use = m_new == -__builtin_huge_valf() ? 0.f : m_new;
      const float alpha = fast_exp2(m_run[hb] - m_use);
      m_run[hb] = m_new;
      float pv[8];
      float psum = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pv[i] = fast_exp2(c[hb][0][i] * scale_log2 - m_use);
        pv[4 + i] = fast_exp2(c[hb][1][i] * scale_log2 - m_use);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) psum += pv[i];
      l_run[hb] = l_run[hb] * alpha + psum;
#pragma unroll
      for (int i = 0; i < kGqaD / 16; ++i) o[hb][i] *= alpha;
      pb[hb] = u32x4{gqa_pack<kF16>(pv[0], pv[1]), gqa_pack<kF16>(pv[2], pv[3]), gqa_pack<kF16>(pv[4], pv[5]),
                     gqa_pack<kF16>(pv[6], pv[7])};
    }
    // O^T += V^T P^T: lane (g, r) of block 2p + h accumulates head r, columns
    // 32p + 8g + 4h .. +3.
#pragma unroll
    for (int i = 0; i < kGqaD / 16; ++i) {
      const u32x4 va = {vop[i][0].x, vop[i][0].y, vop[i][1].x, vop[i][1].y};
#pragma unroll
      for (int hb = 0; hb < kHB; ++hb) o[hb][i] = gqa_mfma<kF16>(va, pb[hb], o[hb][i]);
    }
  }

  // Merge the four waves.  A wave's O goes to its own ring (its DMAs and reads
  // have retired), max and sum to mlbuf.
  __builtin_amdgcn_s_waitcnt(0);
  float* ow = reinterpret_cast<float*>(ring);  // [16 kHB heads][128]
#pragma unroll
  for (int hb = 0; hb < kHB; ++hb) {
    float l = l_run[hb];
    l += __shfl_xor(l, 16, kWave);
    l += __shfl_xor(l, 32, kWave);
#pragma unroll
    for (int i = 0; i < kGqaD / 16; ++i)
      *reinterpret_cast<f32x4*>(ow + (16 * hb + r) * kGqaD + 32 * (i / 2) + 8 * g + 4 * (i % 2)) = o[hb][i];
    if (g == 0) {
      mlbuf[(wave * 16 * kHB + 16 * hb + r) * 2] = m_run[hb];
      mlbuf[(wave * 16 * kHB + 16 * hb + r) * 2 + 1] = l;
    }
  }
  __syncthreads();
  // Thread t: head 16 pass + t / 16, columns 8 (t % 16) .. +7.
  constexpr float kLn2 = 0.6931471805599453f;
#pragma unroll
  for (int pass = 0; pass < kHB; ++pass) {
    const int hh = 16 * pass + tid / 16;
    const int c0 = 8 * (tid % 16);
    float mw[kGqaWaves], M = -__builtin_huge_valf();
#pragma unroll
    for (int w = 0; w < kGqaWaves; ++w) {
      mw[w] = mlbuf[(w * 16 * kHB + hh) * 2];
      M = fmaxf(M, mw[w]);
    }
    const float M_use = M == -__builtin_huge_valf() ? 0.f : M;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float wsum = 0.f;
#pragma unroll
    for (int w = 0; w < kGqaWaves; ++w) {
      const float f = fast_exp2(mw[w] - M_use);
      wsum += f * mlbuf[(w * 16 * kHB + hh) * 2 + 1];
      const float* src = reinterpret_cast<const float*>(lds + w * kStg * kGqaTileBytes) + hh * kGqaD + c0;
      const f32x4 x0 = *reinterpret_cast<const f32x4*>(src);
      const f32x4 x1 = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[i] += f * x0[i];
        acc[4 + i] += f * x1[i];
      }
    }
    const int h = h0 + hh;
    if (h < a.Hg) {
      const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
      const int64_t orow = (int64_t)row * a.Hg + h;
      *reinterpret_cast<u32x4*>(a.out + orow * kGqaD + c0) =
          u32x4{gqa_pack<kF16>(acc[0] * inv, acc[1] * inv), gqa_pack<kF16>(acc[2] * inv, acc[3] * inv),
                gqa_pack<kF16>(acc[4] * inv, acc[5] * inv), gqa_pack<kF16>(acc[6] * inv, acc[7] * inv)};
      if (c0 == 0) a.lse[orow] = wsum > 0.f ? (M + fast_log2(wsum)) * kLn2 : -__builtin_huge_valf();
    }
  }
}

template <bool kF16, int kHB, int kStg>
static hipError_t gqa_launch(const GqaArgs& a, hipStream_t stream) {
  constexpr int kMaxLds = gqa_lds_bytes(kStg, kHB, kGqaMaxTiles);
  static_assert(kMaxLds <= 160 * 1024, "LDS");
  const hipError_t e = set_dynamic_lds_once<sparse_gqa_kernel<kF16, kHB, kStg>>(kMaxLds);
  if (e != hipSuccess) return e;
  const int ntiles = (a.topk + kGqaTile - 1) / kGqaTile;
  const dim3 grid((unsigned)((int64_t)a.B * a.S * a.G), (unsigned)((a.Hg + 16 * kHB - 1) / (16 * kHB)));
  hipLaunchKernelGGL((sparse_gqa_kernel<kF16, kHB, kStg>), grid, dim3(kGqaThreads),
                     gqa_lds_bytes(kStg, kHB, ntiles), stream, a);
  return hipGetLastError();
}

int64_t sparse_gqa_max_topk() { return kGqaMaxTopk; }

// Caller validated: 16-bit q / kv / out, 1 <= Hg <= 1024, 1 <= topk <= 8192,
// B * S * G < 2^31, B * Skv * G < 2^31, sm_scale > 0.
hipError_t launch_sparse_gqa(int is_fp16, const void* q, const void* kv, const int32_t* indices,
                             const int32_t* q_len, const int32_t* kv_len, int64_t B, int64_t S, int64_t G, int64_t Hg,
                             int64_t Skv, int64_t topk, float sm_scale, int causal, void* out, float* lse,
                             hipStream_t stream) {
  if (B * S * G == 0 || Hg == 0) return hipSuccess;
  GqaArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.kv = static_cast<const uint16_t*>(kv);
  a.indices = indices;
  a.q_len = q_len;
  a.kv_len = kv_len;
  a.out = static_cast<uint16_t*>(out);
  a.lse = lse;
  a.B = (int)B;
  a.S = (int)S;
  a.G = (int)G;
  a.Hg = (int)Hg;
  a.Skv = (int)Skv;
  a.topk = (int)topk;
  a.causal = causal;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  // Two 16-head blocks per wave share every K and V operand read; one when the
  // group has at most 16 heads.
  if (Hg > 16) return is_fp16 ? gqa_launch<true, 2, 2>(a, stream) : gqa_launch<false, 2, 2>(a, stream);
  return is_fp16 ? gqa_launch<true, 1, 2>(a, stream) : gqa_launch<false, 1, 2>(a, stream);
}

}  // namespace dsa
