// Lightning-indexer logits on gfx950 MFMA.
//
//   logits[b, t, s] = k_scale[b, s] * sum_h w[b, t, h] * ReLU(q[b, t, h, :] . k[b, s, :]),  D in {64, 128}
//
// (examples/deepseek_v4/lightning_indexer.py:291-316; example_lightning_indexer.py:137-142;
// k_scale is the per-token scale of fp8 keys, 1 when absent.)  Masked positions
// -- beyond the causal bound of sparse_mode 3 (lightning_indexer.py:308-314),
// beyond actual_k_len, or on padded query rows -- are written as -inf, so the
// logits feed the top-k selector directly.
//
// Work split.  A 256-thread workgroup (4 waves) owns kTok query tokens (kTokPW
// per wave) and one chunk of keys.  q is stationary: every wave keeps its
// tokens' [H, D] rows in VGPRs as MFMA A operands (16 heads per operand).  k
// streams through a double-buffered LDS tile of 64 keys; each 16-key slice is
// one MFMA B operand.  fp8 e4m3 inputs use one v_mfma_f32_16x16x128_f8f6f4 per
// 16 heads x 16 keys (K = D = 128 in a single instruction); fp16/bf16 inputs use
// D/32 16x16x32 MFMAs.  The K dimension is read with the same lane -> byte
// mapping for A and B, so the dot products do not depend on the hardware's
// internal K order.  k tiles stream two ahead through a 3-buffer LDS ring,
// one barrier per tile.
//
// Head reduction.  fp8: on the matrix cores.  The scores leave the QK MFMA
// scaled per head into [-1, 1] (its E8M0 A scales; fp8 scores are bounded by
// the row sums of |q|), go to f16 with ReLU as the conversion's clamp
// (v_cvt_pk_f16_f32 ... clamp), and form the B operand of a 16x16x32 f16 MFMA
// whose A operand holds the token's 32 head weights (f16, times the heads'
// scales and a per-token power of two) in every row: every row of the result
// is sum_h w[h] ReLU(S[h][key]), accumulated in fp32, two MFMAs per 64 heads.  bf16/fp16 inputs (unbounded scores): fp32 ReLU,
// multiply by w[t, h], sum the lane's 4 head rows, then two cross-lane adds
// over the 4 row groups.  After four 16-key slices lane l holds key l of the
// 64-key tile, so each token's logits go out as one coalesced 256-byte store.
#include <algorithm>

#include "common.hpp"

namespace dsa {

constexpr int kIdxThreads = 256;
constexpr int kIdxWaves = kIdxThreads / kWave;
constexpr int kIdxKeyTile = 64;

enum ElemKind : int { kFp8 = 0, kBf16 = 1, kFp16 = 2 };

// Row bytes and the bytes each lane feeds one 16-row MFMA operand: the 64
// lanes split a key/query row into 4 K-slices (lane group g = lane / 16 takes
// bytes [g * row / 4, (g + 1) * row / 4)).
template <int kKind, int kD>
struct IdxTraits {
  static constexpr int kElem = kKind == kFp8 ? 1 : 2;
  static constexpr int kRowBytes = kD * kElem;
  static constexpr int kLaneBytes = kRowBytes / 4;
};

// LDS row pitch: 16 bytes of padding per key row spreads the 16 rows one
// MFMA operand reads over different banks.
template <int kKind, int kD>
constexpr int lds_pitch() { return IdxTraits<kKind, kD>::kRowBytes + 16; }

// A lane's K-slice of one 16-row operand, as 16-byte pieces.  fp8 with D = 128
// is kept as the 32-byte MFMA operand itself, so no per-instruction copies.
template <int kKind, int kD>
struct Operand {
  static constexpr int kPieces = IdxTraits<kKind, kD>::kLaneBytes / 16;
  static constexpr bool kWhole = kKind == kFp8 && kD == 128;
  i32x8 v;              // kWhole
  u32x4 p[kPieces];     // otherwise
};

template <int kKind, int kD>
__device__ __forceinline__ void set_piece(Operand<kKind, kD>& op, int c, const u32x4& x) {
  if constexpr (Operand<kKind, kD>::kWhole) {
    op.v[4 * c + 0] = (int)x.x; op.v[4 * c + 1] = (int)x.y; op.v[4 * c + 2] = (int)x.z; op.v[4 * c + 3] = (int)x.w;
  } else {
    op.p[c] = x;
  }
}

template <int kKind, int kD>
__device__ __forceinline__ void load_operand_global(Operand<kKind, kD>& op, const uint8_t* p, bool valid) {
#pragma unroll
  for (int c = 0; c < Operand<kKind, kD>::kPieces; ++c)
    set_piece(op, c, valid ? *reinterpret_cast<const u32x4*>(p + 16 * c) : u32x4{0, 0, 0, 0});
}

template <int kKind, int kD>
__device__ __forceinline__ void load_operand_lds(Operand<kKind, kD>& op, const uint8_t* p) {
#pragma unroll
  for (int c = 0; c < Operand<kKind, kD>::kPieces; ++c) set_piece(op, c, *reinterpret_cast<const u32x4*>(p + 16 * c));
}

// fp8 scores come out of the MFMA scaled per head, by 2^-e_h (the E8M0 scale
// of A's rows: lane (g, r) holds row r, one 32-element scale block), with e_h
// chosen so that every score of head h is at most 1: |q . k| <= 448 *
// sum_i |q[h][i]| for e4m3 keys.  ReLU is then the [0, 1] clamp of the
// conversion to f16 (one v_cvt_pk_f16_f32 ... clamp per pair, no separate
// max), the f16 operand of the head-reduction MFMA keeps full precision down to
// 2^-14 of each head's bound, and the head weights carry the 2^e_h back.
//
// scale_a: E8M0 codes of A's scale, byte kOpsel used (fp8 only).
template <int kKind, int kD, int kOpsel = 0>
__device__ __forceinline__ f32x4 mfma_qk(const Operand<kKind, kD>& a, const Operand<kKind, kD>& b, int scale_a) {
  f32x4 c = {0.f, 0.f, 0.f, 0.f};
  if constexpr (Operand<kKind, kD>::kWhole) {
    c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a.v, b.v, c, 0, 0, kOpsel, scale_a, 0, 127);
  } else if constexpr (kKind == kFp8) {
    // One 16x16x128 fp8 MFMA; a D = 64 row leaves half of each lane's K-slice zero.
    const i32x8 av = {(int)a.p[0].x, (int)a.p[0].y, (int)a.p[0].z, (int)a.p[0].w, 0, 0, 0, 0};
    const i32x8 bv = {(int)b.p[0].x, (int)b.p[0].y, (int)b.p[0].z, (int)b.p[0].w, 0, 0, 0, 0};
    c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, c, 0, 0, kOpsel, scale_a, 0, 127);
  } else {
#pragma unroll
    for (int s = 0; s < Operand<kKind, kD>::kPieces; ++s) {
      if constexpr (kKind == kBf16) {
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a.p[s]), __builtin_bit_cast(bf16x8, b.p[s]), c, 0, 0, 0);
      } else {
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a.p[s]), __builtin_bit_cast(f16x8, b.p[s]), c, 0, 0, 0);
      }
    }
  }
  return c;
}

// ReLU of a dot product in one v_med3_f32 (fmaxf adds a NaN-quieting max in
// IEEE mode).  The bound 3e38 is never reached: |q . k| for fp8/bf16/fp16
// inputs is far below it.
__device__ __forceinline__ float relu(float x) { return __builtin_amdgcn_fmed3f(x, 0.f, 3.0e38f); }

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// One v_cvt_pk_f16_f32 (round to nearest even).
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  const f16x2 r = {(_Float16)a, (_Float16)b};
  return __builtin_bit_cast(uint32_t, r);
}

// Two scaled scores (at most 1) to f16 with ReLU: the min / max pair folds into
// the clamp bit of v_cvt_pk_f16_f32, whose [0, 1] clamp is ReLU here.
__device__ __forceinline__ uint32_t relu_f16x2(float a, float b) {
  const f16x2 r = {(_Float16)a, (_Float16)b};
  const f16x2 lo = {(_Float16)0.f, (_Float16)0.f}, hi = {(_Float16)1.f, (_Float16)1.f};
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_elementwise_max(r, lo), hi));
}

// The exponent e_h of head h's score scale: 448 * sum_i |q[h][i]| <= 2^e_h (0
// for a zero row, 25 -- which bounds any e4m3 row, 128 * 448^2 < 2^25 -- for a
// row holding a NaN).
__device__ __forceinline__ int head_score_exponent(float l1) {
  const float bound = 448.f * l1;
  if (!(bound <= 3.0e38f)) return 25;
  if (bound == 0.f) return 0;
  return (int)((__float_as_uint(bound) >> 23) & 0xff) - 127 + 1;  // bound < 2^(E + 1)
}

// One token's fp8 score scales and reduction weights.  The row sums of |q|
// come from MFMAs of |q| against ones, one head block at a time (few registers
// live): with |q| as A, lane (g, r) receives the sums of heads 16 hb + 4g + i
// (rows 4g + i); with |q| as B -- the same registers, the operand layouts
// mirror each other -- it receives the sum of head 16 hb + r (column r) in
// every component.  In: `w` the fp32 weights of heads 16 hb + 4g + i (lane
// (g, r)), scaled in place to W_h = w_h 2^e_h.  Out: `codes` byte hb = the E8M0
// code 127 - e_h of head 16 hb + r (lane (g, r)'s A row); `wa` = W as the f16
// A operands of the head-reduction MFMAs (block pairs (0, 1) and (2, 3)),
// normalised by a power of two so that max |W| lies in [2^14, 2^15); `post`
// undoes that power at the store.  kFixed: every e_h = 25, which bounds any
// e4m3 row (the sample pass, whose logits only place the filter thresholds).
template <int kD, bool kFixed>
__device__ __forceinline__ void fp8_head_scales(const Operand<kFp8, kD> (&qa)[4], f32x4 (&w)[4], int nhb,
                                                uint32_t& codes, u32x4 (&wa)[2], float& post) {
  Operand<kFp8, kD> ones;
  if constexpr (Operand<kFp8, kD>::kWhole) {
#pragma unroll
    for (int i = 0; i < 8; ++i) ones.v[i] = 0x38383838;  // e4m3 1.0
  } else {
    ones.p[0] = u32x4{0x38383838u, 0x38383838u, 0x38383838u, 0x38383838u};
  }
  float m = 0.f;
  codes = 0;
#pragma unroll
  for (int hb = 0; hb < 4; ++hb) {
    f32x4 rows = {0.f, 0.f, 0.f, 0.f}, cols = {0.f, 0.f, 0.f, 0.f};
    if (!kFixed && hb < nhb) {
      Operand<kFp8, kD> aq;
      if constexpr (Operand<kFp8, kD>::kWhole) {
#pragma unroll
        for (int i = 0; i < 8; ++i) aq.v[i] = qa[hb].v[i] & 0x7f7f7f7f;
      } else {
        aq.p[0] = qa[hb].p[0] & 0x7f7f7f7fu;
      }
      rows = mfma_qk<kFp8, kD>(aq, ones, 127);
      cols = mfma_qk<kFp8, kD>(ones, aq, 127);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = kFixed ? 25 : head_score_exponent(rows[i]);
      w[hb][i] *= __uint_as_float((uint32_t)(127 + e) << 23);
      m = fmaxf(m, fabsf(w[hb][i]));
    }
    codes |= (uint32_t)(127 - (kFixed ? 25 : head_score_exponent(cols.x))) << (8 * hb);
  }
  m = fmaxf(m, __shfl_xor(m, 16, kWave));
  m = fmaxf(m, __shfl_xor(m, 32, kWave));
  // m = 2^e * f with f in [1, 2): weights x 2^(14 - e), results x 2^(e - 14).
  const int e = m > 0.f ? (int)((__float_as_uint(m) >> 23) & 0xff) - 127 : 0;
  const float up = __uint_as_float((uint32_t)(127 + 14 - e) << 23);
  // m, and with it post, is the same in every lane (lane (g, r) saw the weights of heads 4g + i + 16 hb).
  post = __uint_as_float((uint32_t)__builtin_amdgcn_readfirstlane((int)((uint32_t)(127 + e - 14) << 23)));
#pragma unroll
  for (int pr = 0; pr < 2; ++pr)
    wa[pr] = u32x4{pack_f16x2(w[2 * pr].x * up, w[2 * pr].y * up), pack_f16x2(w[2 * pr].z * up, w[2 * pr].w * up),
                   pack_f16x2(w[2 * pr + 1].x * up, w[2 * pr + 1].y * up),
                   pack_f16x2(w[2 * pr + 1].z * up, w[2 * pr + 1].w * up)};
}

// B operand of the head-reduction MFMA for head blocks hb0, hb1: lane (g, r)
// holds key r's ReLU'd scores of heads 16*hb0 + 4g + i and 16*hb1 + 4g + i
// (i < 4) as its K = 8g .. 8g+7.
__device__ __forceinline__ u32x4 relu_operand(const f32x4& c0, const f32x4& c1) {
  return u32x4{relu_f16x2(c0.x, c0.y), relu_f16x2(c0.z, c0.w), relu_f16x2(c1.x, c1.y), relu_f16x2(c1.z, c1.w)};
}

struct IdxArgs {
  const uint8_t* q;        // [B, S1, H, 128]
  const uint8_t* k;        // [B, S2, 128] or paged [blocks, block_size, 128]
  const float* k_scale;    // [B, S2] or paged [blocks, block_size]; nullable
  const float* w;          // [B, S1, H] fp32
  const int32_t* aq_len;   // [B] nullable
  const int32_t* ak_len;   // [B] nullable
  // Packed (TND) rows: inclusive prefix sums of the per-batch lengths, [B];
  // batch b owns query rows cu_q[b-1] .. cu_q[b]-1 of q / weights / logits and
  // key rows cu_k[b-1] .. cu_k[b]-1 of k / k_scale.  Null: padded [B, S1] / [B, S2].
  const int32_t* cu_q;
  const int32_t* cu_k;
  const int32_t* block_table;  // [B, max_blocks] nullable (non-paged)
  float* logits;           // [B, S1, ld]
  int64_t ld;
  int S1, S2, H;
  int block_size, max_blocks;
  int sparse_mode;
  int key_chunk;
  // Fused top-k (indexer_topk_fused): the sample and filter passes, and the
  // dense pass restricted to flagged rows.  Rows are global query rows (q_base + t).
  int tile_stride;          // keys between consecutive tiles: 64, or 64 * F in the sample pass
  float* sample;            // [rows, sample_ld]: logits of the first 64 keys of every 64 * F
  int64_t sample_ld;
  int32_t* row_valid;       // [rows]: valid keys per row (written by the sample pass)
  float* thr;               // [rows]: filter thresholds; the filter pass keeps keys with logit >= thr
  int topk;
  u32x2* cand;              // [rows, nseg, cand_cap]: (logit bits, key position) kept per (row, key chunk), in key order
  int32_t* cand_cnt;        // [rows, nseg]: keys kept (may exceed cand_cap: overflow)
  int cand_cap;
  const int32_t* flag_idx;  // dense pass: only workgroups with a row whose flag_idx[row * flag_ld] is kFallbackFlag
  int64_t flag_ld;
  // With flag_idx: only rows row_lo .. row_hi - 1 count, and only they are stored, at
  // logits + (row - row_lo) * ld (the fused path's bounded fallback buffer, one round).
  int64_t row_lo, row_hi;
  // With flag_idx, or null: the count of flagged rows (zero: every workgroup ends at once).
  const int32_t* flag_count;
};

enum IdxMode : int { kModeDense = 0, kModeSample = 1, kModeFilter = 2, kModeFallback = 3 };

// Scale of every key when the call has none (loaded like a real scale, so the
// load is unconditional).
__device__ float kIdxUnitScale[1] = {1.f};
// kModeFallback exists at launch level only: the fused path's bounded dense
// rounds (flag_idx set), run as indexer_fallback_kernel -- the dense body under
// a name of its own, so that kernel traces tell them from the plain dense pass.

// kNhb = H / 16 head blocks, a compile-time count: no branch between the MFMAs.
// kPaged: keys (and their scales) through the block table; otherwise one
// contiguous [B, S2] run, addressed from per-thread bases and tile offsets.
// Filter threshold of one row, by one wave: the r-th largest valid sampled logit
// rounded down to 16 key bits (sign, exponent, 7 mantissa bits: any threshold
// keeps the result exact, this one only decides how many keys are kept),
// r = mu + 4 sqrt(mu) + 2 with mu = k * sampled / valid the expected number of
// sampled keys in the row's top k; -inf (keep every valid key) when the row has
// at most k valid keys.  Absent samples hold key 0, below every candidate, and
// counts over the wave come from ballots (scalar popcounts).
template <int kPer>
__device__ __forceinline__ float row_threshold(const float* __restrict__ sr, int m, int nv, int k, int lane) {
  uint32_t key[kPer];
  float x[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) x[i] = sr[min(lane + i * kWave, m - 1)];  // no branch: the loads overlap
  int present = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const uint32_t kk = float_key(x[i]);
    const bool ok = lane + i * kWave < m && kk > kKeyInvalidMax;  // absent: past m, NaN, <= -1e30
    key[i] = ok ? kk : 0u;
    // Opaque from here on: otherwise the select is folded into every comparison
    // below (a mask AND, a v_cndmask and a re-compare per element and step).
    __asm__ volatile("" : "+v"(key[i]));
    present += (int)__builtin_popcountll(__builtin_amdgcn_ballot_w64(ok));
  }
  if (nv <= k || present == 0) return -__builtin_huge_valf();
  const float mu = (float)k * (float)present / (float)nv;
  const int r = min((int)ceilf(mu + 4.f * sqrtf(mu) + 2.f), present);
  // The largest x (16 high bits) with #(key >= x) >= r, bit by bit.
  uint32_t res = 0u;
  for (int bit = 31; bit >= 16; --bit) {
    const uint32_t cand = res | (1u << bit);
    int c = 0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) c += (int)__builtin_popcountll(__builtin_amdgcn_ballot_w64(key[i] >= cand));
    if (c >= r) res = cand;
  }
  return key_to_float(res);
}

//
// Modes.  Dense: every logit of the chunk to `logits`.  Sample: only the first
// tile of every tile_stride keys, to consecutive slots of `sample` (masked keys
// as -inf), then each row's filter threshold.  Filter: no logits; each wave keeps,
// per token, the valid keys whose logit is >= thr[row] (and > -1e30), appending
// (logit, position) in key order to the row's slot of this key chunk -- a ballot
// prefix gives each lane its slot, so no atomics -- and finally the kept count.
//
// kSplit (dense mode, few query rows): the four waves share the workgroup's
// kTokPW tokens and split each 64-key tile instead, wave w taking keys
// 16 w .. 16 w + 15 -- with one token per row no wave idles.
template <int kKind, int kD, int kTokPW, int kNhb, bool kPaged, int kMode, bool kSplit = false>
__device__ __forceinline__ void indexer_body(const IdxArgs& a) {
  static_assert(!kSplit || kMode == kModeDense, "key split: dense logits only");
  constexpr int kRB = IdxTraits<kKind, kD>::kRowBytes;
  constexpr int kLB = IdxTraits<kKind, kD>::kLaneBytes;
  constexpr int kPitch = lds_pitch<kKind, kD>();
  constexpr int kTok = kSplit ? kTokPW : kTokPW * kIdxWaves;
  constexpr int kTileBytes = kIdxKeyTile * kRB;
  constexpr int kLoads = kTileBytes / 16 / kIdxThreads;  // 16-byte loads per thread per tile
  static_assert(kLoads >= 1, "tile too small");
  __shared__ __align__(16) uint8_t ktile[3][kIdxKeyTile * kPitch];  // ring: tile t in buffer t % 3

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int r = lane & 15;   // MFMA operand row / output column
  const int g = lane >> 4;   // K-slice of the operand, output row group
  const int b = blockIdx.z;
  const int t_base = blockIdx.y * kTok;
  const int tw = kSplit ? 0 : wave * kTokPW;  // this wave's first token, from t_base
  const int key0 = blockIdx.x * a.key_chunk;
  const int key1 = min(a.S2, key0 + a.key_chunk);
  // Row bases of batch b and its real lengths.  Padded layouts write -inf rows
  // up to S1; packed rows past the batch's length belong to the next batch.
  const int64_t q_base = a.cu_q ? (b ? (int64_t)a.cu_q[b - 1] : 0) : (int64_t)b * a.S1;
  const int64_t k_base = a.cu_k ? (b ? (int64_t)a.cu_k[b - 1] : 0) : (int64_t)b * a.S2;
  const int aq = a.cu_q ? min(max(a.cu_q[b] - (int)q_base, 0), a.S1)
                        : (a.aq_len ? min(max(a.aq_len[b], 0), a.S1) : a.S1);
  const int ak = a.cu_k ? min(max(a.cu_k[b] - (int)k_base, 0), a.S2)
                        : (a.ak_len ? min(max(a.ak_len[b], 0), a.S2) : a.S2);
  const int t_rows = a.cu_q ? aq : a.S1;  // rows of this batch that exist in the output
  constexpr int nhb = kNhb;
  // Rows this call stores: every row, or (fallback rounds) row_lo .. row_hi - 1 only.
  const bool ranged = kMode == kModeDense && a.flag_idx;
  auto stored = [&](int t) { return !ranged || (q_base + t >= a.row_lo && q_base + t < a.row_hi); };
  if (ranged) {  // block-uniform: every thread reads the same flags
    typedef const __attribute__((address_space(4))) int32_t const_i32;
    if (a.flag_count && *(const_i32*)a.flag_count == 0) return;
    bool any = false;
#pragma unroll
    for (int j = 0; j < kTok; ++j) {
      const int t = t_base + j;
      if (t < t_rows && stored(t)) any |= a.flag_idx[(q_base + t) * a.flag_ld] == kFallbackFlag;
    }
    if (!any) return;
  }
  float* const logits0 = ranged ? a.logits - a.row_lo * a.ld : a.logits;  // row r at logits0 + r * ld
  const int tstride = kMode == kModeSample ? a.tile_stride : kIdxKeyTile;

  // Valid key count per token of this wave (0 for padded rows).
  int nvalid[kTokPW];
  int max_valid = 0;
#pragma unroll
  for (int j = 0; j < kTokPW; ++j) {
    const int t = t_base + tw + j;
    int nv = 0;
    if (t < aq && t < a.S1 && ak > 0) {
      if (a.sparse_mode == 3) {
        const int cl = ak - aq + t + 1;
        nv = cl > 0 ? cl : ak;
      } else {
        nv = ak;
      }
      nv = min(nv, ak);
    }
    nvalid[j] = nv;
  }
  // Workgroup-wide bound for skipping whole key tiles.
  {
    const int tl = min(t_base + kTok, min(aq, a.S1)) - 1;  // last real token
    if (tl >= t_base && ak > 0) {
      if (a.sparse_mode == 3) {
        const int cl = ak - aq + tl + 1;
        max_valid = min(cl > 0 ? cl : ak, ak);
      } else {
        max_valid = ak;
      }
    }
  }

  // Stationary q operands and head weights.  fp8: the weights become the A
  // operands of the head-reduction MFMAs -- every row of A is W (f16), K =
  // 8g + i standing for head 16*hb0 + 4g + i (i < 4) or 16*hb1 + 4g + i - 4 of
  // the block pair (hb0, hb1) = (0, 1) or (2, 3), as in relu_operand -- built
  // with the per-head score scales once q has arrived (fp8_head_scales).
  constexpr bool kMfmaSum = kKind == kFp8;
  Operand<kKind, kD> qa[kTokPW][4];
  f32x4 wv[kTokPW][4];
  u32x4 wa[kTokPW][2];
  float post[kTokPW];
#pragma unroll
  for (int j = 0; j < kTokPW; ++j) {
    const int t = t_base + tw + j;
    const bool tv = t < t_rows;
    const int64_t trow = q_base + (tv ? t : 0);
    f32x4 wt[4];
#pragma unroll
    for (int hb = 0; hb < 4; ++hb) {
      // H need not be a multiple of 16: the last block's missing heads are
      // zero q rows with zero weight, so they add nothing.
      const bool hv = tv && hb < nhb;
      const uint8_t* p = a.q + (trow * a.H + hb * 16 + r) * kRB + g * kLB;
      load_operand_global<kKind, kD>(qa[j][hb], p, hv && hb * 16 + r < a.H);
      const float* wp = a.w + trow * a.H + hb * 16 + 4 * g;
      if (!hv) {
        wt[hb] = f32x4{0.f, 0.f, 0.f, 0.f};
      } else if ((a.H & 15) == 0) {
        wt[hb] = *reinterpret_cast<const f32x4*>(wp);
      } else {
        const int h0 = hb * 16 + 4 * g;
        wt[hb] = f32x4{h0 < a.H ? wp[0] : 0.f, h0 + 1 < a.H ? wp[1] : 0.f, h0 + 2 < a.H ? wp[2] : 0.f,
                       h0 + 3 < a.H ? wp[3] : 0.f};
      }
    }
    post[j] = 1.f;
#pragma unroll
    for (int hb = 0; hb < 4; ++hb) wv[j][hb] = wt[hb];
  }

  const int tile_end = min(key1, max_valid);  // keys at or past this are -inf for every token
  const int ntiles = tile_end > key0 ? (tile_end - key0 + tstride - 1) / tstride : 0;

  // Filter mode: this wave's tokens' thresholds, kept counts and candidate slots.
  float thr[kTokPW];
  int kept[kTokPW];
  u32x2* crow[kTokPW];
#pragma unroll
  for (int j = 0; j < kTokPW; ++j) {
    const int t = t_base + tw + j;
    kept[j] = 0;
    crow[j] = kMode == kModeFilter ? a.cand + ((q_base + t) * gridDim.x + blockIdx.x) * a.cand_cap : nullptr;
    // Raised to the float just above -1e30: v >= thr then also rejects masked keys
    // (-inf), scores the top-k never selects (<= -1e30) and NaN.
    thr[j] = (kMode == kModeFilter && t < t_rows) ? fmaxf(a.thr[q_base + t], __uint_as_float(0xF149F2C9u))
                                                  : __builtin_huge_valf();
    thr[j] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(thr[j])));  // wave-uniform
  }

  // Global -> register staging, two tiles in flight: tile t lands in
  // stage[t & 1] two tiles ahead of its use and goes to LDS one tile ahead.
  u32x4 stage[2][kLoads];
  // Thread tid stages 16-byte element tid + 256 i of a tile: key row
  // tid / (kRB/16) + i * (256 / (kRB/16)), column tid % (kRB/16).
  constexpr int kRowsPerLoad = kIdxThreads / (kRB / 16);
  const int kr0 = tid / (kRB / 16);
  const uint8_t* kthread = a.k + (k_base + key0 + kr0) * kRB + (tid % (kRB / 16)) * 16;
  // The key whose scale this lane applies in the epilogue of a tile (at this offset).
  const int sc_off = kSplit ? 16 * wave + r : lane;
  // Scale of key tile * tstride + sc_off of the chunk (1 past the valid keys or without scales).
  auto load_scale = [&](int tile, int blk) -> float {
    const int ss = key0 + tile * tstride + sc_off;
    if (!a.k_scale || ss >= tile_end) return 1.f;
    if constexpr (kPaged) {
      if (!kSplit) blk = a.block_table[(int64_t)b * a.max_blocks + ss / a.block_size];
      return a.k_scale[(int64_t)blk * a.block_size + ss % a.block_size];
    } else {
      return a.k_scale[k_base + ss];
    }
  };
  // kSplit, whose steps hold little work to hide a load behind: the scales of the
  // tiles in the two staging slots, loaded with their keys; with paged keys a
  // fetch also takes its block ids (of this thread's key rows and of its scale
  // key) from the previous fetch, which issues them before its own key rows, so
  // waiting for them never waits for key rows.  Every load of a kSplit fetch is
  // issued whatever the tile (clamped to the last valid key, as kUL below), so
  // that the compiler can count the loads behind each one.
  float scl[2] = {1.f, 1.f};
  int bid[kLoads], sbid = 0;
  // Key scales without a branch per load: without scales every index maps to
  // the one unit scale.
  const float* const ks_base = a.k_scale ? a.k_scale : kIdxUnitScale;
  const int64_t ks_mul = a.k_scale ? 1 : 0;
  auto block_ids = [&](int tile, int (&ids)[kLoads], int& sid) {
    const int64_t tb = (int64_t)b * a.max_blocks;
    const int base = key0 + tile * tstride;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int s = min(max(base + kr0 + i * kRowsPerLoad, key0), tile_end - 1);  // clamped: always a real entry
      ids[i] = a.block_table[tb + s / a.block_size];
    }
    const int ss = min(max(base + sc_off, key0), tile_end - 1);
    sid = a.block_table[tb + ss / a.block_size];
  };
  if constexpr (kPaged && kSplit) {
    if (ntiles > 0) block_ids(0, bid, sbid);
  }
  auto fetch = [&](auto slot_c, int tile) {
    constexpr int slot = decltype(slot_c)::value;
    const int rows_left = tile_end - key0 - tile * tstride;  // block-uniform
    if constexpr (kSplit) {
      // The scale first: a wait for it (the compiler copies these registers
      // across the loop's back edge) then never waits for this fetch's keys.
      const int ss = min(key0 + tile * tstride + sc_off, tile_end - 1);
      const int64_t si = kPaged ? (int64_t)sbid * a.block_size + ss % a.block_size : k_base + ss;
      scl[slot] = ks_base[si * ks_mul];
    }
    int nid[kLoads], nsid = sbid;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) nid[i] = bid[i];
    if constexpr (kPaged && kSplit) block_ids(min(tile + 1, ntiles - 1), nid, nsid);
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int kr = kr0 + i * kRowsPerLoad;    // key row in tile
      if constexpr (kSplit) {
        const int s = key0 + tile * tstride + min(kr, max(rows_left, 1) - 1);  // a valid key
        const int64_t rowi = kPaged ? (int64_t)bid[i] * a.block_size + s % a.block_size : k_base + s;
        stage[slot][i] = *reinterpret_cast<const u32x4*>(a.k + rowi * kRB + (tid % (kRB / 16)) * 16);
        continue;
      }
      u32x4 v = {0, 0, 0, 0};
      if (kr < rows_left) {
        if constexpr (kPaged) {
          const int s = key0 + tile * tstride + kr;
          const int blk = kSplit ? bid[i] : a.block_table[(int64_t)b * a.max_blocks + s / a.block_size];
          const int64_t rowi = (int64_t)blk * a.block_size + s % a.block_size;
          v = *reinterpret_cast<const u32x4*>(a.k + rowi * kRB + (tid % (kRB / 16)) * 16);
        } else {
          v = *reinterpret_cast<const u32x4*>(kthread + ((int64_t)tile * tstride + i * kRowsPerLoad) * kRB);
        }
      }
      stage[slot][i] = v;
    }
    if constexpr (kSplit) {
      if constexpr (kPaged) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) bid[i] = nid[i];
        sbid = nsid;
      }
    }
  };
  // Contiguous keys, tokens split over the waves (kUL): every load is issued
  // whatever the tile -- rows past the valid keys re-load the last valid row
  // (their logits are masked) and a fetch past the last tile re-loads it -- so
  // the compiler knows how many loads follow each one and waits for exactly the
  // data it needs.  Keys go out two tiles ahead, each tile's key scale one tile
  // ahead (scale slot tile & 1).
  constexpr bool kUL = !kPaged && !kSplit;
  auto fetch_ul = [&](auto slot_c, int tile) {
    constexpr int slot = decltype(slot_c)::value;
    const int rl = max(tile_end - key0 - tile * tstride, 1);
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int kr = min(kr0 + i * kRowsPerLoad, rl - 1);
      stage[slot][i] = *reinterpret_cast<const u32x4*>(a.k + (k_base + key0 + (int64_t)tile * tstride + kr) * kRB +
                                                        (tid % (kRB / 16)) * 16);
    }
  };
  auto scale_ul = [&](auto slot_c, int tile) {
    constexpr int slot = decltype(slot_c)::value;
    const int ss = min(key0 + tile * tstride + sc_off, tile_end - 1);
    scl[slot] = ks_base[(k_base + ss) * ks_mul];
  };
  auto commit = [&](auto slot_c, int buf) {
    constexpr int slot = decltype(slot_c)::value;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int e = tid + i * kIdxThreads;
      const int kr = e / (kRB / 16);
      const int kc = e % (kRB / 16);
      *reinterpret_cast<u32x4*>(&ktile[buf][kr * kPitch + kc * 16]) = stage[slot][i];
    }
  };
  using Slot0 = std::integral_constant<int, 0>;
  using Slot1 = std::integral_constant<int, 1>;

  // fp8: the per-head score scales and the scaled weights, computed once q has
  // arrived -- after the first key tile was requested, so the two latencies
  // overlap, and before the second, which keeps fewer registers live.
  uint32_t qscale[kTokPW];
  if constexpr (kUL) {
    if (ntiles > 0) {
      fetch_ul(Slot0{}, 0);
      scale_ul(Slot0{}, 0);
    }
  } else {
    if (ntiles > 0) fetch(Slot0{}, 0);
  }
#pragma unroll
  for (int j = 0; j < kTokPW; ++j) {
    qscale[j] = 0x7f7f7f7fu;
    if constexpr (kMfmaSum) fp8_head_scales<kD, kMode == kModeSample>(qa[j], wv[j], nhb, qscale[j], wa[j], post[j]);
  }
  if (ntiles > 0) commit(Slot0{}, 0);
  if constexpr (kUL) {
    if (ntiles > 0) fetch_ul(Slot1{}, min(1, ntiles - 1));
  } else if constexpr (kSplit) {
    if (ntiles > 0) fetch(Slot1{}, min(1, ntiles - 1));
  } else {
    if (ntiles > 1) fetch(Slot1{}, 1);
  }
  __syncthreads();

  // One tile of work; kSlot = tile & 1 (the loop runs two tiles per trip, so
  // the staging slots are compile-time).
  auto step = [&](auto slot_c, int tile) {
    constexpr int slot = decltype(slot_c)::value;
    const int buf = tile % 3;
    // This tile's scale: kSplit's from its slot before the fetch below reuses it;
    // kUL's from its slot at the stores (loaded a tile ago); otherwise loaded
    // now, its latency behind the tile's MFMAs.
    float sc_early = 1.f;
    if constexpr (kUL) {
      fetch_ul(slot_c, min(tile + 2, ntiles - 1));
      scale_ul(std::integral_constant<int, slot ^ 1>{}, min(tile + 1, ntiles - 1));
    } else if constexpr (kSplit) {
      sc_early = scl[slot];
      fetch(slot_c, min(tile + 2, ntiles - 1));
    } else {
      sc_early = load_scale(tile, 0);
      if (tile + 2 < ntiles) fetch(slot_c, tile + 2);
    }

    float res[kTokPW];
#pragma unroll
    for (int j = 0; j < kTokPW; ++j) res[j] = 0.f;
#pragma unroll
    for (int si = 0; si < (kSplit ? 1 : kIdxKeyTile / 16); ++si) {
      const int sub = kSplit ? wave : si;
      Operand<kKind, kD> kb;
      load_operand_lds<kKind, kD>(kb, &ktile[buf][(sub * 16 + r) * kPitch + g * kLB]);
#pragma unroll
      for (int j = 0; j < kTokPW; ++j) {
        if constexpr (kMfmaSum) {
          // sum_h w[h] ReLU(S[h][key]) on the matrix cores: A = w in every row,
          // B = the ReLU'd scores, so every row of D holds key r's logit.
          f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int pr = 0; pr < 2; ++pr) {
            if (2 * pr < nhb) {
              const f32x4 c0 = pr == 0 ? mfma_qk<kKind, kD, 0>(qa[j][0], kb, qscale[j])
                                       : mfma_qk<kKind, kD, 2>(qa[j][2], kb, qscale[j]);
              const f32x4 c1 = 2 * pr + 1 >= nhb ? f32x4{0.f, 0.f, 0.f, 0.f}
                               : pr == 0        ? mfma_qk<kKind, kD, 1>(qa[j][1], kb, qscale[j])
                                                : mfma_qk<kKind, kD, 3>(qa[j][3], kb, qscale[j]);
              d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, wa[j][pr]),
                                                         __builtin_bit_cast(f16x8, relu_operand(c0, c1)), d, 0, 0, 0);
            }
          }
          res[j] = (kSplit || g == sub) ? d.x : res[j];
        } else {
          float acc2[2] = {0.f, 0.f};  // two chains: head blocks 0, 2 and 1, 3
#pragma unroll
          for (int hb = 0; hb < 4; ++hb) {
            if (hb < nhb) {
              const f32x4 c = mfma_qk<kKind, kD>(qa[j][hb], kb, 127);
              float& acc = acc2[hb & 1];
              acc = fmaf(wv[j][hb].x, relu(c.x), acc);
              acc = fmaf(wv[j][hb].y, relu(c.y), acc);
              acc = fmaf(wv[j][hb].z, relu(c.z), acc);
              acc = fmaf(wv[j][hb].w, relu(c.w), acc);
            }
          }
          float acc = acc2[0] + acc2[1];
          acc += __shfl_xor(acc, 16, kWave);
          acc += __shfl_xor(acc, 32, kWave);
          res[j] = (kSplit || g == sub) ? acc : res[j];
        }
      }
    }
    // kUL, kSplit: the next tile goes to LDS before this one's stores, so that
    // waiting for its keys never waits for stores issued after them.
    if constexpr (kUL || kSplit) {
      if (tile + 1 < ntiles) commit(std::integral_constant<int, slot ^ 1>{}, (tile + 1) % 3);
    }
    // Lane l now holds key (tile * tstride + l) of the chunk for each token
    // (kSplit: lane (g, r) of wave w holds key 16 w + r, and group 0 stores it).
    const int s = key0 + tile * tstride + sc_off;
    const bool storer = !kSplit || g == 0;
    const float sc = kUL ? scl[slot] : sc_early;
#pragma unroll
    for (int j = 0; j < kTokPW; ++j) {
      const int t = t_base + tw + j;
      const float v = (s < nvalid[j]) ? res[j] * (sc * post[j]) : -__builtin_huge_valf();
      if constexpr (kMode == kModeDense) {
        if (storer && t < t_rows && s < key1 && stored(t))
          __builtin_nontemporal_store(v, &logits0[(q_base + t) * a.ld + s]);
      } else if constexpr (kMode == kModeSample) {
        if (t < t_rows && s < key1)
          a.sample[(q_base + t) * a.sample_ld + (int64_t)(key0 / tstride + tile) * kIdxKeyTile + lane] = v;
      } else {
        // Masked keys (s >= nvalid, which covers keys past the chunk: chunks are
        // whole tiles) hold -inf and fail v >= thr; thr is +inf on padded rows.
        const bool keep = v >= thr[j];
        const uint64_t bal = __builtin_amdgcn_ballot_w64(keep);
        if (bal) {  // wave-uniform
          const int pos = kept[j] + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
          if (keep && pos < a.cand_cap) crow[j][pos] = u32x2{__float_as_uint(v), (uint32_t)s};
          kept[j] += (int)__builtin_popcountll(bal);
        }
      }
    }
    // Buffer (tile + 1) % 3 was last read two tiles ago, before the previous barrier.
    if constexpr (!kUL && !kSplit) {
      if (tile + 1 < ntiles) commit(std::integral_constant<int, slot ^ 1>{}, (tile + 1) % 3);
    }
    __syncthreads();
  };
  // Pairs of tiles, the odd last one after the loop: with a conditional second
  // step the loop's back edge could follow the first step alone, and the
  // compiler waited at the top of every trip for the loads that path leaves
  // in flight.
  int tile = 0;
  for (; tile + 1 < ntiles; tile += 2) {
    step(Slot0{}, tile);
    step(Slot1{}, tile + 1);
  }
  if (tile < ntiles) step(Slot0{}, tile);

  if constexpr (kMode == kModeDense) {
    // Keys of this chunk past every token's bound: -inf.
    const int masked0 = key0 + ntiles * kIdxKeyTile;
#pragma unroll
    for (int j = 0; j < kTokPW; ++j) {
      const int t = t_base + tw + j;
      if (t < t_rows && stored(t)) {
        float* row = logits0 + (q_base + t) * a.ld;
        for (int s = masked0 + (kSplit ? tid : lane); s < key1; s += kSplit ? kIdxThreads : kWave)
          __builtin_nontemporal_store(-__builtin_huge_valf(), &row[s]);
      }
    }
  } else if constexpr (kMode == kModeSample) {
    // Sample slots of this chunk's tiles past every token's bound: -inf.
    const int slot0 = key0 / tstride * kIdxKeyTile;
    const int slot1 = (key1 + tstride - 1) / tstride * kIdxKeyTile;
#pragma unroll
    for (int j = 0; j < kTokPW; ++j) {
      const int t = t_base + tw + j;
      if (t < t_rows) {
        float* row = a.sample + (q_base + t) * a.sample_ld;
        for (int c = slot0 + ntiles * kIdxKeyTile + lane; c < slot1; c += kWave) row[c] = -__builtin_huge_valf();
        if (blockIdx.x == 0 && lane == 0) a.row_valid[q_base + t] = nvalid[j];
      }
    }
    // fused_threshold_kernel turns the rows' samples into thresholds afterwards.
  } else {
#pragma unroll
    for (int j = 0; j < kTokPW; ++j) {
      const int t = t_base + tw + j;
      if (t < t_rows && lane == 0) a.cand_cnt[(q_base + t) * gridDim.x + blockIdx.x] = kept[j];
    }
  }
}

// fp8 with D = 128 is held to three waves per SIMD (the compiler would
// otherwise trade a wave for a deeper operand prefetch); the key split, with
// one token's operands per wave, leaves the compiler free.
template <int kKind, int kD, int kTokPW, int kNhb, bool kPaged, int kMode, bool kSplit = false>
__global__ __launch_bounds__(kIdxThreads)
__attribute__((amdgpu_waves_per_eu(kKind == kFp8 && kD == 128 && !kSplit ? 3 : 1,
                                   kKind == kFp8 && kD == 128 && !kSplit ? 3 : 8)))
void indexer_logits_kernel(IdxArgs a) {
  indexer_body<kKind, kD, kTokPW, kNhb, kPaged, kMode, kSplit>(a);
}

// The fp8 filter pass, held to the dense pass's three waves per SIMD (its few
// extra registers would otherwise cost a wave).
template <int kD, int kTokPW, int kNhb, bool kPaged>
__global__ __launch_bounds__(kIdxThreads) __attribute__((amdgpu_waves_per_eu(3, 3)))
void indexer_filter_fp8_kernel(IdxArgs a) {
  indexer_body<kFp8, kD, kTokPW, kNhb, kPaged, kModeFilter>(a);
}

// The fused path's fallback rounds: the dense pass under its own kernel name.
template <int kKind, int kD, int kTokPW, int kNhb, bool kPaged>
__global__ __launch_bounds__(kIdxThreads)
__attribute__((amdgpu_waves_per_eu(kKind == kFp8 && kD == 128 ? 3 : 1, kKind == kFp8 && kD == 128 ? 3 : 8)))
void indexer_fallback_kernel(IdxArgs a) {
  indexer_body<kKind, kD, kTokPW, kNhb, kPaged, kModeDense>(a);
}

// Query rows per batch up to which dense logits split each key tile over the
// waves (one token per workgroup) instead of giving each wave its own tokens.
constexpr int kIdxSplitRows = 4;

template <int kKind, int kD>
static hipError_t launch_indexer_split(const IdxArgs& a, int B, hipStream_t stream) {
  const dim3 grid((unsigned)((a.S2 + a.key_chunk - 1) / a.key_chunk), (unsigned)a.S1, (unsigned)B);
#define DSA_IDX(N, P) \
  hipLaunchKernelGGL((indexer_logits_kernel<kKind, kD, 1, N, P, kModeDense, true>), grid, dim3(kIdxThreads), 0, stream, a)
#define DSA_IDX2(N) \
  if (a.block_table) DSA_IDX(N, true); else DSA_IDX(N, false)
  switch ((a.H + 15) >> 4) {
    case 1: DSA_IDX2(1); break;
    case 2: DSA_IDX2(2); break;
    case 3: DSA_IDX2(3); break;
    default: DSA_IDX2(4); break;
  }
#undef DSA_IDX2
#undef DSA_IDX
  return hipGetLastError();
}

template <int kKind, int kD, int kMode = kModeDense>
static hipError_t launch_indexer_kind(const IdxArgs& a, int B, hipStream_t stream) {
  if constexpr (kMode == kModeDense || kMode == kModeFallback)
    if (a.S1 <= kIdxSplitRows) return launch_indexer_split<kKind, kD>(a, B, stream);
  constexpr int kTokPW = 2;
  constexpr int kTok = kTokPW * kIdxWaves;
  const dim3 grid((unsigned)((a.S2 + a.key_chunk - 1) / a.key_chunk), (unsigned)((a.S1 + kTok - 1) / kTok), (unsigned)B);
#define DSA_IDX(N, P)                                                                                           \
  if constexpr (kKind == kFp8 && kMode == kModeFilter)                                                          \
    hipLaunchKernelGGL((indexer_filter_fp8_kernel<kD, kTokPW, N, P>), grid, dim3(kIdxThreads), 0, stream, a);   \
  else if constexpr (kMode == kModeFallback)                                                                    \
    hipLaunchKernelGGL((indexer_fallback_kernel<kKind, kD, kTokPW, N, P>), grid, dim3(kIdxThreads), 0, stream, a); \
  else                                                                                                          \
    hipLaunchKernelGGL((indexer_logits_kernel<kKind, kD, kTokPW, N, P, kMode>), grid, dim3(kIdxThreads), 0, stream, a)
#define DSA_IDX2(N) \
  if (a.block_table) DSA_IDX(N, true); else DSA_IDX(N, false)
  switch ((a.H + 15) >> 4) {
    case 1: DSA_IDX2(1); break;
    case 2: DSA_IDX2(2); break;
    case 3: DSA_IDX2(3); break;
    default: DSA_IDX2(4); break;
  }
#undef DSA_IDX2
#undef DSA_IDX
  return hipGetLastError();
}

static IdxArgs make_idx_args(const void* q, const void* k, const float* k_scale, const float* w, int64_t S1,
                             int64_t S2, int64_t H, const int32_t* aq_len, const int32_t* ak_len, const int32_t* cu_q,
                             const int32_t* cu_k, const int32_t* block_table, int64_t block_size, int64_t max_blocks,
                             int sparse_mode) {
  IdxArgs a = {};
  a.q = static_cast<const uint8_t*>(q);
  a.k = static_cast<const uint8_t*>(k);
  a.k_scale = k_scale;
  a.w = w;
  a.aq_len = aq_len;
  a.ak_len = ak_len;
  a.cu_q = cu_q;
  a.cu_k = cu_k;
  a.block_table = block_table;
  a.S1 = (int)S1;
  a.S2 = (int)S2;
  a.H = (int)H;
  a.block_size = (int)block_size;
  a.max_blocks = (int)max_blocks;
  a.sparse_mode = sparse_mode;
  a.tile_stride = kIdxKeyTile;
  return a;
}

// Keys per workgroup: enough workgroups to fill 256 CUs several times over.
// split: one token per workgroup (dense logits of few query rows).
static int64_t indexer_key_chunk(int64_t B, int64_t S1, int64_t S2, bool split = false) {
  const int64_t tok_groups = B * (split ? S1 : (S1 + 7) / 8);
  const int64_t chunks = (2048 + tok_groups - 1) / tok_groups;
  int64_t chunk = (S2 + chunks - 1) / chunks;
  chunk = ((chunk + kIdxKeyTile - 1) / kIdxKeyTile) * kIdxKeyTile;
  return chunk < 1024 ? 1024 : chunk;
}

template <int kMode>
static hipError_t launch_indexer_mode(int kind, int64_t D, const IdxArgs& a, int64_t B, hipStream_t stream) {
  const bool d128 = (D == 128);
  switch (kind) {
    case kFp8: return d128 ? launch_indexer_kind<kFp8, 128, kMode>(a, (int)B, stream)
                           : launch_indexer_kind<kFp8, 64, kMode>(a, (int)B, stream);
    case kBf16: return d128 ? launch_indexer_kind<kBf16, 128, kMode>(a, (int)B, stream)
                            : launch_indexer_kind<kBf16, 64, kMode>(a, (int)B, stream);
    case kFp16: return d128 ? launch_indexer_kind<kFp16, 128, kMode>(a, (int)B, stream)
                            : launch_indexer_kind<kFp16, 64, kMode>(a, (int)B, stream);
    default: return hipErrorInvalidValue;
  }
}

// kind: 0 fp8 e4m3fn, 1 bf16, 2 fp16.  Caller validated: D in {64, 128}, 1 <= H <= 64.
hipError_t launch_indexer_logits(int kind, const void* q, const void* k, const float* k_scale, const float* w,
                                 int64_t B, int64_t S1, int64_t S2, int64_t H, int64_t D,
                                 const int32_t* aq_len, const int32_t* ak_len, const int32_t* cu_q,
                                 const int32_t* cu_k, const int32_t* block_table, int64_t block_size,
                                 int64_t max_blocks, int sparse_mode, float* logits, int64_t ld, hipStream_t stream) {
  if (B == 0 || S1 == 0 || S2 == 0) return hipSuccess;
  IdxArgs a = make_idx_args(q, k, k_scale, w, S1, S2, H, aq_len, ak_len, cu_q, cu_k, block_table, block_size,
                            max_blocks, sparse_mode);
  a.logits = logits;
  a.ld = ld;
  a.key_chunk = (int)indexer_key_chunk(B, S1, S2, S1 <= kIdxSplitRows);
  return launch_indexer_mode<kModeDense>(kind, D, a, B, stream);
}

// ---------------------------------------------------------------------------
// Fused indexer -> top-k.  The logits of a row are never written whole:
//   1. sample pass: the logits of the first 64 keys of every 64 F (1024 to
//      2048 keys per row);
//   2. per row, in a kernel of its own (the sample spans several workgroups):
//      thr = the r-th largest valid sampled logit, r = mu + 4 sqrt(mu) + 2 with
//      mu = k * sampled / valid the expected number of sampled keys in the
//      row's top k (thr = -inf when the row has at most k valid keys);
//   3. filter pass: the indexer again, keeping (logit, key) for logit >= thr,
//      per (row, key chunk) in key order (at most four chunks a row);
//   4. per row, the kept keys of all chunks read in key order as one packed
//      row; the row is flagged when a chunk overflowed, when more keys were kept
//      than a packed row holds, or when thr is finite and fewer than k keys
//      reached it -- otherwise every key outside the kept set is below thr,
//      which is at most the k-th largest logit, so the top k (ties to the
//      lower index included) lie in the kept set;
//   5. k <= 4096: the register top-k over those rows where the filter left
//      them (positions map back to keys), and the exact radix top-k over packed
//      copies of the rows it could not bound (ties); k > 4096: every row packed,
//      then the exact radix top-k over the packed rows;
//   6. rows flagged in step 4 only, in rounds of consecutive rows: their dense
//      logits into a bounded buffer (the candidate slots, dead by then) and the
//      exact radix top-k -- an early exit per workgroup when nothing is flagged.
// Steps 5-6 give the same output as the dense path bit for bit.
hipError_t launch_topk_candidates(const CandSegments& cs, int64_t rows, int64_t k, int32_t* out_idx,
                                  float* out_val, hipStream_t stream);
hipError_t launch_topk_packed(const CandSegments& cs, int64_t rows, int64_t k, int32_t* out_idx, float* out_val,
                              hipStream_t stream);
hipError_t launch_topk_flagged(const float* x, int64_t ld, int64_t rows, int64_t n, int64_t k, int32_t* out_idx,
                               float* out_val, hipStream_t stream, const int32_t* gate);

// Sampled tiles per row: S2 / (2 k) clamped to [16, 32], so that mu = k * sampled / S2 stays
// at least 32 where the row allows it (a smaller mu widens the spread of the kept count
// relative to its mean, and rows whose kept keys outrun ldc = 4 k go back to the dense
// path: 8 tiles at 131072 keys, k = 2048, sent 2% of the rows back), while short rows
// sample half as many keys as long ones (C2: the sample pass at 1/32 of the keys, not 1/16).
constexpr int kFusedSampleTilesMin = 16;
constexpr int kFusedSampleTilesMax = 32;
// Key chunks (candidate slots) per row: four keep the filter pass's grid at thousands
// of workgroups for long rows (two cost C5 10%: 3.50 -> 3.84 ms); past the register
// top-k's k, whose slots are twice as large, two.
constexpr int kFusedMaxSeg = 4;
constexpr int kFusedMaxSegLargeK = 2;
static_assert(kFusedMaxSeg <= kCandMaxSeg, "the register top-k walks at most kCandMaxSeg chunks");
constexpr int kFusedSampleChunkTiles = 8;  // sampled tiles per workgroup of the sample pass
constexpr int kFusedMaxK = 8192;
constexpr int kFusedRegK = 4096;           // largest k the register top-k takes (beyond: radix)
constexpr size_t kFusedMinFallback = size_t(64) << 20;  // dense-fallback rows per round: at least 64 MB

struct FusedPlan {
  bool fused;
  int64_t rows, ld, sample_ld, ldc;
  int64_t key_chunk, tile_stride;
  int nseg, cap;
  int64_t fb_rows;  // rows per dense-fallback round
  int rounds;
  size_t cval, sample, thr, valid, ccnt, pval, pidx, plen, counts, total;
};

static size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// rows: B * S1 (padded queries) or T (packed queries, S1 = the longest batch).
static FusedPlan fused_plan(int64_t rows, int64_t B, int64_t S1, int64_t S2, int64_t k) {
  FusedPlan p = {};
  p.rows = rows;
  p.ld = (S2 + 3) & ~int64_t(3);
  const int max_seg = k <= kFusedRegK ? kFusedMaxSeg : kFusedMaxSegLargeK;
  const int64_t min_chunk = ((S2 + max_seg - 1) / max_seg + kIdxKeyTile - 1) / kIdxKeyTile * kIdxKeyTile;
  p.key_chunk = indexer_key_chunk(B, S1, S2);
  if (p.key_chunk < min_chunk) p.key_chunk = min_chunk;
  p.nseg = (int)((S2 + p.key_chunk - 1) / p.key_chunk);
  const int64_t tiles = (S2 + kIdxKeyTile - 1) / kIdxKeyTile;
  const int64_t sample_tiles = std::min<int64_t>(std::max<int64_t>(S2 / (2 * k), kFusedSampleTilesMin),
                                                 kFusedSampleTilesMax);
  const int64_t F = tiles / sample_tiles > 1 ? tiles / sample_tiles : 1;
  p.tile_stride = F * kIdxKeyTile;
  p.sample_ld = (S2 + p.tile_stride - 1) / p.tile_stride * kIdxKeyTile;  // <= 4096: F >= tiles / 64
  // Packed-row capacity: 4 k for the register top-k, 2 k + 2048 past it (radix top-k).
  // A chunk's slot holds 2 k + 1024 (resp. a whole packed row) -- more than the kept
  // count of a whole row (about 1.8 k at C5, 1.4 k at k = 8192), so only a row whose
  // kept keys crowd into one chunk past that overflows (and goes back to its dense logits).
  const int64_t cap_k = k <= kFusedRegK ? (2 * k + 1024 + 63) & ~int64_t(63) : (2 * k + 2048 + 63) & ~int64_t(63);
  p.ldc = k <= kFusedRegK ? ((4 * k + 4095) / 4096) * 4096 : cap_k;
  p.cap = (int)std::min<int64_t>(p.key_chunk, cap_k);
  p.fused = k <= kFusedMaxK && S2 >= 16384 && S2 >= 8 * k && p.nseg <= max_seg &&
            (k > kFusedRegK || p.ldc <= 32768) && p.sample_ld <= 4096 && p.rows > 0;
  if (!p.fused) return p;
  const size_t R = (size_t)p.rows;
  // The candidate slots, which the dense-fallback rounds reuse once the top-k has read them.
  const size_t slots = R * p.nseg * p.cap * 8;
  const size_t row_bytes = (size_t)p.ld * 4;
  p.fb_rows = (int64_t)(std::max(slots, kFusedMinFallback) / row_bytes);
  if (p.fb_rows < 1) p.fb_rows = 1;
  if (p.fb_rows > p.rows) p.fb_rows = p.rows;
  p.rounds = (int)((p.rows + p.fb_rows - 1) / p.fb_rows);
  size_t off = 0;
  p.cval = off; off = align256(off + std::max(slots, (size_t)p.fb_rows * row_bytes));
  p.sample = off; off = align256(off + R * p.sample_ld * 4);
  p.thr = off; off = align256(off + R * 4);
  p.valid = off; off = align256(off + R * 4);
  p.ccnt = off; off = align256(off + R * p.nseg * 4);
  p.pval = off; off = align256(off + R * p.ldc * 4);
  p.pidx = off; off = align256(off + R * p.ldc * 4);
  p.plen = off; off = align256(off + R * 4);
  p.counts = off; off = align256(off + 2 * 4);  // rows spilled to the radix kernel, rows sent back
  p.total = off;
  return p;
}

// 0 when the fused path does not apply to this shape (the caller runs the dense path).
size_t indexer_topk_fused_bytes(int64_t rows, int64_t B, int64_t S1, int64_t S2, int64_t k) {
  const FusedPlan p = fused_plan(rows, B, S1, S2, k);
  return p.fused ? p.total : 0;
}

// Thresholds after a sample pass of several key chunks: one wave per row.
// It also clears the two row counters of the top-k passes behind it (no memset: graph capture).
__global__ __launch_bounds__(256) void fused_threshold_kernel(const float* __restrict__ sample, int64_t sld,
                                                              const int32_t* __restrict__ row_valid, int64_t rows,
                                                              int k, float* __restrict__ thr,
                                                              int32_t* __restrict__ counts) {
  const int lane = threadIdx.x & (kWave - 1);
  if (blockIdx.x == 0 && threadIdx.x < 2) counts[threadIdx.x] = 0;
  const int64_t row = (int64_t)blockIdx.x * (256 / kWave) + threadIdx.x / kWave;
  if (row >= rows) return;
  const float* sr = sample + row * sld;
  const float t = sld <= 16 * kWave   ? row_threshold<16>(sr, (int)sld, row_valid[row], k, lane)
                  : sld <= 32 * kWave ? row_threshold<32>(sr, (int)sld, row_valid[row], k, lane)
                                      : row_threshold<64>(sr, (int)sld, row_valid[row], k, lane);
  if (lane == 0) thr[row] = t;
}

__global__ __launch_bounds__(256) void fused_count_flagged_kernel(const int32_t* __restrict__ plen, int64_t rows,
                                                                  int32_t* __restrict__ count) {
  __shared__ int part[256 / kWave];
  int c = 0;
  for (int64_t r = threadIdx.x; r < rows; r += 256) c += plen[r] < 0;
  c = wave_sum_i(c);
  if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = c;
  __syncthreads();
  if (threadIdx.x == 0) count[0] = part[0] + part[1] + part[2] + part[3];
}

// Rows of the last fused call on `workspace` that went back to the dense logits because
// the sampled threshold was too high or a key chunk overflowed (one int, written on `stream`).
hipError_t launch_fused_fallback_rows(const void* workspace, int64_t rows, int64_t B, int64_t S1, int64_t S2,
                                      int64_t k, int32_t* count, hipStream_t stream) {
  const FusedPlan p = fused_plan(rows, B, S1, S2, k);
  if (!p.fused) return hipErrorInvalidValue;
  const int32_t* plen = reinterpret_cast<const int32_t*>(static_cast<const uint8_t*>(workspace) + p.plen);
  hipLaunchKernelGGL(fused_count_flagged_kernel, dim3(1), dim3(256), 0, stream, plen, p.rows, count);
  return hipGetLastError();
}

// Caller validated as for launch_indexer_logits (padded or packed rows, optional paging), plus
// 1 <= k <= 8192 and a workspace of indexer_topk_fused_bytes bytes.  rows: B * S1, or T with cu_q.
hipError_t launch_indexer_topk_fused(int kind, const void* q, const void* k, const float* k_scale, const float* w,
                                     int64_t rows, int64_t B, int64_t S1, int64_t S2, int64_t H, int64_t D,
                                     const int32_t* aq_len, const int32_t* ak_len, const int32_t* cu_q,
                                     const int32_t* cu_k, const int32_t* block_table, int64_t block_size,
                                     int64_t max_blocks, int sparse_mode, int64_t topk, int32_t* out_idx,
                                     float* out_val, void* workspace, hipStream_t stream) {
  const FusedPlan p = fused_plan(rows, B, S1, S2, topk);
  if (!p.fused || B == 0 || S1 == 0) return hipErrorInvalidValue;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  IdxArgs a = make_idx_args(q, k, k_scale, w, S1, S2, H, aq_len, ak_len, cu_q, cu_k, block_table, block_size,
                            max_blocks, sparse_mode);
  a.sample = reinterpret_cast<float*>(ws + p.sample);
  a.sample_ld = p.sample_ld;
  a.thr = reinterpret_cast<float*>(ws + p.thr);
  a.topk = (int)topk;
  a.cand = reinterpret_cast<u32x2*>(ws + p.cval);
  a.cand_cnt = reinterpret_cast<int32_t*>(ws + p.ccnt);
  a.cand_cap = p.cap;
  // 1-2. Sample pass (tiles tile_stride apart, kFusedSampleChunkTiles per workgroup), then
  // the thresholds.
  a.tile_stride = (int)p.tile_stride;
  a.row_valid = reinterpret_cast<int32_t*>(ws + p.valid);
  a.key_chunk = (int)(p.tile_stride * kFusedSampleChunkTiles);
  hipError_t e = launch_indexer_mode<kModeSample>(kind, D, a, B, stream);
  if (e != hipSuccess) return e;
  int32_t* counts = reinterpret_cast<int32_t*>(ws + p.counts);
  hipLaunchKernelGGL(fused_threshold_kernel, dim3((unsigned)((p.rows + 3) / 4)), dim3(256), 0, stream, a.sample,
                     p.sample_ld, a.row_valid, p.rows, (int)topk, a.thr, counts);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  // 3. Filter pass over the key chunks (one candidate slot per chunk).
  a.tile_stride = kIdxKeyTile;
  a.key_chunk = (int)p.key_chunk;
  if ((e = launch_indexer_mode<kModeFilter>(kind, D, a, B, stream)) != hipSuccess) return e;
  // 4-5. Top-k over the candidates.
  const CandSegments cs = {a.cand, a.cand_cnt, a.thr, p.nseg, p.cap, (int)p.ldc,
                           reinterpret_cast<float*>(ws + p.pval), reinterpret_cast<int32_t*>(ws + p.pidx),
                           reinterpret_cast<int32_t*>(ws + p.plen), counts, counts + 1};
  e = topk <= kFusedRegK ? launch_topk_candidates(cs, p.rows, topk, out_idx, out_val, stream)
                         : launch_topk_packed(cs, p.rows, topk, out_idx, out_val, stream);
  if (e != hipSuccess) return e;
  // 6. Rows still flagged, fb_rows consecutive rows a round: dense logits into the
  // candidate slots (read by now), then the exact radix top-k of those rows.
  float* fb = reinterpret_cast<float*>(ws + p.cval);
  a.logits = fb;
  a.ld = p.ld;
  a.flag_idx = out_idx;
  a.flag_ld = topk;
  a.flag_count = counts + 1;
  a.key_chunk = (int)p.key_chunk;
  for (int rd = 0; rd < p.rounds; ++rd) {
    a.row_lo = (int64_t)rd * p.fb_rows;
    a.row_hi = std::min<int64_t>(p.rows, a.row_lo + p.fb_rows);
    if ((e = launch_indexer_mode<kModeFallback>(kind, D, a, B, stream)) != hipSuccess) return e;
    if ((e = launch_topk_flagged(fb, p.ld, a.row_hi - a.row_lo, S2, topk, out_idx + a.row_lo * topk,
                                 out_val ? out_val + a.row_lo * topk : nullptr, stream, counts + 1)) != hipSuccess)
      return e;
  }
  return hipSuccess;
}

}  // namespace dsa
