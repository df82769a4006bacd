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
// of up to 128 heads); a wave owns 32 heads (two 16-head MFMA blocks that share
// every K and V operand read from LDS) and keeps their Q rows in registers, the
// O accumulators (32 x 512 fp32) in AGPRs: one wave per SIMD.
//
// Gather.  The workgroup first turns its slots into physical KV row numbers
// (index -> validity -> block table) in LDS, once.  Tiles of 32 slots then
// stream HBM -> LDS with global_load_lds_dwordx4 (no VGPR staging) through a
// 4-stage ring, up to three tiles ahead of the MFMAs; each wave waits on its
// own vmcnt, then a barrier publishes the tile.  A tile is 36 blocks of 1 KB,
// each 8 slots x 8 chunks of 16 bytes, XOR-swizzled (lds_swizzle below): one
// DMA instruction fetches 8 whole 128-byte lines, and the 16-slot MFMA
// operand reads are bank-conflict free.  Empty /
// masked slots re-load a valid row of the same workgroup and get probability 0;
// leading tiles with no valid slot are skipped.
//
// Math per tile and wave: S^T = K Q^T with the 32 keys on the MFMA M axis
// (18 x 2 v_mfma_f32_16x16x32_bf16 over d = 576, two accumulator chains), so
// each lane ends up with 8 scores of one head; softmax in base 2 against a
// reference max fixed by the first valid tile (plus a bias: 2^60 for bf16), so
// O is never rescaled in the loop (a score beyond the representable headroom
// sends the workgroup to an exact two-pass fallback).  P to bf16 is the lane's
// own B operand of O^T += V^T P^T; V^T comes straight from the row-major tile
// through ds_read_b64_tr_b16 (4x4 transposes across lane quads), two reads per
// 16 output columns, and each lane ends up holding 8 consecutive output
// columns of one head, stored straight from registers.  The tile loop runs in
// two phases: the QK MFMAs of tile t+1 with the DMA of tile t+kDepth spread
// between them, then the PV MFMAs of tile t with the softmax of tile t+1 cut
// into slices between them.  With more than one split a workgroup writes a
// normalised bf16 partial and its LSE; a combine kernel merges them.
//
// The 512-wide row lists of up to 64 heads (one or two waves) run the same
// body from a two-stage ring instead (sparse_mla_rows2_kernel): one tile is
// computed at a time while the next arrives, in 73 KB of LDS, so that two
// workgroups share a CU and every SIMD holds a wave.
#include "common.hpp"

namespace dsa {

constexpr int kMlaDV = 512;
constexpr int kMlaTile = 32;                       // slots per tile
constexpr int kStages = 4;
constexpr int kAhead = kStages - 1;                // tiles in flight ahead of compute
constexpr int kSlotsCap = 2048;                    // slots per workgroup (physical rows kept in LDS)
// Rows with this bit set live in the second KV source (MlaArgs::kv2).
constexpr int32_t kSrc2Bit = 0x40000000;

// Geometry of a KV row of kD 16-bit elements: 576 (latent 512 + rope 64,
// DeepSeek V3.2) or 512 (V4: K = V, no rope tail).  V is always the first 512.
template <int kD>
struct MlaGeom {
  static_assert(kD == 576 || kD == 512, "row width");
  static constexpr int kRowBytes = kD * 2;                      // 1152 / 1024
  static constexpr int kRowChunks = kRowBytes / 16;             // 72 / 64
  static constexpr int kStageBytes = kMlaTile * kRowBytes;      // 36864 / 32768
  static constexpr int kTileInstr = kStageBytes / 1024;         // wave-wide 16-byte DMA loads per tile
  static constexpr int kRowsOffset = kStages * kStageBytes;
  static constexpr int kTileMaskOffset = kRowsOffset + kSlotsCap * 4 + 16;  // after rows, overflow flag, first and last valid slot
  static constexpr int kLds = kTileMaskOffset + (kSlotsCap / 32) * 4;       // + one valid-slot bitmask per tile
  static constexpr int kSteps = kD / 32;                        // 32-dim steps of Q K^T
  static constexpr int kQkHalf = 2 * kSteps;                    // half-steps (one K operand read each)
  // V4 (512) reads per-row lists of physical rows from two caches, with
  // per-row slot counts and attention sinks; V3.2 (576) reads index lists into
  // one cache.  Fixed per width, so neither pays for the other's features.
  static constexpr bool kRowLists = kD == 512;
};
// LDS of a workgroup whose ring has kSt stages: the stages, then the slot table
// (physical rows), the flag words and one valid-slot bitmask per tile.
template <int kD, int kSt>
struct MlaLayout {
  static constexpr int kRowsOffset = kSt * MlaGeom<kD>::kStageBytes;
  static constexpr int kTileMaskOffset = kRowsOffset + kSlotsCap * 4 + 16;
  static constexpr int kLds = kTileMaskOffset + (kSlotsCap / 32) * 4;
};
static_assert(MlaLayout<576, kStages>::kLds == MlaGeom<576>::kLds, "the 4-stage layout is MlaGeom's");

// Reference max = first valid tile's max + kRefBias (log2); the fast path accepts
// P up to 2^kOverflowGuard.  bf16 shares fp32's exponent range; fp16 P must stay
// within [2^-14, 65504].
template <bool kF16> struct PRange;
template <> struct PRange<false> { static constexpr float kRefBias = 60.f, kOverflowGuard = 60.f; };
template <> struct PRange<true> { static constexpr float kRefBias = 8.f, kOverflowGuard = 15.f; };
// 2^kOverflowGuard as the bound on a lane's per-tile sum of probabilities.
template <bool kF16> constexpr float kOverflowSumOf = kF16 ? 32768.f : 1152921504606846976.f;
constexpr int kHeadsPerWave = 32;                  // two 16-head MFMA blocks share every K / V operand

struct MlaArgs {
  const uint16_t* q;          // [B, S, H, D] bf16 / fp16
  const uint16_t* kv;         // [B, Skv, D] or paged [blocks, block_size, D]
  const uint16_t* kv2;        // second row source (rows tagged kSrc2Bit) or null
  const int32_t* indices;     // [B, S, topk]; physical rows with row lists (D = 512)
  const int32_t* slot_count;  // [B*S] used slots per row (row lists)
  const float* sinks;         // [H] attention-sink logits (natural log units) or null
  const int32_t* block_table; // [B, max_blocks] or null
  const int32_t* q_len;       // [B] or null
  const int32_t* kv_len;      // [B] or null
  uint16_t* out;              // [B, S, H, 512]
  float* lse;                 // [B, S, H]
  uint16_t* part_o;           // [splits, B*S, H, 512] (splits > 1)
  float* part_lse;            // [splits, B*S, H]
  // Row lists only: when set, out is written here in fp32 instead (and the
  // split partials go to part_o32 in fp32), so no 16-bit rounding is applied.
  float* out32;               // [B, S, H, 512] or null
  float* part_o32;            // [splits, B*S, H, 512] (splits > 1, out32 set)
  int B, S, H, Skv, topk;
  // KV groups (kv_group): query row t = (b * S + s) * G + g reads KV column g
  // through its own index row, heads g * H .. (g + 1) * H - 1 of the caller's q
  // (H here is the heads per group); its physical rows are (pool row) * G + g.
  int G;
  int block_size, max_blocks;
  int causal;
  int splits, keys_per_split;
  float scale_log2;           // sm_scale * log2(e)
};

typedef __attribute__((address_space(3))) void lds_void;
typedef const __attribute__((address_space(1))) void gbl_void;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Workgroup barrier that the compiler may not move memory accesses across; it
// emits no waitcnt of its own (the DMA pipeline manages vmcnt explicitly).
__device__ __forceinline__ void raw_barrier() {
  __asm__ __volatile__("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  __asm__ __volatile__("" ::: "memory");
}

// s_waitcnt with only vmcnt constrained (expcnt, lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Wait until at most `ahead` tiles (of L loads each) issued after the current one are pending.
template <int L>
__device__ __forceinline__ void wait_tiles(int ahead) {
  switch (ahead) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<L>(); break;
    case 2: wait_vmcnt<(2 * L < 64 ? 2 * L : 0)>(); break;
    default: wait_vmcnt<(3 * L < 64 ? 3 * L : 0)>(); break;
  }
}

template <int kNW, int kD>
struct MlaCfg {
  static constexpr int kThreads = kNW * kWave;
  static constexpr int kTileInstr = MlaGeom<kD>::kTileInstr;
  // DMA instructions per tile for wave w: I = w, w + kNW, ... < kTileInstr.
  static constexpr int kMaxPerWave = (kTileInstr + kNW - 1) / kNW;
  static_assert(kTileInstr % kNW == 0, "every wave issues the same number of DMA loads per tile");
  // Tiles issued ahead of the one being multiplied by P V.  Iteration t needs
  // tile t+1 resident (for its Q K^T) and keeps tiles t+2 .. t+kDepth-1 in
  // flight, so kDepth >= 2; kDepth - 1 tiles of loads must fit the 6-bit vmcnt
  // and the ring must hold tiles t .. t+kDepth.
  static constexpr int kDepth = (1 + 63 / kMaxPerWave) < kAhead ? (1 + 63 / kMaxPerWave) : kAhead;
  static_assert(kDepth >= 2 && kDepth + 1 <= kStages, "DMA ring depth");
};

// Tile layout in a stage.  The tile is 32 slots x 72 (64) 16-byte chunks, stored
// as 36 (32) blocks of 1 KB: block a + 4b holds slots 8a .. 8a+7 x chunks
// 8b .. 8b+7, with (slot 8a+u, chunk 8b+w) at 16-byte position
// 8u + (w ^ lds_swizzle(u, a)) of the block.  One DMA instruction fills one
// block, so its 64 lanes fetch 8 whole 128-byte lines (8 lanes per slot) --
// a gather of full cache lines.  The swizzle is set by the LDS of gfx950:
// 128 banks of 4 bytes, a ds_read_b128 served per 32-lane half-wave, which
// is conflict-free when its 32 16-byte chunks fall on distinct positions
// modulo 512 bytes.  A Q K^T operand read (half-wave: slots r = 0..15 of row
// groups a, a+1, chunks 4 par + g for two g) lands on position
// 8 (u & 3) + (w ^ lds_swizzle(u, a)) mod 32, so the swizzle maps
// (u >> 2, a & 1) one-to-one onto bits 2 and 1, leaving bit 0 to g: all 32
// distinct.  The transposed V reads (8 bytes a lane, one half of each chunk
// per instruction) keep the 2-way sharing that such reads have in any
// layout; the DMA writes are contiguous.
__host__ __device__ constexpr int lds_swizzle(int u, int a) {
  return ((u & 2) ? 4 : 0) ^ ((u & 4) ? 4 : 0) ^ ((a & 1) ? 2 : 0);
}

// The DMA of tile `tile` (slots tile*32 .. +31 of this workgroup) into a
// stage.  Wave w fills the row groups a = w, w + kNW, ...; lane 8u + v loads
// chunk 8b + (v ^ lds_swizzle(u, a)) of slot 8a + u, so its row address is
// fixed per row group and only the chunk-group offset 128*b changes between
// instructions.  Empty / masked slots re-load `safe_row` (a valid row of this
// workgroup; its probability is forced to 0), so every load stays inside the
// KV cache.
// The same DMA, split so that its instructions can be spread over the
// matrix work of an iteration: prepare() computes the lane's row addresses
// (reading the slot -> row map from LDS; a row tagged kSrc2Bit is read from
// the second source), issue<D>() sends instruction D.
// Sent in one burst, the instructions of the four waves queue behind each
// other in the memory pipeline and stall the issuing waves.
template <int kNW, int kD>
struct TileDma {
  static constexpr int kRowChunks = MlaGeom<kD>::kRowChunks;
  static constexpr int kGroups = 4 / kNW;                    // row groups per wave
  static constexpr int kCount = kGroups * (kRowChunks / 8);  // instructions per wave and tile
  const uint8_t* src[kGroups];
  uint8_t* stage;
  int wave;

  __device__ __forceinline__ void prepare(const uint8_t* kv, const uint8_t* kv2, const int32_t* rows, int safe_row,
                                          int tile, uint8_t* stage_base, int wave_, int lane) {
    wave = wave_;
    stage = stage_base;
    const int u = lane >> 3;
#pragma unroll
    for (int ag = 0; ag < kGroups; ++ag) {
      const int a = wave + ag * kNW;
      int row = rows[tile * kMlaTile + 8 * a + u];
      row = row >= 0 ? row : safe_row;
      const uint8_t* base = kv;
      if constexpr (MlaGeom<kD>::kRowLists) {
        base = (row & kSrc2Bit) ? kv2 : kv;
        row &= ~kSrc2Bit;
      }
      src[ag] = base + (int64_t)row * MlaGeom<kD>::kRowBytes + 16 * ((lane & 7) ^ lds_swizzle(u, a));
    }
  }
  template <int D>
  __device__ __forceinline__ void issue() {
    static_assert(D >= 0 && D < kCount, "DMA instruction index");
    constexpr int kAg = D / (kRowChunks / 8), kB = D % (kRowChunks / 8);
    const int a = wave + kAg * kNW;
    __builtin_amdgcn_global_load_lds((gbl_void*)(src[kAg] + 128 * kB), (lds_void*)(stage + (a + 4 * kB) * 1024), 16,
                                     0, 0);
  }
};

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

// ds_read_b64_tr_b16 as inline asm: through the builtin the compiler waits for
// every outstanding DMA before each read.  Completion is tracked explicitly
// with lgkm_wait below.
template <int kOff>
__device__ __forceinline__ void tr_read(u32x2& out, uint32_t lds_addr) {
  __asm__ __volatile__("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(out) : "v"(lds_addr), "i"(kOff));
}

// Wait until at most N LDS operations are outstanding; the four values pass
// through the asm so no use of them can be scheduled before the wait.
template <int N>
__device__ __forceinline__ void lgkm_wait(u32x2 (&v)[4]) {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  __asm__ __volatile__("s_waitcnt lgkmcnt(%4)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]) : "i"(N));
}

// The two transposed reads of V block kCb (keys 4g..4g+3 and 16+4g..16+4g+3):
// block 2p + h holds columns 32p + 8m' + 4h + i for MFMA row 4m' + i, read at
// bytes vbase[p % 2] + 4096*(p / 2) + 8h (+2048).
template <int kCb>
__device__ __forceinline__ void pv_block_reads(u32x2& lo, u32x2& hi, const uint32_t (&vbase)[2]) {
  constexpr int kP = kCb / 2, kH = kCb % 2;
  tr_read<4096 * (kP / 2) + 8 * kH>(lo, vbase[kP % 2]);
  tr_read<4096 * (kP / 2) + 8 * kH + 2048>(hi, vbase[kP % 2]);
}

// The four transposed reads of one pair of V blocks 2*kGrp, 2*kGrp + 1:
// v[2j], v[2j+1] = keys 4g..4g+3 and 16+4g..16+4g+3 of block 2*kGrp + j.
template <int kGrp>
__device__ __forceinline__ void pv_group_reads(u32x2 (&v)[4], const uint32_t (&vbase)[2]) {
  pv_block_reads<2 * kGrp>(v[0], v[1], vbase);
  pv_block_reads<2 * kGrp + 1>(v[2], v[3], vbase);
}

// O^T += V^T P^T: V^T is the A operand, P the B operand, so lane (g, r) of
// block 2p + h accumulates head r, columns 32p + 8g + 4h .. +3.
template <bool kF16, int kGrp>
__device__ __forceinline__ void pv_group_mfma(f32x4 (&o)[2][kMlaDV / 16], const u32x4 (&pa)[2], const u32x2 (&v)[4]) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const u32x4 vb = {v[2 * j].x, v[2 * j].y, v[2 * j + 1].x, v[2 * j + 1].y};
    o[0][2 * kGrp + j] = mfma16<kF16>(vb, pa[0], o[0][2 * kGrp + j]);
    o[1][2 * kGrp + j] = mfma16<kF16>(vb, pa[1], o[1][2 * kGrp + j]);
  }
}

// O += P V over one tile: 16 pairs of 16-column blocks, the reads of pairs
// k+1 and k+2 in flight while pair k runs on the matrix cores.
template <bool kF16, int kGrp>
__device__ __forceinline__ void pv_pipeline(f32x4 (&o)[2][kMlaDV / 16], const u32x4 (&pa)[2],
                                            const uint32_t (&vaddr)[2], u32x2 (&cur)[4], u32x2 (&nxt)[4]) {
  constexpr int kGroups = kMlaDV / 32;
  if constexpr (kGrp + 2 < kGroups) {
    u32x2 n2[4];
    pv_group_reads<kGrp + 2>(n2, vaddr);
    lgkm_wait<8>(cur);
    pv_group_mfma<kF16, kGrp>(o, pa, cur);
    pv_pipeline<kF16, kGrp + 1>(o, pa, vaddr, nxt, n2);
  } else if constexpr (kGrp + 1 < kGroups) {
    lgkm_wait<4>(cur);
    pv_group_mfma<kF16, kGrp>(o, pa, cur);
    lgkm_wait<0>(nxt);
    pv_group_mfma<kF16, kGrp + 1>(o, pa, nxt);
  }
}

template <int kOff>
__device__ __forceinline__ void b128_read(u32x4& out, uint32_t lds_addr) {
  __asm__ __volatile__("ds_read_b128 %0, %1 offset:%2" : "=v"(out) : "v"(lds_addr), "i"(kOff));
}

template <int N>
__device__ __forceinline__ void lgkm_wait_k(u32x4& k) {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  __asm__ __volatile__("s_waitcnt lgkmcnt(%1)" : "+v"(k) : "i"(N));
}

template <int kNW, int kD, int D = 0>
__device__ __forceinline__ void il_dma_all(TileDma<kNW, kD>& dma) {
  if constexpr (D < TileDma<kNW, kD>::kCount) {
    dma.template issue<D>();
    il_dma_all<kNW, kD, D + 1>(dma);
  }
}

// DMA instructions D with D * kQkHalf / kCount == J go out at half-step J.
template <int kNW, int kD, int J, int D = 0>
__device__ __forceinline__ void il_dma(TileDma<kNW, kD>& dma) {
  if constexpr (D < TileDma<kNW, kD>::kCount) {
    if constexpr (D * MlaGeom<kD>::kQkHalf / TileDma<kNW, kD>::kCount == J) dma.template issue<D>();
    il_dma<kNW, kD, J, D + 1>(dma);
  }
}

// P V alone (the last tile).
template <bool kF16>
__device__ __forceinline__ void pv_only(f32x4 (&o)[2][kMlaDV / 16], const u32x4 (&pa)[2], const uint32_t (&va)[2]) {
  u32x2 vg0[4], vg1[4];
  pv_group_reads<0>(vg0, va);
  pv_group_reads<1>(vg1, va);
  pv_pipeline<kF16, 0>(o, pa, va, vg0, vg1);
}

// ---------------------------------------------------------------------------
// Phase A of an iteration: S^T(t+1) = K(t+1) Q^T in half-steps.  Half-step J
// reads one K operand (key half J % 2 of 32-dim step J / 2, one
// ds_read_b128) and runs its 2 MFMAs (both head blocks).  Even and odd dim
// steps accumulate into separate sets, so eight independent MFMA chains are in
// flight, and kQkAhead reads stay outstanding.  The DMA of a future tile is
// spread over the half-steps.
constexpr int kQkAhead = 6;

// One Q K^T MFMA with its accumulator in VGPRs, as inline asm.  The compiler
// writes every MFMA result of this kernel to AGPRs, where the O accumulators
// already take all 256: it then parked O columns in VGPRs around each tile's
// Q K^T (about 100 v_accvgpr moves a tile).  The accumulator chains are eight
// MFMAs apart (no back-to-back dependence); qk_phase waits out the last
// results before any VALU instruction reads them.  kZero: start the chain (C = 0).
template <bool kF16, bool kZero>
__device__ __forceinline__ void mfma_qk(f32x4& c, const u32x4& a, const u32x4& b) {
  if constexpr (kZero) {
    if constexpr (kF16) __asm__ __volatile__("v_mfma_f32_16x16x32_f16 %0, %1, %2, 0" : "=v"(c) : "v"(a), "v"(b));
    else __asm__ __volatile__("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=v"(c) : "v"(a), "v"(b));
  } else {
    if constexpr (kF16) __asm__ __volatile__("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
    else __asm__ __volatile__("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
  }
}

template <bool kF16, int kNW, int kD, bool kDma, int J>
__device__ __forceinline__ void qk_half(f32x4 (&c)[2][2][2], const u32x4 (&qb)[2][kD / 32],
                                        const uint32_t (&qa)[2], u32x4 (&k)[kQkAhead + 1], TileDma<kNW, kD>& dma) {
  constexpr int kQkHalf = MlaGeom<kD>::kQkHalf;
  constexpr int kNext = J + kQkAhead;
  if constexpr (kNext < kQkHalf) {
    b128_read<4096 * (kNext / 4) + 2048 * (kNext % 2)>(k[kNext % (kQkAhead + 1)], qa[(kNext / 2) % 2]);
  }
  if constexpr (kDma) il_dma<kNW, kD, J>(dma);
  constexpr int kWait = (kQkHalf - 1 - J) < kQkAhead ? (kQkHalf - 1 - J) : kQkAhead;
  constexpr int kSlot = J % (kQkAhead + 1);
  lgkm_wait_k<kWait>(k[kSlot]);
  constexpr int kSet = (J / 2) % 2, kKb = J % 2, kSt = J / 2;
  // Half-steps 0..3 start the four chains of each head block.
  mfma_qk<kF16, (J < 4)>(c[kSet][0][kKb], k[kSlot], qb[0][kSt]);
  mfma_qk<kF16, (J < 4)>(c[kSet][1][kKb], k[kSlot], qb[1][kSt]);
  if constexpr (J + 1 < kQkHalf) qk_half<kF16, kNW, kD, kDma, J + 1>(c, qb, qa, k, dma);
}

template <int J>
__device__ __forceinline__ void qk_prologue(u32x4 (&k)[kQkAhead + 1], const uint32_t (&qa)[2]) {
  if constexpr (J < kQkAhead) {
    b128_read<4096 * (J / 4) + 2048 * (J % 2)>(k[J], qa[(J / 2) % 2]);
    qk_prologue<J + 1>(k, qa);
  }
}

template <bool kF16, int kNW, int kD, bool kDma>
__device__ __forceinline__ void qk_phase(f32x4 (&s)[2][2], const u32x4 (&qb)[2][kD / 32],
                                         const uint32_t (&qa)[2], TileDma<kNW, kD>& dma) {
  f32x4 c[2][2][2];
  u32x4 k[kQkAhead + 1];
  qk_prologue<0>(k, qa);
  qk_half<kF16, kNW, kD, kDma, 0>(c, qb, qa, k, dma);
  static_assert(kQkAhead + 1 == 7, "the wait below names every K operand register");
  // The asm MFMAs are opaque to the compiler's hazard checks: 24 wait states
  // (a 16-pass MFMA needs 19) before a VALU instruction reads a result, and
  // before the K operand registers may be reused.
  __asm__ __volatile__("s_nop 7\n\ts_nop 7\n\ts_nop 7"
                       : "+v"(c[0][0][0]), "+v"(c[0][0][1]), "+v"(c[0][1][0]), "+v"(c[0][1][1]), "+v"(c[1][0][0]),
                         "+v"(c[1][0][1]), "+v"(c[1][1][0]), "+v"(c[1][1][1]), "+v"(k[0]), "+v"(k[1]), "+v"(k[2]),
                         "+v"(k[3]), "+v"(k[4]), "+v"(k[5]), "+v"(k[6]));
#pragma unroll
  for (int hb = 0; hb < 2; ++hb)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) s[hb][kb] = c[0][hb][kb] + c[1][hb][kb];
}

// Phase B: O += P(t) V(t) while the softmax of tile t+1 turns its scores into
// P(t+1).  The softmax is cut into slices run between the MFMA groups of the
// P V pipeline, so its VALU work overlaps the matrix cores.  Lane (g, r)
// holds scores of keys 4g+i (kb 0) and 16+4g+i (kb 1) of heads head0 + 16*hb
// + r; scores of empty slots were set to -inf beforehand.
// kRoundSum: also sum the probabilities as rounded to 16 bits (lsum_r), so O
// can be normalised by the weights the P V products actually used: with a
// fixed reference the dominant key's P is rounded too (a running max would
// make it exactly 1), and dividing by the rounded sum cancels that error.
template <bool kF16, bool kRoundSum = false>
struct SoftmaxSlices {
  static constexpr int kSlices = 10;  // per head block: 4 x (2 exponentials), 1 x (sum, pack)
  const f32x4 (&c)[2][2];
  u32x4 (&pa)[2];
  float (&lsum)[2];
  float (&lsum_r)[2];
  bool& overflow;
  float neg_m[2];
  float scale;
  float p[2][8];

  template <int kS>
  __device__ __forceinline__ void run() {
    if constexpr (kS < kSlices) {
      constexpr int kHb = kS / 5, kPart = kS % 5;
      if constexpr (kPart < 4) {
#pragma unroll
        for (int e = 2 * kPart; e < 2 * kPart + 2; ++e) {
          p[kHb][e] = fast_exp2(fmaf(c[kHb][e / 4][e % 4], scale, neg_m[kHb]));
        }
      } else {
        const float* q = p[kHb];
        const float ps = ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
        lsum[kHb] += ps;
        overflow = overflow || !(ps <= kOverflowSumOf<kF16>);
        pa[kHb] = u32x4{pack2<kF16>(q[0], q[1]), pack2<kF16>(q[2], q[3]), pack2<kF16>(q[4], q[5]),
                        pack2<kF16>(q[6], q[7])};
        if constexpr (kRoundSum) {
          const u32x4 w = pa[kHb];
          lsum_r[kHb] += ((unpack_lo<kF16>(w.x) + unpack_hi<kF16>(w.x)) + (unpack_lo<kF16>(w.y) + unpack_hi<kF16>(w.y))) +
                         ((unpack_lo<kF16>(w.z) + unpack_hi<kF16>(w.z)) + (unpack_lo<kF16>(w.w) + unpack_hi<kF16>(w.w)));
        }
      }
    }
  }
};

template <bool kF16, int kGrp, bool kRoundSum>
__device__ __forceinline__ void pv_softmax_pipeline(f32x4 (&o)[2][kMlaDV / 16], const u32x4 (&pa)[2],
                                                    const uint32_t (&vaddr)[2], u32x2 (&cur)[4], u32x2 (&nxt)[4],
                                                    SoftmaxSlices<kF16, kRoundSum>& sm) {
  constexpr int kGroups = kMlaDV / 32;
  if constexpr (kGrp + 2 < kGroups) {
    u32x2 n2[4];
    pv_group_reads<kGrp + 2>(n2, vaddr);
    sm.template run<kGrp>();
    lgkm_wait<8>(cur);
    pv_group_mfma<kF16, kGrp>(o, pa, cur);
    pv_softmax_pipeline<kF16, kGrp + 1, kRoundSum>(o, pa, vaddr, nxt, n2, sm);
  } else if constexpr (kGrp + 1 < kGroups) {
    sm.template run<kGrp>();
    lgkm_wait<4>(cur);
    pv_group_mfma<kF16, kGrp>(o, pa, cur);
    sm.template run<kGrp + 1>();
    lgkm_wait<0>(nxt);
    pv_group_mfma<kF16, kGrp + 1>(o, pa, nxt);
  }
}
static_assert(SoftmaxSlices<false>::kSlices <= kMlaDV / 32, "every softmax slice has a P V group");

__device__ __forceinline__ uint32_t lds_u32(const void* p) {
  return (uint32_t)(uintptr_t)(const lds_void*)p;
}

// Exact two-pass fallback for a workgroup whose scores outgrew the fast
// path's fixed reference: per head, the scores of all slots go to LDS, then
// max, sum and P V from them.  Slow (VALU, KV re-read per head) and only taken
// for pathological score ranges.  Writes the same outputs as the fast path
// (with the attention sink of each head when `sinks` is given, in base-2
// units).  Arguments are passed by value (a reference to the kernel's
// argument block would force that block into scratch memory for the whole
// kernel).
template <bool kF16, int kD>
__device__ __forceinline__ const uint16_t* mla_row(const uint8_t* kvb, const uint8_t* kvb2, int row) {
  const uint8_t* base = kvb;
  if constexpr (MlaGeom<kD>::kRowLists) {
    base = (row & kSrc2Bit) ? kvb2 : kvb;
    row &= ~kSrc2Bit;
  }
  return reinterpret_cast<const uint16_t*>(base + (int64_t)row * MlaGeom<kD>::kRowBytes);
}

template <bool kF16, int kD>
__device__ __attribute__((noinline)) void mla_exact_fallback(const uint16_t* q, const uint8_t* kvb, const uint8_t* kvb2,
                                                             const float* sinks, uint16_t* obase, float* obase32,
                                                             float* lbase, int H,
                                                             float scale_log2, const int32_t* rows, int nslots,
                                                             int token, int head_begin, int nheads, float* sc,
                                                             int threads) {
  const int tid = threadIdx.x;
  float* red = sc + kSlotsCap;  // per-wave partials
  for (int hl = 0; hl < nheads; ++hl) {
    const int h = head_begin + hl;
    if (h >= H) break;
    const uint16_t* qh = q + ((int64_t)token * H + h) * kD;
    float mx = -__builtin_huge_valf();
    for (int j = tid; j < nslots; j += threads) {
      const int row = rows[j];
      float sj = -__builtin_huge_valf();
      if (row >= 0) {
        const uint16_t* kr = mla_row<kF16, kD>(kvb, kvb2, row);
        float acc = 0.f;
        for (int d = 0; d < kD; d += 2) {
          const uint32_t qv = *reinterpret_cast<const uint32_t*>(qh + d);
          const uint32_t kv = *reinterpret_cast<const uint32_t*>(kr + d);
          acc = fmaf(unpack_lo<kF16>(qv), unpack_lo<kF16>(kv), acc);
          acc = fmaf(unpack_hi<kF16>(qv), unpack_hi<kF16>(kv), acc);
        }
        sj = acc * scale_log2;
      }
      sc[j] = sj;
      mx = fmaxf(mx, sj);
    }
    mx = wave_max(mx);
    if ((tid & (kWave - 1)) == 0) red[tid / kWave] = mx;
    __syncthreads();
    mx = -__builtin_huge_valf();
    for (int w = 0; w < threads / kWave; ++w) mx = fmaxf(mx, red[w]);
    __syncthreads();
    const float sink = sinks ? sinks[h] * 1.4426950408889634f : -__builtin_huge_valf();
    mx = fmaxf(mx, sink);
    const float m_use = mx == -__builtin_huge_valf() ? 0.f : mx;
    float l = 0.f;
    for (int j = tid; j < nslots; j += threads) l += fast_exp2(sc[j] - m_use);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o, kWave);
    if ((tid & (kWave - 1)) == 0) red[tid / kWave] = l;
    __syncthreads();
    l = sinks ? fast_exp2(sink - m_use) : 0.f;
    for (int w = 0; w < threads / kWave; ++w) l += red[w];
    const float inv = l > 0.f ? 1.f / l : 0.f;
    for (int c = tid; c < kMlaDV; c += threads) {
      float acc = 0.f;
      for (int j = 0; j < nslots; ++j) {
        const int row = rows[j];
        if (row < 0) continue;
        const uint16_t v = mla_row<kF16, kD>(kvb, kvb2, row)[c];
        acc = fmaf(fast_exp2(sc[j] - m_use), unpack_lo<kF16>(v), acc);
      }
      if (obase32) obase32[((int64_t)token * H + h) * kMlaDV + c] = acc * inv;
      else obase[((int64_t)token * H + h) * kMlaDV + c] = cvt1<kF16>(acc * inv);
    }
    if (tid == 0) lbase[(int64_t)token * H + h] = l > 0.f ? (mx + fast_log2(l)) * 0.69314718055994531f : -__builtin_huge_valf();
    __syncthreads();
  }
}

// kPaged: the KV rows are addressed through a block table (a.block_table).
// kSt: ring stages.  4 (sparse_mla_kernel): the pipelined loop below.  2
// (sparse_mla_rows2_kernel: the 512-wide row lists with one or two waves, i.e. up
// to 64 heads): each tile is computed in turn -- Q K^T, softmax, P V -- while the
// next tile's DMA fills the other stage; the 73 KB of LDS let two workgroups
// share a CU, so all four SIMDs work and each workgroup's exposed DMA latency,
// prologue and epilogue overlap the other's.
template <int kNW, bool kF16, int kD, bool kPaged, int kSt>
__device__ __forceinline__ void sparse_mla_body(MlaArgs a) {
  static_assert(kSt == kStages || kSt == 2, "ring stages");
  using Cfg = MlaCfg<kNW, kD>;
  using Geo = MlaGeom<kD>;
  using Lay = MlaLayout<kD, kSt>;
  extern __shared__ __align__(16) uint8_t lds[];
  int32_t* rows = reinterpret_cast<int32_t*>(lds + Lay::kRowsOffset);
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // wave-uniform
  const int r = lane & 15;
  const int g = lane >> 4;

  const int T = a.B * a.S * a.G;
  const int token = blockIdx.x % T;
  const int split = blockIdx.x / T;
  const int bs_row = token / a.G;  // b * S + s
  const int kvg = token - bs_row * a.G;
  const int b = bs_row / a.S;
  const int s = bs_row % a.S;
  // A wave owns two 16-head blocks: heads head0 + 16*hb + r.
  const int head0 = blockIdx.y * (kNW * kHeadsPerWave) + wave * kHeadsPerWave;
  bool hb_on[2];
  hb_on[0] = head0 < a.H;
  hb_on[1] = head0 + 16 < a.H;

  // The prologue is a chain of global-memory latencies; it is ordered so
  // they overlap: the lengths and this lane's slot indices go out first, then
  // the Q rows (the largest load; a compiler barrier keeps that order) -- for
  // a paged cache only after the block-table lookups, which need the indices
  // -- so that the slot table and the first tiles' DMA are issued while Q is
  // still arriving: nothing waits for Q before the first tile (vector-memory
  // loads complete in issue order, so the first tile's wait covers Q).
  const int32_t* irow = a.indices + (int64_t)token * a.topk;
  const int slot_begin = split * a.keys_per_split;
  // Row lists: a negative count marks a padded query row (out = 0, lse = 0).
  const int count_raw = Geo::kRowLists ? a.slot_count[token] : 0;
  const int row_slots = Geo::kRowLists ? min(max(count_raw, 0), a.topk) : a.topk;
  const int slot_end = min(row_slots, slot_begin + a.keys_per_split);
  const int nslots = slot_end > slot_begin ? slot_end - slot_begin : 0;
  // Every load below is issued unconditionally, from a clamped valid address
  // (its value is discarded later if out of range): conditional loads would
  // make the compiler wait for them on the spot.
  constexpr int kIdxPerLane = kSlotsCap / (kNW * kWave);  // slot indices a lane may translate
  const int last_slot = max(min(slot_end, a.topk) - 1, 0);  // clamped: slot_end may be 0
  int idx_raw[kIdxPerLane];
#pragma unroll
  for (int j = 0; j < kIdxPerLane; ++j) {
    const int i = wave * kWave + j * Cfg::kThreads + lane;
    idx_raw[j] = irow[min(slot_begin + i, last_slot)];
  }
  // Per-sequence lengths through the scalar cache (wave-uniform).
  typedef const __attribute__((address_space(4))) int32_t const_i32;
  const int ql_raw = a.q_len ? *(const_i32*)(a.q_len + b) : a.S;
  const int kl_raw = a.kv_len ? *(const_i32*)(a.kv_len + b) : a.Skv;
  __asm__ __volatile__("" ::: "memory");

  // Q operands (B of S^T = K Q^T): head head0 + 16*hb + r, dims 32*st + 8*g .. +8.
  // Heads past H (a wave's second head block when H is not a multiple of 32)
  // repeat head H - 1; their results are not stored.
  u32x4 qb[2][kD / 32];
  auto load_q = [&]() {
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      const int h = min(head0 + 16 * hb + r, a.H - 1);
      const uint16_t* qp = a.q + ((int64_t)token * a.H + h) * kD + 8 * g;
#pragma unroll
      for (int st = 0; st < kD / 32; ++st) qb[hb][st] = *reinterpret_cast<const u32x4*>(qp + 32 * st);
    }
  };
  if constexpr (!kPaged) load_q();
  const int ql = min(max(ql_raw, 0), a.S);
  const int kl = Geo::kRowLists ? 0x7fffffff : min(max(kl_raw, 0), a.Skv);
  const bool row_active = Geo::kRowLists ? count_raw >= 0 : s < ql;
  const int lim = a.causal ? (kl - ql + s) : 0x7fffffff;
  int ntiles = row_active ? (nslots + kMlaTile - 1) / kMlaTile : 0;

  // Slots -> physical rows (-1: empty or masked); the lowest valid slot's row
  // doubles as the DMA source of the empty ones.
  int row_of[kIdxPerLane];
  bool ok[kIdxPerLane];
#pragma unroll
  for (int j = 0; j < kIdxPerLane; ++j) {
    const int i = wave * kWave + j * Cfg::kThreads + lane;
    const int idx = idx_raw[j];
    ok[j] = i < nslots && idx >= 0 && idx < kl && idx <= lim;
  }
  if constexpr (Geo::kRowLists) {
#pragma unroll
    for (int j = 0; j < kIdxPerLane; ++j) row_of[j] = ok[j] ? idx_raw[j] : -1;
  } else if constexpr (kPaged) {
    // All lookups first (from a clamped valid entry), then Q, then the translation.
    int blk[kIdxPerLane];
    const int32_t* bt = a.block_table + (int64_t)b * a.max_blocks;
#pragma unroll
    for (int j = 0; j < kIdxPerLane; ++j) blk[j] = bt[ok[j] ? idx_raw[j] / a.block_size : 0];
    __asm__ __volatile__("" ::: "memory");
    load_q();
#pragma unroll
    for (int j = 0; j < kIdxPerLane; ++j)
      row_of[j] = ok[j] ? (blk[j] * a.block_size + idx_raw[j] % a.block_size) * a.G + kvg : -1;
  } else {
#pragma unroll
    for (int j = 0; j < kIdxPerLane; ++j) row_of[j] = ok[j] ? (b * a.Skv + idx_raw[j]) * a.G + kvg : -1;
  }
#pragma unroll
  for (int j = 0; j < kIdxPerLane; ++j) __asm__ __volatile__("" : "+v"(row_of[j]));
  int32_t* first_valid = rows + kSlotsCap + 1;
  int32_t* last_valid = rows + kSlotsCap + 2;
  if (tid == 0) {
    *first_valid = 0x7fffffff;
    *last_valid = -1;
  }
  __syncthreads();
  // Each wave wrote 64 consecutive slots per pass; record, per tile of 32,
  // the bitmask of its valid slots.
  uint32_t* tile_mask = reinterpret_cast<uint32_t*>(lds + Lay::kTileMaskOffset);
  int wave_first = 0x7fffffff;  // lowest valid slot this wave saw (wave-uniform)
  int wave_last = -1;           // highest
#pragma unroll
  for (int j = 0; j < kIdxPerLane; ++j) {
    const int i0 = wave * kWave + j * Cfg::kThreads;
    const int i = i0 + lane;
    const int row = row_active ? row_of[j] : -1;
    if (i < ntiles * kMlaTile) rows[i] = row;
    const uint64_t vm = __ballot(row >= 0 && i < ntiles * kMlaTile);
    if (vm != 0) {
      wave_first = min(wave_first, i0 + (int)__builtin_ctzll(vm));
      wave_last = max(wave_last, i0 + 63 - (int)__builtin_clzll(vm));
    }
    if (lane == 0 && i0 < ntiles * kMlaTile) {
      tile_mask[i0 / kMlaTile] = (uint32_t)vm;
      if (i0 / kMlaTile + 1 < ntiles) tile_mask[i0 / kMlaTile + 1] = (uint32_t)(vm >> 32);
    }
  }
  // One LDS atomic per wave (one per valid slot would serialise hundreds).
  if (lane == 0 && wave_first != 0x7fffffff) {
    atomicMin(first_valid, wave_first);
    atomicMax(last_valid, wave_last);
  }
  __syncthreads();
  const int fv = *first_valid;
  const int safe_row = fv < kSlotsCap ? rows[fv] : -1;
  const int nslots_all = ntiles * kMlaTile;  // the exact fallback walks every slot
  if (safe_row < 0) ntiles = 0;              // no valid slot: out = 0, lse = -inf
  // Tiles before the first valid slot contribute nothing: start at its tile,
  // which then also fixes the softmax reference.  Tiles after the last valid
  // slot contribute nothing either (a causal row shorter than topk ends in
  // empty slots): stop at its tile.
  const int t_first = safe_row < 0 ? 0 : fv / kMlaTile;
  if (safe_row >= 0) ntiles = min(ntiles, *last_valid / kMlaTile + 1);
  ntiles -= t_first;
  const int32_t* trows = rows + t_first * kMlaTile;
  const uint32_t* tmask = tile_mask + t_first;

  const uint8_t* kvb = reinterpret_cast<const uint8_t*>(a.kv);
  const uint8_t* kvb2 = reinterpret_cast<const uint8_t*>(a.kv2);
  constexpr int kStageBytes = Geo::kStageBytes;
  constexpr int kDepth = Cfg::kDepth;
  constexpr int kL = Cfg::kMaxPerWave;

  f32x4 o[2][kMlaDV / 16];
#pragma unroll
  for (int hb = 0; hb < 2; ++hb)
#pragma unroll
    for (int i = 0; i < kMlaDV / 16; ++i) o[hb][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_ref[2] = {-__builtin_huge_valf(), -__builtin_huge_valf()};  // reference max (base 2)
  float lsum[2] = {0.f, 0.f};  // this lane's share of sum exp2(t - m_ref)
  float lsum_r[2] = {0.f, 0.f};  // the same sum of P as rounded for P V (row lists only)
  using Softmax = SoftmaxSlices<kF16, Geo::kRowLists>;
  int32_t* overflow_flag = rows + kSlotsCap;
  bool overflow = false;

  // Per-lane LDS byte offsets in a stage (layout: see lds_swizzle).
  // QK A operand of step st: chunk 4*st + g of slots r (+16): slot r is row
  // u = r & 7 of row group r >> 3, chunk 4*st + g is chunk 4*(st & 1) + g of
  // chunk group st / 2 -> qk_lane[st & 1] + 4096*(st / 2) (+2048).
  uint32_t qk_lane[2];
#pragma unroll
  for (int par = 0; par < 2; ++par)
    qk_lane[par] = 1024 * (r >> 3) + 128 * (r & 7) + 16 * ((4 * par + g) ^ lds_swizzle(r & 7, r >> 3));
  // V^T operand of block 2p + h through transposed reads: lane (g, r)
  // addresses slot 4g + (r >> 2) (+16), columns 32p + 8*(r & 3) + 4h .. +3,
  // i.e. chunk 4p + (r & 3), byte 8h: row u = 4*(g & 1) + (r >> 2) of row
  // group g >> 1, chunk 4*(p & 1) + (r & 3) of chunk group p / 2
  // -> pv_lane[p & 1] + 4096*(p / 2) + 8h (+2048).
  uint32_t pv_lane[2];
  {
    const int u = 4 * (g & 1) + (r >> 2);
#pragma unroll
    for (int par = 0; par < 2; ++par)
      pv_lane[par] = 1024 * (g >> 1) + 128 * u + 16 * ((4 * par + (r & 3)) ^ lds_swizzle(u, g >> 1));
  }
  auto stage_k = [&](int tile, uint32_t (&out)[2]) {
    const uint32_t base = lds_u32(lds + (tile % kSt) * kStageBytes);
    out[0] = base + qk_lane[0];
    out[1] = base + qk_lane[1];
  };
  auto stage_v = [&](int tile, uint32_t (&out)[2]) {
    const uint32_t base = lds_u32(lds + (tile % kSt) * kStageBytes);
    out[0] = base + pv_lane[0];
    out[1] = base + pv_lane[1];
  };

  // Softmax of one tile's scores (S^T: lane (g, r) holds keys 4g+i and
  // 16+4g+i of heads head0 + 16*hb + r) into the P operands of O += P V.
  // The reference max m_ref is fixed by the first tile with a valid slot
  // (the same tile for every head: validity is per slot), biased up by
  // 2^kRefBias so later scores may exceed it by 2^(kRefBias + kOverflowGuard)
  // without a rescale of O (scaling by a power of two is exact; for bf16,
  // contributions more than 2^66 below the first tile's max underflow,
  // negligibly).  After that tile no cross-lane maximum is needed: a later
  // score beyond the headroom makes its probability -- hence the lane's sum of
  // this tile's probabilities -- exceed 2^kOverflowGuard, which flags the
  // workgroup for the exact fallback after the loop.
  // (A reference to the kernel argument block would put it in scratch memory:
  // the lambda captures locals only.)
  const float scale_log2 = a.scale_log2;
  // Scores of empty slots -> -inf (a partly valid tile is rare: uniform branch).
  auto mask_scores = [&](f32x4 (&c)[2][2], uint32_t m) {
    if (m != 0xffffffffu) {
      const uint32_t lane_bits = ((m >> (4 * g)) & 15u) | (((m >> (16 + 4 * g)) & 15u) << 4);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const bool v = (lane_bits >> e) & 1u;
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) c[hb][e / 4][e % 4] = v ? c[hb][e / 4][e % 4] : -__builtin_huge_valf();
      }
    }
  };

  // Software pipeline over tiles.  Before iteration t, P(t) is known.  The
  // iteration computes S(t+1) = Q K(t+1)^T (phase A, with the DMA of tile
  // t + kDepth spread over it), then accumulates O += P(t) V(t) while the
  // softmax turns S(t+1) into P(t+1) (phase B).  One barrier per tile: it
  // publishes tile t+1 and certifies that every wave is done with tile t-1,
  // whose stage the DMA of tile t + kDepth then refills.
  if (kSt == 2 && ntiles > 0) {
    // Two stages: tile t in stage t & 1; the DMA of tile t + 1 goes out spread
    // over the Q K^T of tile t, into the stage tile t - 1 left.
    {
      TileDma<kNW, kD> dma;
      dma.prepare(kvb, kvb2, trows, safe_row, 0, lds, wave, lane);
      il_dma_all(dma);
    }
    u32x4 pa[2];
    for (int tile = 0; tile < ntiles; ++tile) {
      // Tile `tile` has arrived (vector-memory loads complete in order, so this
      // also covers Q); the barrier publishes it and certifies that every wave
      // is done with tile - 1.
      wait_vmcnt<0>();
      raw_barrier();
      const bool more = tile + 1 < ntiles;  // workgroup-uniform
      TileDma<kNW, kD> dma;
      if (more) dma.prepare(kvb, kvb2, trows, safe_row, tile + 1, lds + ((tile + 1) % kSt) * kStageBytes, wave, lane);
      f32x4 c[2][2];
      uint32_t qa[2], va[2];
      stage_k(tile, qa);
      stage_v(tile, va);
      if (more) qk_phase<kF16, kNW, kD, true>(c, qb, qa, dma);
      else qk_phase<kF16, kNW, kD, false>(c, qb, qa, dma);
      mask_scores(c, __builtin_amdgcn_readfirstlane(tmask[tile]));
      if (tile == 0) {
        // The first processed tile holds the first valid slot: it fixes m_ref.
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
          float cmax = -__builtin_huge_valf();
#pragma unroll
          for (int e = 0; e < 8; ++e) cmax = fmaxf(cmax, c[hb][e / 4][e % 4]);
          cmax = fmaxf(cmax, __shfl_xor(cmax, 16, kWave));
          cmax = fmaxf(cmax, __shfl_xor(cmax, 32, kWave));
          m_ref[hb] = cmax * scale_log2 + PRange<kF16>::kRefBias;
        }
      }
      Softmax sm{c, pa, lsum, lsum_r, overflow, {-m_ref[0], -m_ref[1]}, scale_log2, {}};
      sm.template run<0>();
      sm.template run<1>();
      sm.template run<2>();
      sm.template run<3>();
      sm.template run<4>();
      sm.template run<5>();
      sm.template run<6>();
      sm.template run<7>();
      sm.template run<8>();
      sm.template run<9>();
      pv_only<kF16>(o, pa, va);
    }
  }
  if (kSt == kStages && ntiles > 0) {
    // The first kDepth stages are filled now (a row of fewer tiles re-loads its
    // last tile into the stages it does not use), unconditionally, so that the
    // compiler sees a fixed count of loads behind Q: the wait for tile 0 then
    // also covers Q, and no wait for every load in flight is added before the
    // first MFMA.  Iteration t sends tile t + kDepth while it exists.
#pragma unroll
    for (int t = 0; t < kDepth; ++t) {
      TileDma<kNW, kD> dma;
      dma.prepare(kvb, kvb2, trows, safe_row, min(t, ntiles - 1), lds + (t % kStages) * kStageBytes, wave, lane);
      il_dma_all(dma);
    }
    u32x4 pa[2];
    {
      wait_vmcnt<(kDepth - 1) * kL>();
      raw_barrier();
      f32x4 c[2][2];
      uint32_t qa[2];
      stage_k(0, qa);
      TileDma<kNW, kD> none;
      qk_phase<kF16, kNW, kD, false>(c, qb, qa, none);
      mask_scores(c, __builtin_amdgcn_readfirstlane(tmask[0]));
      // The first processed tile holds the first valid slot: it fixes m_ref.
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
        float cmax = -__builtin_huge_valf();
#pragma unroll
        for (int e = 0; e < 8; ++e) cmax = fmaxf(cmax, c[hb][e / 4][e % 4]);
        cmax = fmaxf(cmax, __shfl_xor(cmax, 16, kWave));
        cmax = fmaxf(cmax, __shfl_xor(cmax, 32, kWave));
        // sm_scale > 0, so the max commutes with the scaling.
        m_ref[hb] = cmax * scale_log2 + PRange<kF16>::kRefBias;
      }
      Softmax sm{c, pa, lsum, lsum_r, overflow, {-m_ref[0], -m_ref[1]}, scale_log2, {}};
      sm.template run<0>();
      sm.template run<1>();
      sm.template run<2>();
      sm.template run<3>();
      sm.template run<4>();
      sm.template run<5>();
      sm.template run<6>();
      sm.template run<7>();
      sm.template run<8>();
      sm.template run<9>();
    }
    auto iteration = [&](auto dma_c, int tile) {
      constexpr bool kDma = decltype(dma_c)::value;
      // The DMA of tile + kDepth (into the stage tile - 1 left) goes out
      // spread over phase A.
      TileDma<kNW, kD> dma;
      if constexpr (kDma)
        dma.prepare(kvb, kvb2, trows, safe_row, tile + kDepth, lds + ((tile + kDepth) % kStages) * kStageBytes, wave,
                    lane);
      f32x4 c[2][2];
      uint32_t qa[2], va[2];
      stage_k(tile + 1, qa);
      stage_v(tile, va);
      qk_phase<kF16, kNW, kD, kDma>(c, qb, qa, dma);
      mask_scores(c, __builtin_amdgcn_readfirstlane(tmask[tile + 1]));
      u32x4 pa_next[2];
      Softmax sm{c, pa_next, lsum, lsum_r, overflow, {-m_ref[0], -m_ref[1]}, scale_log2, {}};
      u32x2 vg0[4], vg1[4];
      pv_group_reads<0>(vg0, va);
      pv_group_reads<1>(vg1, va);
      pv_softmax_pipeline<kF16, 0, Geo::kRowLists>(o, pa, va, vg0, vg1, sm);
      pa[0] = pa_next[0];
      pa[1] = pa_next[1];
    };
    // Steady state: tiles t+2 .. t+kDepth-1 stay in flight past tile t+1.
    int tile = 0;
    for (; tile + kDepth < ntiles; ++tile) {
      wait_tiles<kL>(kDepth - 2);
      raw_barrier();
      iteration(std::true_type{}, tile);
    }
    // The last kDepth - 1 iterations send nothing: fewer tiles remain behind t+1.
    for (; tile + 1 < ntiles; ++tile) {
      wait_tiles<kL>(ntiles - 2 - tile);
      raw_barrier();
      iteration(std::false_type{}, tile);
    }
    // The last tile is resident and published; no DMA targets its stage.
    uint32_t va[2];
    stage_v(ntiles - 1, va);
    pv_only<kF16>(o, pa, va);
  }
  // All LDS reads and DMAs retire before the ring is reused below.
  __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) expcnt(0) lgkmcnt(0)
  // Any wave whose scores outgrew the biased reference: recompute exactly.
  if (tid == 0) *overflow_flag = 0;
  __syncthreads();
  if (__any(overflow) && lane == 0) *overflow_flag = 1;
  __syncthreads();
  const bool final_out = (a.splits == 1);
  uint16_t* obase = final_out ? a.out : a.part_o + (int64_t)split * T * a.H * kMlaDV;
  float* obase32 = nullptr;  // fp32 output (row lists only)
  if constexpr (Geo::kRowLists) {
    if (a.out32) obase32 = final_out ? a.out32 : a.part_o32 + (int64_t)split * T * a.H * kMlaDV;
  }
  float* lbase = final_out ? a.lse : a.part_lse + (int64_t)split * T * a.H;
  // Sinks join the softmax once: here when this workgroup writes the final
  // output, in the combine kernel otherwise.
  const float* sinks = Geo::kRowLists && final_out ? a.sinks : nullptr;
  if (*overflow_flag) {
    mla_exact_fallback<kF16, kD>(a.q, kvb, kvb2, sinks, obase, obase32, lbase, a.H, a.scale_log2, rows, nslots_all,
                                 token,
                                 blockIdx.y * (kNW * kHeadsPerWave), kNW * kHeadsPerWave,
                                 reinterpret_cast<float*>(lds), kNW * kWave);
    return;
  }

  // Epilogue: normalise, write out (or the split partial) and the LSE.  Lane
  // (g, r) holds, for head 16*hb + r, columns 32p + 8g .. 32p + 8g + 7 in
  // blocks 2p and 2p + 1: normalised, they go out as one 16-byte store each.
  //
  // Vector-memory stores and loads share one in-order counter, so a register
  // reload from scratch placed between the stores would wait for every store
  // before it to be acknowledged.  Hence: the lane's coordinates are taken
  // afresh from the hardware (nothing address-like is carried across the tile
  // loop to be spilled), every value is normalised and packed first, and the
  // stores follow behind a compiler barrier.
  uint32_t lane_e;
  __asm__ volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane_e));
  const int r_e = (int)(lane_e & 15);
  const int g_e = (int)(lane_e >> 4);
  float inv_h[2], ltot_h[2], mout_h[2];
#pragma unroll
  for (int hb = 0; hb < 2; ++hb) {
    float l_tot = lsum[hb];
    l_tot += __shfl_xor(l_tot, 16, kWave);
    l_tot += __shfl_xor(l_tot, 32, kWave);
    float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    const int h = head0 + 16 * hb + r_e;
    float m_out = m_ref[hb];
    if constexpr (Geo::kRowLists) {
      // O is normalised by the rounded weights (see SoftmaxSlices), the LSE by
      // the exact sum.
      float l_r = lsum_r[hb];
      l_r += __shfl_xor(l_r, 16, kWave);
      l_r += __shfl_xor(l_r, 32, kWave);
      inv = l_r > 0.f ? 1.f / l_r : 0.f;
      if (sinks) {
        // The sink adds exp(sink) to the denominator only: against M = max(m_ref,
        // sink), l = l 2^(m_ref - M) + 2^(sink - M) and O scales by 2^(m_ref - M).
        const float sink = sinks[min(h, a.H - 1)] * 1.4426950408889634f;
        const float mm = fmaxf(m_ref[hb], sink);
        const float so = fast_exp2(m_ref[hb] - mm);  // 0 when no slot was valid (m_ref = -inf)
        const float es = fast_exp2(sink - mm);
        l_tot = l_tot * so + es;
        inv = so / (l_r * so + es);
        m_out = mm;
      }
    }
    if (Geo::kRowLists && !row_active) {  // padded row: out = 0, lse = 0
      inv = 0.f;
      l_tot = 1.f;
      m_out = 0.f;
    }
    inv_h[hb] = inv;
    ltot_h[hb] = l_tot;
    mout_h[hb] = m_out;
  }
  if (Geo::kRowLists && obase32) {
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      if (!hb_on[hb]) continue;
      float* orow = obase32 + ((int64_t)token * a.H + head0 + 16 * hb + r_e) * kMlaDV + 8 * g_e;
#pragma unroll
      for (int p2 = 0; p2 < kMlaDV / 32; ++p2) {
        *reinterpret_cast<f32x4*>(orow + 32 * p2) = o[hb][2 * p2] * inv_h[hb];
        *reinterpret_cast<f32x4*>(orow + 32 * p2 + 4) = o[hb][2 * p2 + 1] * inv_h[hb];
      }
    }
  } else {
    u32x4 pk[2][kMlaDV / 32];
#pragma unroll
    for (int hb = 0; hb < 2; ++hb)
#pragma unroll
      for (int p2 = 0; p2 < kMlaDV / 32; ++p2) {
        const f32x4& x = o[hb][2 * p2];
        const f32x4& y = o[hb][2 * p2 + 1];
        const float inv = inv_h[hb];
        pk[hb][p2] = u32x4{pack2<kF16>(x[0] * inv, x[1] * inv), pack2<kF16>(x[2] * inv, x[3] * inv),
                           pack2<kF16>(y[0] * inv, y[1] * inv), pack2<kF16>(y[2] * inv, y[3] * inv)};
      }
    // Every packed value exists before the first store (none is sunk into a
    // store's branch, where it would need the reloads the order avoids).
#pragma unroll
    for (int hb = 0; hb < 2; ++hb)
#pragma unroll
      for (int p2 = 0; p2 < kMlaDV / 32; ++p2) __asm__ __volatile__("" : "+v"(pk[hb][p2]));
    __asm__ __volatile__("" ::: "memory");
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      if (!hb_on[hb]) continue;
      uint16_t* orow = obase + ((int64_t)token * a.H + head0 + 16 * hb + r_e) * kMlaDV + 8 * g_e;
#pragma unroll
      for (int p2 = 0; p2 < kMlaDV / 32; ++p2) *reinterpret_cast<u32x4*>(orow + 32 * p2) = pk[hb][p2];
    }
  }
#pragma unroll
  for (int hb = 0; hb < 2; ++hb)
    if (hb_on[hb] && g_e == 0)
      lbase[(int64_t)token * a.H + head0 + 16 * hb + r_e] =
          ltot_h[hb] > 0.f ? (mout_h[hb] + fast_log2(ltot_h[hb])) * 0.69314718055994531f : -__builtin_huge_valf();
}

template <int kNW, bool kF16, int kD, bool kPaged>
__global__ __launch_bounds__(kNW * kWave) void sparse_mla_kernel(MlaArgs a) {
  sparse_mla_body<kNW, kF16, kD, kPaged, kStages>(a);
}

template <int kNW, bool kF16>
__global__ __launch_bounds__(kNW * kWave) void sparse_mla_rows2_kernel(MlaArgs a) {
  sparse_mla_body<kNW, kF16, 512, false, 2>(a);
}

// Merge split partials: lse = log(sum_i exp(lse_i) [+ exp(sink)]),
// out = sum_i exp(lse_i - lse) * o_i.  kF32: partials and out are fp32 (row
// lists with an fp32 output), else 16-bit.  kU: splits visited at a time; with
// at most kU splits (the launch picks kU >= splits up to 8) every LSE and
// partial of the row is loaded at once, in one round trip.
template <bool kF16, bool kF32, int kU>
__global__ __launch_bounds__(256) void sparse_mla_combine_kernel(const void* __restrict__ part_o,
                                                                 const float* __restrict__ part_lse, int splits,
                                                                 int64_t rows, const float* __restrict__ sinks,
                                                                 const int32_t* __restrict__ slot_count, int H,
                                                                 void* __restrict__ out, float* __restrict__ lse) {
  // One thread per (row = token*H + head, 8 columns).
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = gid >> 6;
  const int c = (int)(gid & 63) * 8;
  if (row >= rows) return;
  // 8 columns of partial i as 8 floats.
  auto load8 = [&](int64_t i, float (&x)[8]) {
    if constexpr (kF32) {
      const float* p = static_cast<const float*>(part_o) + (i * rows + row) * kMlaDV + c;
      const f32x4 lo = *reinterpret_cast<const f32x4*>(p), hi = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x[j] = lo[j];
        x[4 + j] = hi[j];
      }
    } else {
      const u32x4 v = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(part_o) + (i * rows + row) * kMlaDV + c);
      const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x[2 * j] = unpack_lo<kF16>(vv[j]);
        x[2 * j + 1] = unpack_hi<kF16>(vv[j]);
      }
    }
  };
  auto store8 = [&](const float (&x)[8]) {
    if constexpr (kF32) {
      float* p = static_cast<float*>(out) + row * kMlaDV + c;
      *reinterpret_cast<f32x4*>(p) = f32x4{x[0], x[1], x[2], x[3]};
      *reinterpret_cast<f32x4*>(p + 4) = f32x4{x[4], x[5], x[6], x[7]};
    } else {
      *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + row * kMlaDV + c) =
          u32x4{pack2<kF16>(x[0], x[1]), pack2<kF16>(x[2], x[3]), pack2<kF16>(x[4], x[5]), pack2<kF16>(x[6], x[7])};
    }
  };
  if (slot_count && slot_count[row / H] < 0) {  // padded query row of a row-list call
    const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    store8(z);
    if (c == 0) lse[row] = 0.f;
    return;
  }
  // Splits are visited kU at a time, every load of a group issued before any is
  // used (a split-serial loop is a chain of load latencies); the sums keep the
  // split order.
  const float sink = sinks ? sinks[row % H] : -__builtin_huge_valf();
  if (splits <= kU) {
    float li[kU];
    float v[kU][8];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int i = min(u, splits - 1);  // clamped: a real partial, unused past splits
      li[u] = u < splits ? part_lse[(int64_t)i * rows + row] : -__builtin_huge_valf();
      load8(i, v[u]);
    }
    float m1 = sink;
#pragma unroll
    for (int u = 0; u < kU; ++u) m1 = fmaxf(m1, li[u]);
    float a1[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float ws = sinks && m1 != -__builtin_huge_valf() ? __expf(sink - m1) : 0.f;
    if (m1 != -__builtin_huge_valf()) {
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        if (li[u] == -__builtin_huge_valf()) continue;
        const float w = __expf(li[u] - m1);
        ws += w;
#pragma unroll
        for (int j = 0; j < 8; ++j) a1[j] += w * v[u][j];
      }
    }
    const float inv1 = ws > 0.f ? 1.f / ws : 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) a1[j] *= inv1;
    store8(a1);
    if (c == 0) lse[row] = ws > 0.f ? m1 + __logf(ws) : -__builtin_huge_valf();
    return;
  }
  float mx = sink;
  for (int i0 = 0; i0 < splits; i0 += kU) {
    float li[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u)
      li[u] = i0 + u < splits ? part_lse[(int64_t)(i0 + u) * rows + row] : -__builtin_huge_valf();
#pragma unroll
    for (int u = 0; u < kU; ++u) mx = fmaxf(mx, li[u]);
  }
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float wsum = sinks && mx != -__builtin_huge_valf() ? __expf(sink - mx) : 0.f;
  if (mx != -__builtin_huge_valf()) {
    for (int i0 = 0; i0 < splits; i0 += kU) {
      float li[kU];
      float v[kU][8];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int i = min(i0 + u, splits - 1);  // clamped: a real partial, unused past splits
        li[u] = i0 + u < splits ? part_lse[(int64_t)i * rows + row] : -__builtin_huge_valf();
        load8(i, v[u]);
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        if (li[u] == -__builtin_huge_valf()) continue;
        const float w = __expf(li[u] - mx);
        wsum += w;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += w * v[u][j];
      }
    }
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] *= inv;
  store8(acc);
  if (c == 0) lse[row] = wsum > 0.f ? mx + __logf(wsum) : -__builtin_huge_valf();
}

// Few rows: split each row's slot list over workgroups until the grid fills
// the CUs.  A split costs a partial write and a share of the combine, so past
// 8 tiles a row keeps at least 4 tiles per split (one query row with 2048
// slots: 64 one-tile splits take 65 us, 16 four-tile splits 36 us); short
// lists (a V4 window) split down to single tiles.
int mla_choose_splits(int64_t tokens, int64_t head_groups, int64_t topk) {
  const int64_t wgs = tokens * head_groups;
  const int tiles = (int)((topk + kMlaTile - 1) / kMlaTile);
  const int max_splits = tiles > 8 ? tiles / 4 : tiles;
  int splits = (int)((topk + kSlotsCap - 1) / kSlotsCap);  // each split's slots must fit in LDS
  while (wgs * splits < 256 && splits * 2 <= max_splits) splits *= 2;
  return splits;
}

static int64_t mla_keys_per_split(int64_t topk, int splits) {
  const int64_t per = (topk + splits - 1) / splits;
  return ((per + kMlaTile - 1) / kMlaTile) * kMlaTile;
}

// Split partials: O (16-bit, or fp32 for an fp32 output) and the LSE per (split, token, head).
size_t mla_workspace_bytes(int64_t tokens, int64_t H, int64_t topk, bool f32) {
  const int64_t hg = (H + 127) / 128;
  const int splits = mla_choose_splits(tokens, hg, topk);
  if (splits == 1) return 0;
  return (size_t)splits * tokens * H * (kMlaDV * (f32 ? 4 : 2) + 4) + 256;
}

bool mla_decode_applies(int64_t T, int64_t H, int64_t topk);
size_t mla_decode_part_bytes(int64_t T, int64_t H, int64_t topk);
hipError_t launch_mla_decode_rows(int is_fp16, const void* q, const void* kv, const int32_t* indices,
                                  const int32_t* block_table, const int32_t* q_len, const int32_t* kv_len, int64_t B,
                                  int64_t S, int64_t G, int64_t H, int64_t Skv, int64_t block_size,
                                  int64_t max_blocks, int64_t topk, float sm_scale, int causal, void* out, float* lse,
                                  void* workspace, hipStream_t stream);

// Workspace of launch_sparse_mla: decode rows take the decode kernel's partials.
size_t sparse_mla_workspace_bytes(int64_t tokens, int64_t H, int64_t topk) {
  return mla_decode_applies(tokens, H, topk) ? mla_decode_part_bytes(tokens, H, topk)
                                             : mla_workspace_bytes(tokens, H, topk, false);
}

// Split partials of the allocation-free entry (dsa_sparse_mla_fwd_noalloc): one
// array per GPU, resident from the library's load on that GPU until the process
// ends.  64 MiB holds the split partials of decode batches up to 64 sequences x
// 128 heads x topk 2048 (33.7 MB).  Every partial slot the kernels read is
// written earlier in the same call (a split with no valid slot writes zeros and
// an LSE of -inf), so nothing needs clearing between calls; calls that overlap
// on one GPU share the array and race.
constexpr size_t kMlaScratchBytes = size_t(64) << 20;
static __device__ __align__(256) uint8_t scratch[kMlaScratchBytes];

size_t mla_scratch_bytes() { return kMlaScratchBytes; }

// The device address of `scratch` on the current device.  In host code the
// array's name only stands for the symbol; its address on a GPU comes from
// hipGetSymbolAddress, looked up once per device (each GPU holds its own copy)
// and kept.
hipError_t mla_scratch_ptr(void** out) {
  static std::once_flag once[kMaxDevices];
  static void* addr[kMaxDevices];
  static hipError_t result[kMaxDevices];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::call_once(once[dev], [&] { result[dev] = hipGetSymbolAddress(&addr[dev], HIP_SYMBOL(scratch)); });
  *out = result[dev] == hipSuccess ? addr[dev] : nullptr;
  return result[dev];
}

template <int kNW, bool kF16, int kD, bool kPaged>
static hipError_t launch_mla_kernel(const MlaArgs& a, int head_groups, hipStream_t stream) {
  const dim3 grid((unsigned)((int64_t)a.B * a.S * a.G * a.splits), (unsigned)head_groups);
  if constexpr (kD == 512 && kNW <= 2) {
    // Two-stage ring for the 512-wide row lists of up to 64 heads (see the kernel).
    constexpr int kLds = MlaLayout<512, 2>::kLds;
    const hipError_t ea = set_dynamic_lds_once<sparse_mla_rows2_kernel<kNW, kF16>>(kLds);
    if (ea != hipSuccess) return ea;
    hipLaunchKernelGGL((sparse_mla_rows2_kernel<kNW, kF16>), grid, dim3(kNW * kWave), kLds, stream, a);
  } else {
    constexpr int kLds = MlaLayout<kD, kStages>::kLds;
    const hipError_t ea = set_dynamic_lds_once<sparse_mla_kernel<kNW, kF16, kD, kPaged>>(kLds);
    if (ea != hipSuccess) return ea;
    hipLaunchKernelGGL((sparse_mla_kernel<kNW, kF16, kD, kPaged>), grid, dim3(kNW * kWave), kLds, stream, a);
  }
  return hipGetLastError();
}

// Row lists (D = 512) never use a block table.
template <int kNW, bool kF16, int kD>
static hipError_t launch_mla_nw(const MlaArgs& a, int head_groups, hipStream_t stream) {
  if constexpr (kD == 576) {
    if (a.block_table) return launch_mla_kernel<kNW, kF16, kD, true>(a, head_groups, stream);
  }
  return launch_mla_kernel<kNW, kF16, kD, false>(a, head_groups, stream);
}

template <bool kF16, int kD>
static hipError_t launch_mla_dtype(const MlaArgs& a, int head_groups, int hpg, hipStream_t stream) {
  hipError_t e;
  if (hpg > 64) e = launch_mla_nw<4, kF16, kD>(a, head_groups, stream);
  else if (hpg > 32) e = launch_mla_nw<2, kF16, kD>(a, head_groups, stream);
  else e = launch_mla_nw<1, kF16, kD>(a, head_groups, stream);
  if (e != hipSuccess || a.splits == 1) return e;
  const int64_t rows = (int64_t)a.B * a.S * a.G * a.H;
  const int64_t threads = rows * (kMlaDV / 8);
  const dim3 grid((unsigned)((threads + 255) / 256));
  if (a.out32)
    hipLaunchKernelGGL((sparse_mla_combine_kernel<kF16, true, 4>), grid, dim3(256), 0, stream, a.part_o32, a.part_lse,
                       a.splits, rows, a.sinks, a.slot_count, a.H, a.out32, a.lse);
  else if (a.splits <= 4)
    hipLaunchKernelGGL((sparse_mla_combine_kernel<kF16, false, 4>), grid, dim3(256), 0, stream, a.part_o, a.part_lse,
                       a.splits, rows, a.sinks, a.slot_count, a.H, a.out, a.lse);
  else
    hipLaunchKernelGGL((sparse_mla_combine_kernel<kF16, false, 8>), grid, dim3(256), 0, stream, a.part_o, a.part_lse,
                       a.splits, rows, a.sinks, a.slot_count, a.H, a.out, a.lse);
  return hipGetLastError();
}

// a.out32 must be set first: the partials' width follows the output's.
static void mla_set_splits(MlaArgs& a, int64_t T, int64_t H, int64_t topk, void* workspace) {
  const int head_groups = (int)((H + 127) / 128);
  a.splits = mla_choose_splits(T, head_groups, topk);
  a.keys_per_split = (int)mla_keys_per_split(topk, a.splits);
  a.part_o = nullptr;
  a.part_o32 = nullptr;
  a.part_lse = nullptr;
  if (a.splits > 1) {
    const size_t ebytes = a.out32 ? 4 : 2;
    a.part_o = static_cast<uint16_t*>(workspace);
    a.part_o32 = a.out32 ? static_cast<float*>(workspace) : nullptr;
    a.part_lse = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + (size_t)a.splits * T * H * kMlaDV * ebytes);
  }
}

// Caller validated: d_qk 576, d_v 512, H (heads per KV group) % 16 == 0, 16-bit inputs,
// workspace >= sparse_mla_workspace_bytes(B * S * G, H, topk), physical KV rows times G < 2^31.
hipError_t launch_sparse_mla(int is_fp16, const void* q, const void* kv, const int32_t* indices,
                             const int32_t* block_table, const int32_t* q_len, const int32_t* kv_len, int64_t B,
                             int64_t S, int64_t G, int64_t H, int64_t Skv, int64_t block_size, int64_t max_blocks,
                             int64_t topk, float sm_scale, int causal, void* out, float* lse, void* workspace,
                             hipStream_t stream) {
  const int64_t T = B * S * G;
  if (T == 0 || H == 0) return hipSuccess;
  // Few query rows (decode): the decode kernel, slots across waves and chunks.
  if (mla_decode_applies(T, H, topk))
    return launch_mla_decode_rows(is_fp16, q, kv, indices, block_table, q_len, kv_len, B, S, G, H, Skv, block_size,
                                  max_blocks, topk, sm_scale, causal, out, lse, workspace, stream);
  MlaArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.kv = static_cast<const uint16_t*>(kv);
  a.kv2 = nullptr;
  a.indices = indices;
  a.slot_count = nullptr;
  a.sinks = nullptr;
  a.block_table = block_table;
  a.q_len = q_len;
  a.kv_len = kv_len;
  a.out = static_cast<uint16_t*>(out);
  a.out32 = nullptr;
  a.lse = lse;
  a.B = (int)B;
  a.S = (int)S;
  a.H = (int)H;
  a.Skv = (int)Skv;
  a.topk = (int)topk;
  a.G = (int)G;
  a.block_size = (int)block_size;
  a.max_blocks = (int)max_blocks;
  a.causal = causal;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  const int head_groups = (int)((H + 127) / 128);
  mla_set_splits(a, T, H, topk, workspace);
  const int hpg = H >= 128 ? 128 : (int)H;  // heads per workgroup
  return is_fp16 ? launch_mla_dtype<true, 576>(a, head_groups, hpg, stream)
                 : launch_mla_dtype<false, 576>(a, head_groups, hpg, stream);
}

// Attention of T query rows over per-row lists of physical KV rows (D = 512,
// K = V): rows[t][0 .. count[t]) index kv, or kv2 when tagged kSrc2Bit, -1 =
// empty; sinks [H] (natural log units) or null.  The V4 sparse_flash_mla
// kernel below builds the lists.  Caller validated: H % 16 == 0, H <= 1024,
// cap <= 2^31 / T, workspace >= mla_workspace_bytes(T, H, cap, out_f32).  out_f32: out is fp32.
hipError_t launch_sparse_mla_rows(int is_fp16, const void* q, const void* kv, const void* kv2, const int32_t* rows,
                                  const int32_t* count, int64_t T, int64_t H, int64_t cap, const float* sinks,
                                  float sm_scale, void* out, float* lse, void* workspace, hipStream_t stream,
                                  int out_f32) {
  if (T == 0 || H == 0) return hipSuccess;
  MlaArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.kv = static_cast<const uint16_t*>(kv);
  a.kv2 = static_cast<const uint16_t*>(kv2);
  a.indices = rows;
  a.slot_count = count;
  a.sinks = sinks;
  a.block_table = nullptr;
  a.q_len = nullptr;
  a.kv_len = nullptr;
  a.out = out_f32 ? nullptr : static_cast<uint16_t*>(out);
  a.out32 = out_f32 ? static_cast<float*>(out) : nullptr;
  a.lse = lse;
  a.B = 1;
  a.S = (int)T;
  a.H = (int)H;
  a.Skv = 0x7fffffff;
  a.topk = (int)cap;
  a.G = 1;
  a.block_size = 0;
  a.max_blocks = 0;
  a.causal = 0;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  const int head_groups = (int)((H + 127) / 128);
  mla_set_splits(a, T, H, cap, workspace);
  const int hpg = H >= 128 ? 128 : (int)H;
  return is_fp16 ? launch_mla_dtype<true, 512>(a, head_groups, hpg, stream)
                 : launch_mla_dtype<false, 512>(a, head_groups, hpg, stream);
}

}  // namespace dsa
