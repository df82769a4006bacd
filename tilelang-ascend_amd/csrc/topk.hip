// Row-wise top-k selector: deterministic radix select on gfx950.
//
// Semantics (examples/deepseek_v4/lightning_indexer.py:317-325, the stable rule
// the build adopts for examples/topk_selector/example_topk_selector.py:57-58):
// per row, the k largest scores under the order (value desc, index asc); a
// score <= -1e30 (masked, -inf) or NaN never takes a slot, slots left over hold
// index -1 / value -inf.  With `sorted` the row comes out in that order (as the
// reference's Sort/TopK templates produce, src/tl_templates/ascend/common.h:1685-1899);
// without it the selected set comes out in a fixed, data-determined order
// (ascending index among the strictly-above-threshold elements, ties appended).
//
// One 1024-thread workgroup owns one row.  The row is read from HBM once with
// 16-byte loads; when it fits, its order-preserving uint32 keys stay in LDS
// for the later passes.  Three LDS-histogram passes (11/11/10 key bits, atomics
// into 2048 bins, a block scan to find the bin holding the k-th key) fix the
// threshold key exactly; a pass stops early once a bin is taken whole.  The
// output pass walks the row in index order with block-wide prefix sums, so the
// (k - #above) lowest-index elements equal to the threshold win the ties,
// deterministically.  `sorted` then runs a bitonic network over
// (key << 32 | ~index) in LDS.
#include <algorithm>

#include "common.hpp"

namespace dsa {

constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / kWave;
constexpr int kHistBins = 2048;
constexpr int kRedWords = 64;
constexpr int kLdsBytes = 160 * 1024;
constexpr int kRowsStaticLds = (kTopkThreads / kWave) * 8;  // topk_rows_kernel's flag masks

// Inclusive wave scan and wave reductions on DPP (row shifts, then the row
// broadcasts 15 and 31).
#define DSA_DPP(old, x, ctrl, rmask) __builtin_amdgcn_update_dpp((int)(old), (int)(x), ctrl, rmask, 0xf, false)

__device__ __forceinline__ uint32_t wave_scan_add(uint32_t x) {
  x += (uint32_t)DSA_DPP(0, x, 0x111, 0xf);
  x += (uint32_t)DSA_DPP(0, x, 0x112, 0xf);
  x += (uint32_t)DSA_DPP(0, x, 0x114, 0xf);
  x += (uint32_t)DSA_DPP(0, x, 0x118, 0xf);
  x += (uint32_t)DSA_DPP(0, x, 0x142, 0xa);
  x += (uint32_t)DSA_DPP(0, x, 0x143, 0xc);
  return x;
}

// Block-wide exclusive scan of one uint32 per thread; `total` receives the sum.
// Uses red[0..kTopkWaves); with kTrailingBarrier it ends with a barrier so red
// can be reused.
template <bool kTrailingBarrier = true>
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* red, uint32_t& total) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t incl = wave_scan_add(v);
  if (lane == kWave - 1) red[wave] = incl;
  __syncthreads();
  // Lanes 0..15 scan the 16 wave totals.
  uint32_t w = lane < kTopkWaves ? red[lane] : 0u;
  w += (uint32_t)DSA_DPP(0, w, 0x111, 0xf);
  w += (uint32_t)DSA_DPP(0, w, 0x112, 0xf);
  w += (uint32_t)DSA_DPP(0, w, 0x114, 0xf);
  w += (uint32_t)DSA_DPP(0, w, 0x118, 0xf);
  total = (uint32_t)__builtin_amdgcn_readlane((int)w, kTopkWaves - 1);
  const uint32_t before = wave ? (uint32_t)__builtin_amdgcn_readlane((int)w, wave - 1) : 0u;
  if constexpr (kTrailingBarrier) __syncthreads();
  return before + incl - v;
}

template <bool kCached>
__device__ __forceinline__ uint32_t load_key(const float* __restrict__ xr, const uint32_t* keys, int i) {
  if constexpr (kCached) return keys[i];
  return float_key(xr[i]);
}

// One row by the whole workgroup (every thread calls it, with the same row), in
// `lds`: (kHistBins + kRedWords) words, kpad * 8 bytes when sorted, then the
// row's keys when kCached.
template <bool kCached>
__device__ __forceinline__ void radix_row(const int row, const float* __restrict__ x, int64_t ld, int n, int k,
                                          const int32_t* __restrict__ row_len, int sorted, int kpad,
                                          int32_t* __restrict__ out_idx, float* __restrict__ out_val,
                                          int only_flagged, const int32_t* __restrict__ idx_map, uint32_t* lds) {
  uint32_t* hist = lds;                                     // kHistBins
  uint32_t* red = hist + kHistBins;                         // kRedWords
  uint64_t* sbuf = reinterpret_cast<uint64_t*>(red + kRedWords);  // kpad (sorted only)
  uint32_t* keys = reinterpret_cast<uint32_t*>(sbuf + (sorted ? kpad : 0));

  const int tid = threadIdx.x;
  const float* __restrict__ xr = x + (int64_t)row * ld;
  int32_t* __restrict__ oi = out_idx + (int64_t)row * k;
  float* __restrict__ ov = out_val ? out_val + (int64_t)row * k : nullptr;
  // Second pass behind topk_reg_kernel: only the rows it handed over.  Over
  // packed candidate rows (idx_map), a negative row length keeps the flag: the
  // row's candidates are incomplete and it needs its dense logits.
  if (only_flagged && oi[0] != kFallbackFlag) return;
  if (idx_map && row_len[row] < 0) return;
  __syncthreads();  // every thread has read the flag before any overwrites it
  int nv = n;
  if (row_len) nv = min(max(row_len[row], 0), n);
  const int32_t* __restrict__ imap = idx_map ? idx_map + (int64_t)row * ld : nullptr;

  for (int b = tid; b < kHistBins; b += kTopkThreads) hist[b] = 0;
  __syncthreads();

  // ---- pass 0: stream the row once, cache keys, histogram the top 11 bits ----
  uint32_t present = 0;
  const bool vec = ((reinterpret_cast<uintptr_t>(xr) & 15) == 0);
  int head = 0;
  if (vec) {
    const int n4 = nv >> 2;
    const f32x4* x4 = reinterpret_cast<const f32x4*>(xr);
    for (int i = tid; i < n4; i += kTopkThreads) {
      const f32x4 v = __builtin_nontemporal_load(&x4[i]);
      uint32_t kk0 = float_key(v[0]), kk1 = float_key(v[1]), kk2 = float_key(v[2]), kk3 = float_key(v[3]);
      if constexpr (kCached) {
        *reinterpret_cast<u32x4*>(&keys[4 * i]) = u32x4{kk0, kk1, kk2, kk3};
      }
      if (kk0 > kKeyInvalidMax) { ++present; atomicAdd(&hist[kk0 >> 21], 1u); }
      if (kk1 > kKeyInvalidMax) { ++present; atomicAdd(&hist[kk1 >> 21], 1u); }
      if (kk2 > kKeyInvalidMax) { ++present; atomicAdd(&hist[kk2 >> 21], 1u); }
      if (kk3 > kKeyInvalidMax) { ++present; atomicAdd(&hist[kk3 >> 21], 1u); }
    }
    head = n4 << 2;
  }
  for (int i = head + tid; i < nv; i += kTopkThreads) {
    uint32_t kk0 = float_key(xr[i]);
    if constexpr (kCached) keys[i] = kk0;
    if (kk0 > kKeyInvalidMax) { ++present; atomicAdd(&hist[kk0 >> 21], 1u); }
  }
  uint32_t m_total;
  (void)block_excl_scan(present, red, m_total);  // also orders the histogram atomics
  const int kk = min((int)m_total, k);

  uint32_t prefix = 0, pmask = 0;
  int need = kk;
  bool complete = (kk == 0);
  for (int pass = 0; pass < 3 && !complete; ++pass) {
    const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
    const uint32_t bmask = pass == 2 ? 0x3ffu : 0x7ffu;
    if (pass > 0) {
      for (int b = tid; b < kHistBins; b += kTopkThreads) hist[b] = 0;
      __syncthreads();
      for (int i = tid; i < nv; i += kTopkThreads) {
        uint32_t key = load_key<kCached>(xr, keys, i);
        if (key > kKeyInvalidMax && (key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & bmask], 1u);
      }
      __syncthreads();
    }
    // Thread t owns bins 2047-2t (hi) and 2046-2t (lo): descending order.
    const int bhi = kHistBins - 1 - 2 * tid, blo = bhi - 1;
    const uint32_t chi = hist[bhi], clo = hist[blo];
    uint32_t tot;
    const uint32_t excl = block_excl_scan(chi + clo, red, tot);
    const uint32_t incl = excl + chi + clo;
    if (excl < (uint32_t)need && incl >= (uint32_t)need) {
      if (excl + chi >= (uint32_t)need) {
        red[kTopkWaves + 0] = bhi; red[kTopkWaves + 1] = excl; red[kTopkWaves + 2] = chi;
      } else {
        red[kTopkWaves + 0] = blo; red[kTopkWaves + 1] = excl + chi; red[kTopkWaves + 2] = clo;
      }
    }
    __syncthreads();
    const uint32_t bin = red[kTopkWaves + 0], above = red[kTopkWaves + 1], bcnt = red[kTopkWaves + 2];
    __syncthreads();
    need -= (int)above;
    prefix |= bin << shift;
    pmask |= bmask << shift;
    if (bcnt == (uint32_t)need) complete = true;
  }

  // ---- output pass: index-ordered, deterministic tie resolution ----
  uint32_t base_s = 0, base_e = 0;
  for (int c0 = 0; c0 < nv && kk > 0; c0 += 4 * kTopkThreads) {
    const int i0 = c0 + 4 * tid;
    uint32_t key[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) key[j] = (i0 + j < nv) ? load_key<kCached>(xr, keys, i0 + j) : 0u;
    uint32_t fs = 0, fe = 0, cs = 0, ce = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool pres = key[j] > kKeyInvalidMax;
      const uint32_t mk = key[j] & pmask;
      const bool s = pres && (mk > prefix || (complete && mk == prefix));
      const bool e = pres && !complete && mk == prefix;
      fs |= (uint32_t)s << j; fe |= (uint32_t)e << j;
      cs += s; ce += e;
    }
    uint32_t tot;
    const uint32_t ex = block_excl_scan(cs | (ce << 16), red, tot);
    uint32_t ss = base_s + (ex & 0xffffu), es = base_e + (ex >> 16);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool s = (fs >> j) & 1, e = (fe >> j) & 1;
      if (s || (e && es < (uint32_t)need)) {
        const uint32_t pos = ss + min(es, (uint32_t)need);
        const int idx = i0 + j;
        if (sorted) {
          sbuf[pos] = ((uint64_t)key[j] << 32) | (uint32_t)(~(uint32_t)idx);
        } else {
          oi[pos] = imap ? imap[idx] : idx;
          if (ov) ov[pos] = key_to_float(key[j]);
        }
      }
      ss += s;
      es += e;
    }
    base_s += tot & 0xffffu;
    base_e += tot >> 16;
    if (base_s + min(base_e, (uint32_t)need) >= (uint32_t)kk) break;
  }

  if (sorted) {
    for (int i = kk + tid; i < kpad; i += kTopkThreads) sbuf[i] = 0ull;
    __syncthreads();
    for (int size = 2; size <= kpad; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int t = tid; t < (kpad >> 1); t += kTopkThreads) {
          const int i = 2 * t - (t & (stride - 1));
          const int j = i + stride;
          const uint64_t a = sbuf[i], b = sbuf[j];
          const bool desc = (i & size) == 0;
          if (desc ? (a < b) : (a > b)) { sbuf[i] = b; sbuf[j] = a; }
        }
        __syncthreads();
      }
    }
    for (int i = tid; i < kk; i += kTopkThreads) {
      const uint64_t c = sbuf[i];
      const int32_t p = (int32_t)(~(uint32_t)c);
      oi[i] = imap ? imap[p] : p;
      if (ov) ov[i] = key_to_float((uint32_t)(c >> 32));
    }
  }
  for (int i = kk + tid; i < k; i += kTopkThreads) {
    oi[i] = -1;
    if (ov) ov[i] = -__builtin_huge_valf();
  }
}

// Every row (grid = rows), or with only_flagged the rows whose out_idx[row][0]
// is kFallbackFlag: workgroup g then takes rows g, g + G, g + 2G, ... (G =
// gridDim.x), reads 1024 of their flags at once and runs the flagged ones, so a
// launch with nothing flagged costs one flag load per thread instead of a
// workgroup (and its LDS allocation) per row.
//
// gate (flagged walk only, may be null): a count of flagged rows written by an
// earlier launch; at zero the launch ends after one scalar load per workgroup.
template <bool kCached>
__global__ __launch_bounds__(kTopkThreads) void topk_rows_kernel(
    const float* __restrict__ x, int64_t ld, int n, int k, const int32_t* __restrict__ row_len,
    int sorted, int kpad, int32_t* __restrict__ out_idx, float* __restrict__ out_val, int only_flagged,
    const int32_t* __restrict__ idx_map, int rows, const int32_t* __restrict__ gate) {
  typedef const __attribute__((address_space(4))) int32_t const_i32;
  extern __shared__ __align__(16) uint32_t rows_lds[];  // after the static `flagged` masks
  if (only_flagged && gate && *(const_i32*)gate == 0) return;  // block-uniform
  if (!only_flagged) {
    radix_row<kCached>(blockIdx.x, x, ld, n, k, row_len, sorted, kpad, out_idx, out_val, 0, idx_map, rows_lds);
    return;
  }
  __shared__ uint64_t flagged[kTopkWaves];
  static_assert(sizeof(flagged) == kRowsStaticLds, "static LDS of the flagged walk");
  const int tid = threadIdx.x;
  const int G = gridDim.x;
  for (int64_t r0 = blockIdx.x; r0 < rows; r0 += (int64_t)G * kTopkThreads) {
    const int64_t r = r0 + (int64_t)tid * G;
    const bool f = r < rows && out_idx[r * k] == kFallbackFlag;
    const uint64_t m = __builtin_amdgcn_ballot_w64(f);
    if ((tid & (kWave - 1)) == 0) flagged[tid / kWave] = m;
    __syncthreads();
    for (int w = 0; w < kTopkWaves; ++w) {
      uint64_t mw = flagged[w];  // block-uniform
      while (mw) {
        const int b = __builtin_ctzll(mw);
        mw &= mw - 1;
        radix_row<kCached>((int)(r0 + (int64_t)(w * kWave + b) * G), x, ld, n, k, row_len, sorted, kpad, out_idx,
                           out_val, 1, idx_map, rows_lds);
        __syncthreads();  // the row's LDS is free before the next one
      }
    }
    __syncthreads();  // every wave has read `flagged` before the next round writes it
  }
}


// ----------------------------------------------------------------------------
// Register-resident fast path (rows of up to 4096 * kChunks scores).
//
// The row is loaded once into VGPRs (kChunks 16-byte loads per thread, all in
// flight together) and never re-read.  One score per thread (1024, spread over
// the row) forms a sample.  A two-level histogram of the samples' order keys
// (top 10 key bits, then the next 10 inside the bin that matters) gives a
// threshold t whose expected candidate count (scores >= t) sits midway between
// k and the candidate capacity.  One pass over the registers compacts the
// candidates into LDS with wave ballots, every wave into its own region.  The
// set {score >= t} is closed upwards in the order (value desc, index asc), so
// once it holds at least k scores (or t admits every present score) it holds
// the whole top-k; otherwise t moves by bisection over the sample ranks and
// the pass repeats.  The candidates alone are then bucketed into 4096 bins of
// their binning positions (pos - pos(min)) >> shift (cand_pos: the order key
// with magnitudes far below the largest collapsed), a descending scan finds the bin
// b* holding the k-th largest, the candidates of bins >= b* are regrouped by
// bin, and each counts the entries of its own bin that beat it (bins rarely
// hold more than one): bin start + that rank is its sorted position, exact
// with ties, and it is stored there directly.  Rows the fast path cannot bound
// (no threshold with k..kCandCap candidates, a bin over kBinCap) are flagged
// in out_idx[row][0] for the exact radix kernel, launched right after on the
// same stream.
//
// Rows longer than the registers hold go through it twice.  Stage 1 runs one
// workgroup per segment of a row (nseg > 1): the segment's own sorted top-k,
// with global indices, into a candidate buffer -- every element of the row's
// top-k is in its segment's top-k under the same order.  Stage 2 selects over
// the nseg*k candidates of each row and maps positions back through idx_map
// (the candidates' original indices); among equal scores, candidate position
// order is original index order (segments are contiguous and each is sorted),
// so positions break the ties.  A row any of whose segments was flagged is
// flagged again, so that the radix kernel redoes it from the original row.
// ----------------------------------------------------------------------------
constexpr int kListCap = 4096;                   // largest k the fast path takes
constexpr int kWaveCap = 320;                    // candidates one wave may hold
constexpr int kCandCap = kWaveCap * kTopkWaves;  // 5120
constexpr int kLaneEntries = kWaveCap / kWave;   // 5
constexpr int kCandBins = 4096;
constexpr int kCandBinBits = 12;
constexpr int kSampleBins = 1024;                // per level; one sample per thread
constexpr int kBinCap = 512;                     // longest bin the rank loop walks
constexpr int kMaxTries = 12;
constexpr int kRegChunks = 8;
constexpr int kRegMax = 4 * kTopkThreads * kRegChunks;  // longest row the register path holds (32768)
constexpr uint32_t kFloorBits = 0xF149F2C9u;     // next float above -1e30f: v >= it <=> v > -1e30f
constexpr int kPosBits = 15;                     // positions inside a register row (< kRegMax)
static_assert((kRegMax - 1) >> kPosBits == 0 && kCandBins << kPosBits != 0, "bin and position share a word");

// LDS of the register path, in 32-bit words.  A wave that finds more than
// kWaveCap candidates keeps writing past its region (values into the next
// regions and the position array, positions into cnt); such a try is retried,
// and cnt is cleared after every compaction, so nothing else is reached.
constexpr int kLdsVal = 0;                            // kCandCap candidate values
constexpr int kLdsPos = kLdsVal + kCandCap;           // kCandCap candidate positions
constexpr int kLdsCnt = kLdsPos + kCandCap;           // kCandBins bin counts
constexpr int kLdsOffs = kLdsCnt + kCandBins;         // kCandBins bin offsets; before them the sample histograms
constexpr int kLdsSample = kLdsOffs + kCandBins;      // kTopkThreads sample keys (0: absent)
constexpr int kLdsRed = kLdsSample + kTopkThreads;     // reduction words
constexpr int kLdsRegWords = kLdsRed + 128;
static_assert(kWave * 4 * kRegChunks - kWaveCap <= kCandBins, "a wave's overrun must stay inside cnt");
static_assert(2 * kSampleBins <= kCandBins, "sample histograms live in the offsets array");
// Reduction words.
constexpr int kRedCoarse = 0;      // coarse sample bin of the threshold
constexpr int kRedAbove = 1;       // samples above that bin
constexpr int kRedThresh = 2;      // threshold key
constexpr int kRedFlag = 3;        // a bin over kBinCap
constexpr int kRedBstar = 4;
constexpr int kRedScan = 16;       // block_excl_scan scratch (16)
constexpr int kRedCount = 32;      // per wave: candidates held
constexpr int kRedMin = 48;        // per wave: smallest candidate
constexpr int kRedMax = 64;        // per wave: largest candidate
constexpr int kRedPresent = 80;    // per wave: present samples

// Inclusive sum / max over lanes 0..15 (row 0 of the wave), read from lane 15.
__device__ __forceinline__ uint32_t row0_sum(uint32_t x) {
  x += (uint32_t)DSA_DPP(0, x, 0x111, 0xf);
  x += (uint32_t)DSA_DPP(0, x, 0x112, 0xf);
  x += (uint32_t)DSA_DPP(0, x, 0x114, 0xf);
  x += (uint32_t)DSA_DPP(0, x, 0x118, 0xf);
  return (uint32_t)__builtin_amdgcn_readlane((int)x, 15);
}

__device__ __forceinline__ uint32_t row0_max(uint32_t x) {
  x = max(x, (uint32_t)DSA_DPP(0, x, 0x111, 0xf));
  x = max(x, (uint32_t)DSA_DPP(0, x, 0x112, 0xf));
  x = max(x, (uint32_t)DSA_DPP(0, x, 0x114, 0xf));
  x = max(x, (uint32_t)DSA_DPP(0, x, 0x118, 0xf));
  return (uint32_t)__builtin_amdgcn_readlane((int)x, 15);
}

// Max over the wave of uint32, identical in every lane.
__device__ __forceinline__ uint32_t wave_all_umax(uint32_t x) {
  x = max(x, (uint32_t)DSA_DPP(0, x, 0x111, 0xf));
  x = max(x, (uint32_t)DSA_DPP(0, x, 0x112, 0xf));
  x = max(x, (uint32_t)DSA_DPP(0, x, 0x114, 0xf));
  x = max(x, (uint32_t)DSA_DPP(0, x, 0x118, 0xf));
  x = max(x, (uint32_t)DSA_DPP(0, x, 0x142, 0xa));
  x = max(x, (uint32_t)DSA_DPP(0, x, 0x143, 0xc));
  return (uint32_t)__builtin_amdgcn_readlane((int)x, kWave - 1);
}

// The lane index computed afresh (not a value kept live across a loop).
__device__ __forceinline__ uint32_t fresh_lane() {
  uint32_t l;
  __asm__ volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

__device__ __forceinline__ uint32_t lane_prefix(uint64_t m, uint32_t add) {  // add + set bits of m below this lane
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, add));
}

// Order key with -0 folded onto +0 (x + 0 turns -0 into +0); NaN never reaches it.
__device__ __forceinline__ uint32_t cand_key(float x) {
  const uint32_t u = __float_as_uint(x + 0.0f);
  return u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);
}

// Binning position of a candidate: the order key with every magnitude below
// `floor_bits` collapsed onto zero.  Monotone non-decreasing in the value, so
// bins stay ordered and the in-bin ranking stays exact.  The plain key spreads
// the binades near zero over ~2^31 of its range: candidates on both sides of
// zero then crowded a few bins, and ranking a bin costs its size squared (up to
// 60 us for one C2 row).  Such rows collapse the magnitudes more than
// kBinBinades binades under the largest candidate magnitude; rows of one sign
// keep the plain key (floor_bits = 0).
constexpr uint32_t kBinBinades = 12;
__device__ __forceinline__ uint32_t cand_pos(float x, uint32_t floor_bits) {
  const uint32_t u = __float_as_uint(x + 0.0f);
  const uint32_t mag = u & 0x7fffffffu;
  const uint32_t cm = mag > floor_bits ? mag - floor_bits : 0u;
  return (u >> 31) ? 0x80000000u - cm : 0x80000000u + cm;
}

// Four absent scores: what a register group past a row's last whole group of 4 reads.
__device__ __align__(16) float kTopkAbsent4[4] = {-__builtin_huge_valf(), -__builtin_huge_valf(),
                                                  -__builtin_huge_valf(), -__builtin_huge_valf()};

// Ballot compaction of the scores >= t among a thread's registers into
// lv/lp from index `base` on (wave-uniform), registers in the order the row's
// loads are issued (with 8 chunks the even ones first); returns the wave's
// count.  Position of register (c, j): e4 + 4096 c + j, or with kLaneMajor
// e4 + 1024 (4 c + j).
template <int kChunks, bool kLaneMajor = false>
__device__ __forceinline__ uint32_t compact_scores(const float (&v)[kChunks][4], float t, uint32_t base, uint32_t e4,
                                                   uint32_t* lv, uint32_t* lp) {
  uint32_t wcnt = 0;  // wave-uniform
  // Opaque copy: keeps the 32 positions from being hoisted out of a retry loop as live registers.
  uint32_t e4o;
  __asm__ volatile("v_mov_b32 %0, %1" : "=v"(e4o) : "v"(e4));
#pragma unroll
  for (int q = 0; q < kChunks; ++q)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = kChunks == 8 ? 2 * (q & 3) + (q >> 2) : q;
      const float val = v[c][j];
      const bool p = val >= t;
      const uint64_t m = __builtin_amdgcn_ballot_w64(p);
      if (p) {
        const uint32_t i = lane_prefix(m, base + wcnt);
        lv[i] = __float_as_uint(val);
        lp[i] = e4o + (uint32_t)(kLaneMajor ? kTopkThreads * (4 * c + j) : 4 * kTopkThreads * c + j);
      }
      wcnt += (uint32_t)__builtin_popcountll(m);
    }
  return wcnt;
}

// One wave: the bin of a 1024-bin histogram holding the r-th largest entry
// (1 <= r <= total); `above` receives the entries in higher bins.
__device__ __forceinline__ int rank_bin(const uint32_t* h, uint32_t r, uint32_t& above) {
  const int lane = threadIdx.x & (kWave - 1);
  // Lane l sums bins [1008 - 16 l, 1024 - 16 l): lane 0 holds the top bins.
  const u32x4* h4 = reinterpret_cast<const u32x4*>(h) + (kSampleBins / 4 - 4 - 4 * lane);
  uint32_t sum = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const u32x4 t = h4[q];
    sum += t.x + t.y + t.z + t.w;
  }
  const uint32_t incl = wave_scan_add(sum);
  const int L = (int)__builtin_ctzll(__builtin_amdgcn_ballot_w64(incl >= r));
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)(incl - sum), L);
  // Lanes 0..15 take lane L's bins from the top down.
  const uint32_t c = lane < 16 ? h[kSampleBins - 1 - 16 * L - lane] : 0u;
  uint32_t ci = c;
  ci += (uint32_t)DSA_DPP(0, ci, 0x111, 0xf);
  ci += (uint32_t)DSA_DPP(0, ci, 0x112, 0xf);
  ci += (uint32_t)DSA_DPP(0, ci, 0x114, 0xf);
  ci += (uint32_t)DSA_DPP(0, ci, 0x118, 0xf);
  const int i = (int)__builtin_ctzll(__builtin_amdgcn_ballot_w64(lane < 16 && a + ci >= r));
  above = a + (uint32_t)__builtin_amdgcn_readlane((int)(ci - c), i);
  return kSampleBins - 1 - 16 * L - i;
}

// Slot, in its row's candidate block, of packed position p (soff[z]: pairs in
// the chunks below z; 2^30 past the last chunk).
__device__ __forceinline__ int cand_slot(const int (&soff)[kCandMaxSeg], int cap, int p) {
  int s = p;
#pragma unroll
  for (int z = 1; z < kCandMaxSeg; ++z) s += p >= soff[z] ? cap - (soff[z] - soff[z - 1]) : 0;
  return s;
}

// A candidate row the register path hands to the radix kernel: its pairs
// packed in position order into pval / pidx, and counted.
__device__ void cand_spill(const CandSegments& cs, const u32x2* crow, const int (&soff)[kCandMaxSeg], int row,
                           int nv) {
  if (threadIdx.x == 0 && cs.nspill) atomicAdd(cs.nspill, 1);
  float* pv = cs.pval + (int64_t)row * cs.ldc;
  int32_t* pi = cs.pidx + (int64_t)row * cs.ldc;
  for (int p = threadIdx.x; p < nv; p += kTopkThreads) {
    const u32x2 e = crow[cand_slot(soff, cs.cap, p)];
    pv[p] = __uint_as_float(e.x);
    pi[p] = (int32_t)e.y;
  }
}

// kCand: the rows are the fused indexer's candidates in their key chunks (cs;
// x, row_len and idx_map unused), positions 0..ldc; thread t holds positions
// t + 1024 (4 c + j), so a wave's loads of one register are contiguous.
template <int kChunks, bool kFull, bool kCand = false, bool kAligned = false>
__global__ __launch_bounds__(kTopkThreads) __attribute__((amdgpu_waves_per_eu(8, 8))) void topk_reg_kernel(
    const float* __restrict__ x, int64_t ld, int n, int k, const int32_t* __restrict__ row_len,
    int32_t* __restrict__ out_idx, float* __restrict__ out_val, int nseg, int seg_len,
    const int32_t* __restrict__ idx_map, const CandSegments cs) {
  static_assert(!(kFull && kCand), "candidate rows are ragged");
  static_assert(!(kAligned && (kFull || kCand)), "kAligned: ragged rows of 16-byte aligned scores");
  __shared__ __align__(16) uint32_t lds[kLdsRegWords];
  uint32_t* lv = lds + kLdsVal;
  uint32_t* lp = lds + kLdsPos;
  uint32_t* cnt = lds + kLdsCnt;
  uint32_t* offs = lds + kLdsOffs;
  uint32_t* shc = offs;                // coarse sample histogram
  uint32_t* shf = offs + kSampleBins;  // fine sample histogram
  uint32_t* red = lds + kLdsRed;
  const int vrow = blockIdx.x;  // output row: segment vrow % nseg of input row vrow / nseg
  const int row = vrow / nseg;
  const int seg = vrow - row * nseg;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int base = seg * seg_len;  // index of this segment's first element
  const float* __restrict__ xr = x + (int64_t)row * ld + base;
  int32_t* __restrict__ oi = out_idx + (int64_t)vrow * k;
  float* __restrict__ ov = out_val ? out_val + (int64_t)vrow * k : nullptr;
  const int32_t* __restrict__ imap = idx_map ? idx_map + (int64_t)row * ld : nullptr;
  int nv = n;
  if (row_len) nv = min(max(row_len[row], 0), n);
  nv = min(max(nv - base, 0), seg_len);
  int soff[kCandMaxSeg];
  const u32x2* crow = nullptr;
  if constexpr (kCand) {
    crow = cs.cand + (int64_t)row * cs.nseg * cs.cap;
    int tot = 0;
    bool over = false;
#pragma unroll
    for (int z = 0; z < kCandMaxSeg; ++z) {
      soff[z] = z < cs.nseg ? tot : (1 << 30);
      if (z < cs.nseg) {
        const int c = cs.count[(int64_t)row * cs.nseg + z];
        over |= c > cs.cap;
        tot += min(c, cs.cap);
      }
    }
    const bool back = over || tot > cs.ldc || (tot < k && cs.thr[row] != -__builtin_huge_valf());
    if (tid == 0) cs.plen[row] = back ? -1 : tot;
    if (back) {
      if (tid == 0) {
        oi[0] = kFallbackFlag;  // the radix kernel leaves it for the dense path
        if (cs.nback) atomicAdd(cs.nback, 1);
      }
      return;  // block-uniform
    }
    nv = tot;
  }
  if (imap) {
    // Stage 2: a flagged segment (its first candidate index) sends the whole row to the exact path.
    bool flagged = false;
    for (int sg = 0; sg * k < n; ++sg) flagged |= imap[sg * k] == kFallbackFlag;
    if (flagged) {
      if (tid == 0) oi[0] = kFallbackFlag;
      return;  // block-uniform
    }
  }

  // A row this path cannot bound (block-uniform): a whole row (kFull, one
  // segment) takes the exact radix select right here, in the same LDS, so the
  // launch needs no pass behind; other rows are flagged for the exact pass, and
  // candidate rows also copied out packed for it.  (Inlined into the ragged
  // variants, the select's registers made their main path spill.)
  auto hand_over = [&]() {
    if constexpr (kCand) {
      if (tid == 0) oi[0] = kFallbackFlag;
      cand_spill(cs, crow, soff, row, nv);
    } else if constexpr (kFull) {
      if (nseg == 1) {  // block-uniform
        const int kp = k < 2 ? 2 : k;
        radix_row<false>(row, x, ld, n, k, row_len, 1, 1 << (32 - __builtin_clz(kp - 1)), out_idx, out_val, 0,
                         nullptr, lds);
      } else if (tid == 0) {
        oi[0] = kFallbackFlag;
      }
    } else if (tid == 0) {
      oi[0] = kFallbackFlag;
    }
  };
  static_assert((kHistBins + kRedWords) + 2 * kListCap <= kLdsRegWords,
                "the exact select fits the register path's LDS");

  // 1. Load: thread t holds positions 4*(t + c*1024) .. +3 of chunk c.  kFull:
  // the host has checked that every row is whole (4096 * kChunks scores) and
  // 16-byte aligned, so the loads are straight-line.
  float v[kChunks][4];
  const int g_full = nv >> 2;
  // The chunks the sample reads (every kSampleStep-th; with 8 chunks the even ones).
  constexpr int kSampleChunks = kChunks == 8 ? 4 : kChunks;
  constexpr int kSampleStep = kChunks / kSampleChunks;
  if constexpr (kCand) {
#pragma unroll
    for (int c = 0; c < kChunks; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int p = tid + kTopkThreads * (4 * c + j);
        v[c][j] = p < nv ? __uint_as_float(crow[cand_slot(soff, cs.cap, p)].x) : -__builtin_huge_valf();
      }
  } else if constexpr (kFull) {
    // With 8 chunks the even ones are loaded first: the sample below reads only
    // them, so it waits for half the loads and the rest arrive meanwhile.
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int c = kChunks == 8 ? 2 * (i & 3) + (i >> 2) : i;
      if (kChunks == 8 && i == 4) __builtin_amdgcn_sched_barrier(0);  // the even loads stay first
      const f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(xr) + tid + c * kTopkThreads);
      v[c][0] = t[0]; v[c][1] = t[1]; v[c][2] = t[2]; v[c][3] = t[3];
    }
  } else if constexpr (kAligned) {
    // Every row 16-byte aligned (checked on the host): whole groups of 4 with 16-byte
    // loads in the order above, unconditional -- a group past the row's last whole one
    // reads four absent scores from kTopkAbsent4 -- so that the sample's wait can be
    // counted; the one partial group at the end is filled in after the sample.
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int c = kChunks == 8 ? 2 * (i & 3) + (i >> 2) : i;
      if (kChunks == 8 && i == 4) __builtin_amdgcn_sched_barrier(0);
      const int g = tid + c * kTopkThreads;
      const f32x4* src =
          g < g_full ? reinterpret_cast<const f32x4*>(xr) + g : reinterpret_cast<const f32x4*>(kTopkAbsent4);
      const f32x4 t = __builtin_nontemporal_load(src);
      v[c][0] = t[0]; v[c][1] = t[1]; v[c][2] = t[2]; v[c][3] = t[3];
    }
  } else {
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const int e0 = 4 * (tid + c * kTopkThreads);
#pragma unroll
      for (int j = 0; j < 4; ++j) v[c][j] = (e0 + j < nv) ? xr[e0 + j] : -__builtin_huge_valf();
    }
  }
  // Sample histograms (both levels) start empty.
  reinterpret_cast<u32x2*>(shc)[tid] = u32x2{0u, 0u};
  if (tid == 0) red[kRedFlag] = 0;
  __syncthreads();

  // 2. Sample: wave w takes register (c, j) = (w % kChunks, (w / kChunks) % 4),
  // 64 positions 4 apart in each of 16 windows spread over the row; with 8
  // chunks only the even ones, (2 (w % 4), (w / 4) % 4), which still span the
  // row: each sample then stands for the same number of positions, the odd
  // chunk beside it taken to look alike.  (A separate, earlier sample load costs
  // more than it saves: the row loads fetched its lines from HBM a second time.)
  float s = v[0][0];
#pragma unroll
  for (int c = 0; c < kChunks; c += kSampleStep)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (wave % kSampleChunks == c / kSampleStep && (wave / kSampleChunks) % 4 == j) s = v[c][j];  // wave-uniform
  const uint32_t sk = float_key(s);
  const bool sp = sk > kKeyInvalidMax;  // present: > -1e30, not NaN
  if (sp) atomicAdd(&shc[sk >> 22], 1u);
  // Parked in LDS for the fine level: no register held across the retries.
  lds[kLdsSample + tid] = sp ? sk : 0u;
  const uint32_t wave_present = (uint32_t)__builtin_popcountll(__builtin_amdgcn_ballot_w64(sp));  // all lanes vote
  if (lane == 0) red[kRedPresent + wave] = wave_present;
  __syncthreads();
  const int s_present = (int)row0_sum(lane < kTopkWaves ? red[kRedPresent + lane] : 0u);
  if constexpr (kAligned) {  // the partial group left from the loads
    if (nv & 3) {
      const int g = g_full;  // its owner: thread g % 1024, chunk g / 1024
      if (tid == (g & (kTopkThreads - 1))) {
#pragma unroll
        for (int c = 0; c < kChunks; ++c)
          if (c == g / kTopkThreads) {
#pragma unroll
            for (int j = 0; j < 3; ++j)
              if (4 * g + j < nv) v[c][j] = xr[4 * g + j];
          }
      }
    }
  }

  // 3. Threshold and candidate compaction.  Sample rank r aims at
  // (k + kCandCap) / 2 candidates; r > s_present admits every present score.
  const float floor_t = __uint_as_float(kFloorBits);
  const int span = 4 * kTopkThreads * kChunks;  // positions the sample stands for
  int lo = 0, hi = s_present + 1;
  int r = (int)(((int64_t)((k + kCandCap) / 2) * kTopkThreads + span - 1) / span);
  r = min(max(r, 1), hi);
  const uint32_t e4 = kCand ? (uint32_t)tid : 4u * (uint32_t)tid;
  const uint32_t wreg = (uint32_t)wave * kWaveCap;
  uint32_t total = 0, held = 0;
  bool all_present = false, dense = false, handed = false;
  float t = floor_t;
  for (int tries = 0;; ++tries) {
    all_present = r > s_present;
    t = floor_t;
    if (!all_present) {  // block-uniform
      if (wave == 0) {
        if (tries > 0) reinterpret_cast<u32x4*>(shf)[lane] = u32x4{0u, 0u, 0u, 0u},
                       reinterpret_cast<u32x4*>(shf)[lane + 64] = u32x4{0u, 0u, 0u, 0u},
                       reinterpret_cast<u32x4*>(shf)[lane + 128] = u32x4{0u, 0u, 0u, 0u},
                       reinterpret_cast<u32x4*>(shf)[lane + 192] = u32x4{0u, 0u, 0u, 0u};
        uint32_t above;
        const int bc = rank_bin(shc, (uint32_t)r, above);
        if (lane == 0) { red[kRedCoarse] = (uint32_t)bc; red[kRedAbove] = above; }
      }
      __syncthreads();
      const uint32_t bc = red[kRedCoarse];
      const uint32_t skl = lds[kLdsSample + tid];  // 0 (absent) never matches: present keys sit in coarse bins >= 58
      if ((skl >> 22) == bc) atomicAdd(&shf[(skl >> 12) & (kSampleBins - 1)], 1u);
      __syncthreads();
      if (wave == 0) {
        uint32_t above2;
        const int bf = rank_bin(shf, (uint32_t)r - red[kRedAbove], above2);
        if (lane == 0) red[kRedThresh] = (bc << 22) | ((uint32_t)bf << 12);
      }
      __syncthreads();
      t = fmaxf(key_to_float(red[kRedThresh]), floor_t);
    }
    const uint32_t wcnt = compact_scores<kChunks, kCand>(v, t, wreg, e4, lv, lp);
    // cnt may hold an overrun's positions; clear it for the candidate histogram.
    reinterpret_cast<u32x4*>(cnt)[tid] = u32x4{0u, 0u, 0u, 0u};
    if (lane == 0) red[kRedCount + wave] = wcnt;
    held = min(wcnt, (uint32_t)kWaveCap);
    __syncthreads();
    const uint32_t fl = fresh_lane();
    const uint32_t cw = fl < kTopkWaves ? red[kRedCount + fl] : 0u;
    total = row0_sum(cw);
    const bool over = __builtin_amdgcn_ballot_w64(cw > (uint32_t)kWaveCap) != 0;
    const bool enough = all_present || total >= (uint32_t)k;
    if (!over && enough) break;  // block-uniform
    // Candidates crowded into some waves (sorted runs, say) but few enough in
    // all: compact them again, densely at per-wave prefix offsets.
    if (enough && total <= (uint32_t)kCandCap) {
      dense = true;
      break;
    }
    if (over) hi = r;
    else lo = r;
    if (hi - lo <= 1 || tries + 1 == kMaxTries) {  // block-uniform: nothing selected; handed over at the end
      handed = true;
      break;
    }
    r = (lo + hi + 1) / 2;
  }
  const int kk = handed ? 0 : all_present ? min((int)total, k) : k;
  if (dense) {  // block-uniform
    uint32_t cw = lane < kTopkWaves ? red[kRedCount + lane] : 0u;
    const uint32_t own = cw;
    cw += (uint32_t)DSA_DPP(0, cw, 0x111, 0xf);
    cw += (uint32_t)DSA_DPP(0, cw, 0x112, 0xf);
    cw += (uint32_t)DSA_DPP(0, cw, 0x114, 0xf);
    cw += (uint32_t)DSA_DPP(0, cw, 0x118, 0xf);
    const uint32_t start = (uint32_t)__builtin_amdgcn_readlane((int)(cw - own), wave);
    (void)compact_scores<kChunks, kCand>(v, t, start, e4, lv, lp);
    reinterpret_cast<u32x4*>(cnt)[tid] = u32x4{0u, 0u, 0u, 0u};  // the regions' overrun reached it
    __syncthreads();
  }

  // Each lane takes entries lane + 64 q of its wave's region (a wave's LDS
  // accesses stay in order), or, after a dense compaction, entries tid + 1024 q
  // of the whole list; and the block the candidates' key range.
  float ev[kLaneEntries];
  uint32_t ep[kLaneEntries];
  {
    uint32_t lmin = 0xffffffffu, lmax = 0u;
#pragma unroll
    for (int q = 0; q < kLaneEntries; ++q) {
      const uint32_t i = dense ? (uint32_t)(tid + kTopkThreads * q) : (uint32_t)(lane + kWave * q);
      const uint32_t a = dense ? min(i, (uint32_t)kCandCap - 1) : wreg + min(i, (uint32_t)kWaveCap - 1);
      ev[q] = __uint_as_float(lv[a]);
      ep[q] = lp[a];
      const uint32_t key = cand_key(ev[q]);
      if (i < (dense ? total : held)) { lmin = min(lmin, key); lmax = max(lmax, key); }
      else ev[q] = -__builtin_huge_valf();
    }
    lmax = wave_all_umax(lmax);
    lmin = ~wave_all_umax(~lmin);
    if (lane == 0) {
      red[kRedMin + wave] = lmin;
      red[kRedMax + wave] = lmax;
    }
  }
  __syncthreads();
  const bool wl = lane < kTopkWaves;
  const uint32_t kmin = ~row0_max(wl ? ~red[kRedMin + lane] : 0u);
  const uint32_t kmax = row0_max(wl ? red[kRedMax + lane] : 0u);

  if (kk > 0) {
    // 4. Bucket the candidates by binning position: bin = (pos - pos(min)) >> sh
    // < 4096.  The extreme candidates (keys kmin, kmax) carry the extreme
    // magnitudes, which fix the collapse floor of rows across zero.
    const float vlo = key_to_float(kmin), vhi = key_to_float(kmax);
    const uint32_t mhi = max(__float_as_uint(vlo) & 0x7fffffffu, __float_as_uint(vhi) & 0x7fffffffu);
    const bool across = vlo < 0.f && vhi > 0.f;
    const uint32_t floor_bits = across && (mhi >> 23) > kBinBinades ? ((mhi >> 23) - kBinBinades) << 23 : 0u;
    const uint32_t plo = cand_pos(vlo, floor_bits);
    const uint32_t range = cand_pos(vhi, floor_bits) - plo;
    const int sh = max(0, (range ? 32 - __builtin_clz(range) : 0) - kCandBinBits);
    uint32_t eb[kLaneEntries];
#pragma unroll
    for (int q = 0; q < kLaneEntries; ++q) {
      eb[q] = (cand_pos(ev[q], floor_bits) - plo) >> sh;
      if (ev[q] != -__builtin_huge_valf()) atomicAdd(&cnt[eb[q]], 1u);
      else eb[q] = 0xffffffffu;
    }
    __syncthreads();

    // 5. Descending scan: offs[b] = candidates in bins above b; b* holds the kk-th.
    {
      const u32x4 c4 = reinterpret_cast<const u32x4*>(cnt)[kCandBins / 4 - 1 - tid];  // bins 4095-4t .. 4092-4t
      uint32_t tot;
      const uint32_t excl = block_excl_scan<false>(c4.x + c4.y + c4.z + c4.w, red + kRedScan, tot);
      const uint32_t ow = excl, oz = ow + c4.w, oy = oz + c4.z, ox = oy + c4.y;
      reinterpret_cast<u32x4*>(offs)[kCandBins / 4 - 1 - tid] = u32x4{ox, oy, oz, ow};
      const uint32_t top = kCandBins - 1 - 4 * tid;
      const uint32_t ukk = (uint32_t)kk;
      if (ow < ukk && ox + c4.x >= ukk)
        red[kRedBstar] = oz >= ukk ? top : oy >= ukk ? top - 1 : ox >= ukk ? top - 2 : top - 3;
    }
    __syncthreads();
    const uint32_t bstar = red[kRedBstar];

    // 6. Regroup bins >= b* by bin (offs[b] then ends at the bin's end); the
    // position word carries the bin above its 15 position bits.
#pragma unroll
    for (int q = 0; q < kLaneEntries; ++q)
      if (eb[q] != 0xffffffffu && eb[q] >= bstar) {
        const uint32_t i = atomicAdd(&offs[eb[q]], 1u);
        lv[i] = __float_as_uint(ev[q]);
        lp[i] = (eb[q] << kPosBits) | ep[q];
      }
    __syncthreads();

    // 7. Rank inside the bin; sorted position = bin start + entries of the bin
    // that beat this one.  Entry p of the regrouped list lands within its bin's
    // range, so the stores stay nearly coalesced.
    const uint32_t list_n = offs[bstar];
    for (uint32_t p = (uint32_t)tid; p < list_n; p += kTopkThreads) {
      const float val = __uint_as_float(lv[p]);
      const uint32_t bp = lp[p];
      const uint32_t b = bp >> kPosBits;
      const uint32_t nb = cnt[b];
      const uint32_t start = offs[b] - nb;
      uint32_t rank = 0;
      if (nb > 1) {
        if (nb > (uint32_t)kBinCap) {
          red[kRedFlag] = 1;
          continue;
        }
        for (uint32_t j = start; j < start + nb; ++j) {
          const float u = __uint_as_float(lv[j]);
          rank += (u > val || (u == val && lp[j] < bp));  // same bin bits: compares positions
        }
      }
      const uint32_t fin = start + rank;
      if (fin < (uint32_t)kk) {
        const uint32_t pp = bp & ((1u << kPosBits) - 1);
        if constexpr (kCand) oi[fin] = (int32_t)crow[cand_slot(soff, cs.cap, (int)pp)].y;
        else oi[fin] = imap ? imap[pp] : base + (int)pp;
        if (ov) ov[fin] = val;
      }
    }
  }
  for (int i = kk + tid; i < k; i += kTopkThreads) {
    oi[i] = -1;
    if (ov) ov[i] = -__builtin_huge_valf();
  }
  if (kk > 0) {
    __syncthreads();
    handed = red[kRedFlag] != 0;  // block-uniform
  }
  if (handed) hand_over();  // the one call site: the exact select is inlined once
}

static int next_pow2(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

static int reg_chunks(int64_t seg_len) {
  return seg_len <= 4 * kTopkThreads ? 1 : seg_len <= 8 * kTopkThreads ? 2 : seg_len <= 16 * kTopkThreads ? 4 : 8;
}

// Every row (segment) starts 16-byte aligned: 16-byte loads.
static bool reg_aligned(const float* x, int64_t ld, int64_t seg_len) {
  return (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (ld & 3) == 0 && (seg_len & 3) == 0;
}

// Aligned and whole besides (no row lengths, 4096 * chunks scores a segment): no masks,
// and with one segment the rows it cannot bound are finished in place.
static bool reg_full(const float* x, int64_t ld, const int32_t* row_len, int64_t n, int nseg, int64_t seg_len) {
  return reg_aligned(x, ld, seg_len) && row_len == nullptr && seg_len == 4 * kTopkThreads * reg_chunks(seg_len) &&
         n == nseg * seg_len;
}

// Launch on `stream`: `rows` output rows (rows / nseg input rows of nseg segments of seg_len).
static hipError_t launch_reg(const float* x, int64_t ld, int64_t rows, int64_t n, int64_t k, const int32_t* row_len,
                             int32_t* out_idx, float* out_val, int nseg, int64_t seg_len, const int32_t* idx_map,
                             hipStream_t stream) {
  const dim3 grid((unsigned)rows), block(kTopkThreads);
  const int chunks = reg_chunks(seg_len);
  const bool aligned = reg_aligned(x, ld, seg_len);
  const bool full = reg_full(x, ld, row_len, n, nseg, seg_len);
#define DSA_REG(C, F, A)                                                                                               \
  hipLaunchKernelGGL((topk_reg_kernel<C, F, false, A>), grid, block, 0, stream, x, ld, (int)n, (int)k, row_len, \
                     out_idx, out_val, nseg, (int)seg_len, idx_map, CandSegments{})
#define DSA_REG2(C) \
  if (full) DSA_REG(C, true, false); else if (aligned) DSA_REG(C, false, true); else DSA_REG(C, false, false)
  if (chunks == 1) DSA_REG2(1);
  else if (chunks == 2) DSA_REG2(2);
  else if (chunks == 4) DSA_REG2(4);
  else DSA_REG2(8);
#undef DSA_REG2
#undef DSA_REG
  return hipGetLastError();
}

// Segments per row for the two-stage path (0: not used).  A segment holds at
// most kRegMax scores and at least k; the candidates (nseg * k) must fit the
// register path again.  Small row counts get more segments to fill the GPU,
// while a segment keeps at least 16 k scores: selecting a larger share of a
// segment costs more than the workgroups it adds (32 rows x 131072, k = 2048:
// 4 segments 26 us, 16 segments 34 us).
static int long_row_segments(int64_t rows, int64_t n, int64_t k) {
  if (n <= kRegMax || k > kListCap) return 0;
  int nseg = (int)((n + kRegMax - 1) / kRegMax);
  while (rows * nseg < 512 && (int64_t)(nseg * 2) * k <= kRegMax && (n + nseg * 2 - 1) / (nseg * 2) >= 16 * k)
    nseg *= 2;
  if ((int64_t)nseg * k > kRegMax) return 0;
  return nseg;
}

static int64_t segment_length(int64_t n, int nseg) {
  return ((n + nseg - 1) / nseg + 3) & ~int64_t(3);  // multiple of 4: segments stay 16-byte aligned
}

size_t topk_workspace_bytes(int64_t rows, int64_t n, int64_t k) {
  const int nseg = long_row_segments(rows, n, k);
  if (nseg == 0) return 0;
  return (size_t)rows * nseg * k * 8;  // candidate values + indices
}

// Launch on `stream`.  Caller has validated shapes (rows, n >= 0; 1 <= k <= 8192) and, when
// topk_workspace_bytes() is non-zero, passes a workspace of at least that size (else: nullptr,
// and long rows take the radix kernel alone).
static hipError_t launch_rows(const float* x, int64_t ld, int64_t rows, int64_t n, int64_t k,
                              const int32_t* row_len, int sorted, int32_t* out_idx, float* out_val,
                              int only_flagged, const int32_t* idx_map, hipStream_t stream,
                              const int32_t* gate = nullptr);

hipError_t launch_topk(const float* x, int64_t ld, int64_t rows, int64_t n, int64_t k,
                       const int32_t* row_len, int sorted, int32_t* out_idx, float* out_val,
                       void* workspace, hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  // Fast path for rows that fit in registers (directly, or in segments then
  // over the segments' candidates); the exact radix kernel then takes only the
  // rows the fast path flagged (its output is sorted either way).
  int only_flagged = 0;
  const int nseg = workspace ? long_row_segments(rows, n, k) : 0;
  if (n <= kRegMax && k <= kListCap) {
    hipError_t e = launch_reg(x, ld, rows, n, k, row_len, out_idx, out_val, 1, n, nullptr, stream);
    if (e != hipSuccess || reg_full(x, ld, row_len, n, 1, n)) return e;  // whole rows: finished in place
    only_flagged = 1;
    sorted = 1;
  } else if (nseg > 0) {
    float* cval = static_cast<float*>(workspace);
    int32_t* cidx = reinterpret_cast<int32_t*>(cval + (size_t)rows * nseg * k);
    hipError_t e = launch_reg(x, ld, rows * nseg, n, k, row_len, cidx, cval, nseg, segment_length(n, nseg), nullptr,
                              stream);
    if (e != hipSuccess) return e;
    e = launch_reg(cval, nseg * k, rows, nseg * k, k, nullptr, out_idx, out_val, 1, nseg * k, cidx, stream);
    if (e != hipSuccess) return e;
    only_flagged = 1;
    sorted = 1;
  }
  return launch_rows(x, ld, rows, n, k, row_len, sorted, out_idx, out_val, only_flagged, nullptr, stream);
}

// Top-k over the fused indexer's candidate rows (cs: 1 <= nseg <= kCandMaxSeg, ldc <= kRegMax):
// the register path reads the pairs in their key chunks; the exact radix kernel then takes the
// rows it could not bound, from the packed copies it left in cs.pval / cs.pidx.  Rows that go
// back to the dense path come out flagged in out_idx[row][0].
hipError_t launch_topk_candidates(const CandSegments& cs, int64_t rows, int64_t k, int32_t* out_idx,
                                  float* out_val, hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  if (cs.nseg < 1 || cs.nseg > kCandMaxSeg || cs.ldc > kRegMax || k > kListCap) return hipErrorInvalidValue;
  const int n = cs.ldc;
  const dim3 grid((unsigned)rows), block(kTopkThreads);
#define DSA_CAND(C)                                                                                             \
  hipLaunchKernelGGL((topk_reg_kernel<C, false, true>), grid, block, 0, stream, cs.pval, (int64_t)n, n, (int)k, \
                     nullptr, out_idx, out_val, 1, n, nullptr, cs)
  if (n <= 4 * kTopkThreads) DSA_CAND(1);
  else if (n <= 8 * kTopkThreads) DSA_CAND(2);
  else if (n <= 16 * kTopkThreads) DSA_CAND(4);
  else DSA_CAND(8);
#undef DSA_CAND
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_rows(cs.pval, cs.ldc, rows, cs.ldc, k, cs.plen, 1, out_idx, out_val, 1, cs.pidx, stream, cs.nspill);
}

// Every candidate row packed in key order into cs.pval / cs.pidx (one 256-thread
// workgroup per row), for k beyond the register top-k.  A row whose candidates
// cannot hold its top k -- a chunk overflowed, more kept keys than a packed row
// holds, or a finite threshold that fewer than k keys reached -- gets packed
// length -1 and out_idx[row][0] = kFallbackFlag: its dense logits decide.
__global__ __launch_bounds__(256) void cand_pack_kernel(const CandSegments cs, int k, int32_t* __restrict__ out_idx) {
  const int row = blockIdx.x;
  const u32x2* crow = cs.cand + (int64_t)row * cs.nseg * cs.cap;
  int soff[kCandMaxSeg];
  int tot = 0;
  bool over = false;
#pragma unroll
  for (int z = 0; z < kCandMaxSeg; ++z) {
    soff[z] = z < cs.nseg ? tot : (1 << 30);
    if (z < cs.nseg) {
      const int c = cs.count[(int64_t)row * cs.nseg + z];
      over |= c > cs.cap;
      tot += min(c, cs.cap);
    }
  }
  const bool back = over || tot > cs.ldc || (tot < k && cs.thr[row] != -__builtin_huge_valf());
  if (threadIdx.x == 0) {
    cs.plen[row] = back ? -1 : tot;
    if (back) {
      out_idx[(int64_t)row * k] = kFallbackFlag;
      if (cs.nback) atomicAdd(cs.nback, 1);
    }
  }
  if (back) return;  // block-uniform
  float* pv = cs.pval + (int64_t)row * cs.ldc;
  int32_t* pi = cs.pidx + (int64_t)row * cs.ldc;
  for (int p = threadIdx.x; p < tot; p += 256) {
    const u32x2 e = crow[cand_slot(soff, cs.cap, p)];
    pv[p] = __uint_as_float(e.x);
    pi[p] = (int32_t)e.y;
  }
}

// Top-k over the fused indexer's candidate rows for any k up to 8192: every row
// packed, then the exact radix kernel over the packed rows (positions map back
// through cs.pidx; packed position order is key order, which breaks the ties).
// Rows that go back to the dense path come out flagged in out_idx[row][0].
hipError_t launch_topk_packed(const CandSegments& cs, int64_t rows, int64_t k, int32_t* out_idx, float* out_val,
                              hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  if (cs.nseg < 1 || cs.nseg > kCandMaxSeg) return hipErrorInvalidValue;
  hipLaunchKernelGGL(cand_pack_kernel, dim3((unsigned)rows), dim3(256), 0, stream, cs, (int)k, out_idx);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_rows(cs.pval, cs.ldc, rows, cs.ldc, k, cs.plen, 1, out_idx, out_val, 0, cs.pidx, stream);
}

// The exact radix kernel for the rows whose out_idx[row][0] is kFallbackFlag (sorted output);
// gate (or null): a count of those rows, written by an earlier launch (zero: nothing to do).
hipError_t launch_topk_flagged(const float* x, int64_t ld, int64_t rows, int64_t n, int64_t k, int32_t* out_idx,
                               float* out_val, hipStream_t stream, const int32_t* gate) {
  if (rows == 0) return hipSuccess;
  return launch_rows(x, ld, rows, n, k, nullptr, 1, out_idx, out_val, 1, nullptr, stream, gate);
}

static hipError_t launch_rows(const float* x, int64_t ld, int64_t rows, int64_t n, int64_t k,
                              const int32_t* row_len, int sorted, int32_t* out_idx, float* out_val,
                              int only_flagged, const int32_t* idx_map, hipStream_t stream,
                              const int32_t* gate) {
  const int kpad = sorted ? next_pow2((int)(k < 2 ? 2 : k)) : 0;
  const size_t base = (size_t)(kHistBins + kRedWords) * 4 + (size_t)kpad * 8;
  const size_t cached = base + (size_t)n * 4;
  const bool use_cache = cached <= (size_t)(kLdsBytes - kRowsStaticLds);
  const size_t lds = use_cache ? cached : base;
  // Flagged rows only: one workgroup per CU (two without the LDS row cache) walks its share.
  const int64_t g = only_flagged ? std::min<int64_t>(rows, use_cache ? 256 : 512) : rows;
  const dim3 grid((unsigned)g), block(kTopkThreads);
  if (use_cache) {
    const hipError_t ea = set_dynamic_lds_once<topk_rows_kernel<true>>(kLdsBytes - kRowsStaticLds);
    if (ea != hipSuccess) return ea;
    hipLaunchKernelGGL(topk_rows_kernel<true>, grid, block, lds, stream, x, ld, (int)n, (int)k, row_len,
                       sorted, kpad, out_idx, out_val, only_flagged, idx_map, (int)rows, gate);
  } else {
    const hipError_t ea = set_dynamic_lds_once<topk_rows_kernel<false>>(kLdsBytes - kRowsStaticLds);
    if (ea != hipSuccess) return ea;
    hipLaunchKernelGGL(topk_rows_kernel<false>, grid, block, lds, stream, x, ld, (int)n, (int)k, row_len,
                       sorted, kpad, out_idx, out_val, only_flagged, idx_map, (int)rows, gate);
  }
  return hipGetLastError();
}

}  // namespace dsa
