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
#include "common.hpp"

namespace dsa {

constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / kWave;
constexpr int kHistBins = 2048;
constexpr int kRedWords = 64;
constexpr int kLdsBytes = 160 * 1024;
constexpr int32_t kFallbackFlag = (int32_t)0x80000000;  // out_idx[row][0] marker: row needs the exact radix path

// Block-wide exclusive scan of one uint32 per thread; `total` receives the sum.
// Uses red[0..kTopkWaves) and ends with a barrier so red can be reused.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* red, uint32_t& total) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  uint32_t incl = wave_incl_scan(v);
  if (lane == kWave - 1) red[wave] = incl;
  __syncthreads();
  uint32_t before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kTopkWaves; ++w) {
    uint32_t s = red[w];
    before += (w < wave) ? s : 0u;
    tot += s;
  }
  __syncthreads();
  total = tot;
  return before + incl - v;
}

__device__ __forceinline__ float key_to_float(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

template <bool kCached>
__device__ __forceinline__ uint32_t load_key(const float* __restrict__ xr, const uint32_t* keys, int i) {
  if constexpr (kCached) return keys[i];
  return float_key(xr[i]);
}

template <bool kCached>
__global__ __launch_bounds__(kTopkThreads) void topk_rows_kernel(
    const float* __restrict__ x, int64_t ld, int n, int k, const int32_t* __restrict__ row_len,
    int sorted, int kpad, int32_t* __restrict__ out_idx, float* __restrict__ out_val, int only_flagged) {
  extern __shared__ __align__(16) uint32_t lds[];
  uint32_t* hist = lds;                                     // kHistBins
  uint32_t* red = hist + kHistBins;                         // kRedWords
  uint64_t* sbuf = reinterpret_cast<uint64_t*>(red + kRedWords);  // kpad (sorted only)
  uint32_t* keys = reinterpret_cast<uint32_t*>(sbuf + (sorted ? kpad : 0));

  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const float* __restrict__ xr = x + (int64_t)row * ld;
  int32_t* __restrict__ oi = out_idx + (int64_t)row * k;
  float* __restrict__ ov = out_val ? out_val + (int64_t)row * k : nullptr;
  // Second pass behind topk_reg_kernel: only the rows it handed over.
  if (only_flagged && oi[0] != kFallbackFlag) return;
  __syncthreads();  // every thread has read the flag before any overwrites it
  int nv = n;
  if (row_len) nv = min(max(row_len[row], 0), n);

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
          oi[pos] = idx;
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
      oi[i] = (int32_t)(~(uint32_t)c);
      if (ov) ov[i] = key_to_float((uint32_t)(c >> 32));
    }
  }
  for (int i = kk + tid; i < k; i += kTopkThreads) {
    oi[i] = -1;
    if (ov) ov[i] = -__builtin_huge_valf();
  }
}


// ----------------------------------------------------------------------------
// Register-resident fast path (rows of up to 4096 * kChunks scores).
//
// The row is loaded once into VGPRs (kChunks 16-byte loads per thread, all in
// flight together).  Present scores (> -1e30, not NaN) are bucketed into 2048
// bins linear in value between the row's min and max -- a monotone map, so
// every score in a higher bin is strictly larger -- which spreads the
// histogram atomics far better than key-bit radix digits do.  A descending
// scan finds the bin b* holding the k-th largest; every score in bins >= b*
// goes, as a (key << 32 | ~index) word, into an LDS list grouped by bin.  Each
// list entry then counts the entries of its own bin that beat it: bin offset
// + that rank is its final sorted position (value desc, index asc), exact
// with ties, and entries landing below k are written out directly.  Rows the
// fast path cannot bound (all-equal scores, a list over kListCap, a bin over
// kBinCap, non-finite range) are flagged in out_idx[row][0] for the exact
// radix kernel, launched right after on the same stream.
//
// Rows longer than the registers hold go through it twice.  Stage 1 runs one
// workgroup per segment of a row (nseg > 1): the segment's own top-k, with
// global indices, into a candidate buffer -- every element of the row's top-k
// is in its segment's top-k under the same order.  Stage 2 selects over the
// nseg*k candidates of each row, taking the tie-break index from idx_map (the
// candidates' original indices) and flagging the row if any of its segments
// was flagged, so that the radix kernel redoes it from the original row.
// ----------------------------------------------------------------------------
constexpr int kListCap = 4096;
constexpr int kBinCap = 512;
constexpr int kRegMax = 4 * kTopkThreads * 8;  // longest row the register path holds (32768)

template <int kChunks>
__global__ __launch_bounds__(kTopkThreads) void topk_reg_kernel(const float* __restrict__ x, int64_t ld, int n, int k,
                                                                const int32_t* __restrict__ row_len,
                                                                int32_t* __restrict__ out_idx,
                                                                float* __restrict__ out_val, int nseg, int seg_len,
                                                                const int32_t* __restrict__ idx_map) {
  __shared__ uint32_t cnt[kHistBins];
  __shared__ uint32_t offs[kHistBins];
  __shared__ uint32_t fill[kHistBins];
  __shared__ uint32_t red[kRedWords];
  __shared__ uint64_t list[kListCap];
  const int vrow = blockIdx.x;  // output row: segment vrow % nseg of input row vrow / nseg
  const int row = vrow / nseg;
  const int seg = vrow - row * nseg;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int base = seg * seg_len;  // index of this segment's first element
  const float* __restrict__ xr = x + (int64_t)row * ld + base;
  int32_t* __restrict__ oi = out_idx + (int64_t)vrow * k;
  float* __restrict__ ov = out_val ? out_val + (int64_t)vrow * k : nullptr;
  const int32_t* __restrict__ imap = idx_map ? idx_map + (int64_t)row * ld : nullptr;
  int nv = n;
  if (row_len) nv = min(max(row_len[row], 0), n);
  nv = min(max(nv - base, 0), seg_len);
  if (imap) {
    // Stage 2: a flagged segment (its first candidate index) sends the whole row to the exact path.
    bool flagged = false;
    for (int sg = 0; sg * k < n; ++sg) flagged |= imap[sg * k] == kFallbackFlag;
    if (flagged) {
      if (tid == 0) oi[0] = kFallbackFlag;
      return;  // block-uniform
    }
  }

  // 1. Load: thread t holds elements 4*(t + c*1024) .. +3 of chunk c.
  float v[kChunks][4];
  const bool vec = ((reinterpret_cast<uintptr_t>(xr) & 15) == 0);
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int e0 = 4 * (tid + c * kTopkThreads);
    if (vec && e0 + 3 < nv) {
      const f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(xr) + (tid + c * kTopkThreads));
      v[c][0] = t[0]; v[c][1] = t[1]; v[c][2] = t[2]; v[c][3] = t[3];
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) v[c][j] = (e0 + j < nv) ? xr[e0 + j] : -__builtin_huge_valf();
    }
  }
  for (int b = tid; b < kHistBins; b += kTopkThreads) { cnt[b] = 0; fill[b] = 0; }

  // 2. Count, min and max of the present scores.
  uint32_t present = 0;
  float vmin = __builtin_huge_valf(), vmax = -__builtin_huge_valf();
#pragma unroll
  for (int c = 0; c < kChunks; ++c)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool p = v[c][j] > -1e30f;  // false for NaN too
      present += p;
      if (p) { vmin = fminf(vmin, v[c][j]); vmax = fmaxf(vmax, v[c][j]); }
    }
  present = (uint32_t)wave_sum_i((int)present);
  vmin = -wave_max(-vmin);
  vmax = wave_max(vmax);
  if (lane == 0) {
    red[wave] = present;
    red[16 + wave] = __float_as_uint(vmin);
    red[32 + wave] = __float_as_uint(vmax);
  }
  __syncthreads();
  uint32_t m_total = 0;
  vmin = __builtin_huge_valf();
  vmax = -__builtin_huge_valf();
#pragma unroll
  for (int w = 0; w < kTopkWaves; ++w) {
    m_total += red[w];
    vmin = fminf(vmin, __uint_as_float(red[16 + w]));
    vmax = fmaxf(vmax, __uint_as_float(red[32 + w]));
  }
  const int kk = min((int)m_total, k);
  const float inv = 2048.f / (vmax - vmin);
  // Degenerate ranges go to the exact path (a single distinct value, or a
  // range whose width or inverse is not a normal finite number).
  if (kk > 0 && !(vmax > vmin && inv < 3.0e38f && inv > 0.f)) {
    if (tid == 0) oi[0] = kFallbackFlag;
    return;  // block-uniform
  }
  __syncthreads();

  // 3. Histogram of bin(v) = min(2047, (int)((v - vmin) * inv)).
  if (kk > 0) {
#pragma unroll
    for (int c = 0; c < kChunks; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (v[c][j] > -1e30f) atomicAdd(&cnt[min(kHistBins - 1, (int)((v[c][j] - vmin) * inv))], 1u);
  }
  __syncthreads();

  // 4. Descending scan: offs[b] = number of present scores in bins above b.
  const int bhi = kHistBins - 1 - 2 * tid, blo = bhi - 1;
  const uint32_t chi = cnt[bhi], clo = cnt[blo];
  uint32_t tot;
  const uint32_t excl = block_excl_scan(chi + clo, red, tot);
  offs[bhi] = excl;
  offs[blo] = excl + chi;
  if (excl < (uint32_t)kk && excl + chi + clo >= (uint32_t)kk) red[kTopkWaves] = (excl + chi >= (uint32_t)kk) ? bhi : blo;
  // Largest bin at or above b* bounds the rank work; find it after b* is known.
  __syncthreads();
  const int bstar = kk > 0 ? (int)red[kTopkWaves] : kHistBins;
  const uint32_t list_n = kk > 0 ? offs[bstar] + cnt[bstar] : 0;
  uint32_t bigbin = 0;
  if (bhi >= bstar) bigbin = max(bigbin, chi);
  if (blo >= bstar) bigbin = max(bigbin, clo);
  {
    uint32_t bm = bigbin;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) bm = max(bm, (uint32_t)__shfl_xor((int)bm, o, kWave));
    if (lane == 0) red[kTopkWaves + 1 + wave] = bm;
  }
  __syncthreads();
  uint32_t maxbin = 0;
#pragma unroll
  for (int w = 0; w < kTopkWaves; ++w) maxbin = max(maxbin, red[kTopkWaves + 1 + w]);
  if (kk > 0 && (list_n > (uint32_t)kListCap || maxbin > (uint32_t)kBinCap)) {
    if (tid == 0) oi[0] = kFallbackFlag;
    return;  // block-uniform
  }

  // 5. Scatter the bins >= b* into the list, grouped by bin.
  if (kk > 0) {
#pragma unroll
    for (int c = 0; c < kChunks; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float val = v[c][j];
        if (val > -1e30f) {
          const int b = min(kHistBins - 1, (int)((val - vmin) * inv));
          if (b >= bstar) {
            const uint32_t pos = offs[b] + atomicAdd(&fill[b], 1u);
            const int p = 4 * (tid + c * kTopkThreads) + j;
            const int idx = imap ? imap[p] : base + p;
            list[pos] = ((uint64_t)float_key(val) << 32) | (uint32_t)(~(uint32_t)idx);
          }
        }
      }
  }
  __syncthreads();

  // 6. Rank inside the bin; final position = bin offset + rank.
  for (uint32_t p = tid; p < list_n; p += kTopkThreads) {
    const uint64_t e = list[p];
    const float val = key_to_float((uint32_t)(e >> 32));
    const int b = min(kHistBins - 1, (int)((val - vmin) * inv));
    const uint32_t lo = offs[b], nb = cnt[b];
    uint32_t rank = 0;
    for (uint32_t j = 0; j < nb; ++j) rank += list[lo + j] > e;
    const uint32_t pos = lo + rank;
    if (pos < (uint32_t)kk) {
      oi[pos] = (int32_t)(~(uint32_t)e);
      if (ov) ov[pos] = val;
    }
  }
  for (int i = kk + tid; i < k; i += kTopkThreads) {
    oi[i] = -1;
    if (ov) ov[i] = -__builtin_huge_valf();
  }
}

static int next_pow2(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

// Launch on `stream`: `rows` output rows (rows / nseg input rows of nseg segments of seg_len).
static hipError_t launch_reg(const float* x, int64_t ld, int64_t rows, int64_t n, int64_t k, const int32_t* row_len,
                             int32_t* out_idx, float* out_val, int nseg, int64_t seg_len, const int32_t* idx_map,
                             hipStream_t stream) {
  const dim3 grid((unsigned)rows), block(kTopkThreads);
#define DSA_REG(C)                                                                                                \
  hipLaunchKernelGGL((topk_reg_kernel<C>), grid, block, 0, stream, x, ld, (int)n, (int)k, row_len, out_idx, out_val, \
                     nseg, (int)seg_len, idx_map)
  if (seg_len <= 4 * kTopkThreads) DSA_REG(1);
  else if (seg_len <= 8 * kTopkThreads) DSA_REG(2);
  else if (seg_len <= 16 * kTopkThreads) DSA_REG(4);
  else DSA_REG(8);
#undef DSA_REG
  return hipGetLastError();
}

// Segments per row for the two-stage path (0: not used).  A segment holds at
// most kRegMax scores and at least k; the candidates (nseg * k) must fit the
// register path again; small row counts get more segments to fill the GPU.
static int long_row_segments(int64_t rows, int64_t n, int64_t k) {
  if (n <= kRegMax || k > kListCap) return 0;
  int nseg = (int)((n + kRegMax - 1) / kRegMax);
  while (rows * nseg < 512 && (int64_t)(nseg * 2) * k <= kRegMax && (n + nseg * 2 - 1) / (nseg * 2) >= k) nseg *= 2;
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
    if (e != hipSuccess) return e;
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
  const int kpad = sorted ? next_pow2((int)(k < 2 ? 2 : k)) : 0;
  const size_t base = (size_t)(kHistBins + kRedWords) * 4 + (size_t)kpad * 8;
  const size_t cached = base + (size_t)n * 4;
  const bool use_cache = cached <= (size_t)kLdsBytes;
  const size_t lds = use_cache ? cached : base;
  const dim3 grid((unsigned)rows), block(kTopkThreads);
  if (use_cache) {
    static bool attr = false;
    if (!attr) {
      (void)hipFuncSetAttribute((const void*)topk_rows_kernel<true>, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
      attr = true;
    }
    hipLaunchKernelGGL(topk_rows_kernel<true>, grid, block, lds, stream, x, ld, (int)n, (int)k, row_len,
                       sorted, kpad, out_idx, out_val, only_flagged);
  } else {
    static bool attr = false;
    if (!attr) {
      (void)hipFuncSetAttribute((const void*)topk_rows_kernel<false>, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
      attr = true;
    }
    hipLaunchKernelGGL(topk_rows_kernel<false>, grid, block, lds, stream, x, ld, (int)n, (int)k, row_len,
                       sorted, kpad, out_idx, out_val, only_flagged);
  }
  return hipGetLastError();
}

}  // namespace dsa
