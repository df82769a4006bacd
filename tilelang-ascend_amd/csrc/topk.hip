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
    int sorted, int kpad, int32_t* __restrict__ out_idx, float* __restrict__ out_val) {
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

static int next_pow2(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

// Launch on `stream`.  Caller has validated shapes (rows, n >= 0; 1 <= k <= 8192).
hipError_t launch_topk(const float* x, int64_t ld, int64_t rows, int64_t n, int64_t k,
                       const int32_t* row_len, int sorted, int32_t* out_idx, float* out_val,
                       hipStream_t stream) {
  if (rows == 0) return hipSuccess;
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
                       sorted, kpad, out_idx, out_val);
  } else {
    static bool attr = false;
    if (!attr) {
      (void)hipFuncSetAttribute((const void*)topk_rows_kernel<false>, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
      attr = true;
    }
    hipLaunchKernelGGL(topk_rows_kernel<false>, grid, block, lds, stream, x, ld, (int)n, (int)k, row_len,
                       sorted, kpad, out_idx, out_val);
  }
  return hipGetLastError();
}

}  // namespace dsa
