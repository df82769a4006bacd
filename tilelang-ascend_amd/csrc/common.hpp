// Shared device helpers for the DSA kernels (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

namespace dsa {

constexpr int kWave = 64;

// Devices a process may drive (per-device launch state is kept per index).
constexpr int kMaxDevices = 64;

// Raises Kernel's dynamic-LDS limit to `bytes` on the current device, once per
// device and thread-safely (std::call_once per device index); every later call
// returns the first call's result, so a failure keeps being reported.  The
// limit is a property of the kernel as loaded on one device.
template <auto Kernel>
hipError_t set_dynamic_lds_once(int bytes) {
  static std::once_flag once[kMaxDevices];
  static hipError_t result[kMaxDevices];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::call_once(once[dev], [&] {
    result[dev] = hipFuncSetAttribute(reinterpret_cast<const void*>(Kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  });
  return result[dev];
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Order-preserving map fp32 -> uint32: a > b  <=>  key(a) > key(b).
// -0.0 is folded onto +0.0 (they compare equal, so they must tie); every NaN
// maps to 0, below -inf.
__device__ __forceinline__ uint32_t float_key(float v) {
  if (v != v) return 0u;
  uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Inverse of float_key for keys of non-NaN values.
__device__ __forceinline__ float key_to_float(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

__host__ __device__ constexpr uint32_t float_key_host(uint32_t u) {
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Key of -1e30f: keys at or below it are "absent" (reported as index -1).
// -1e30f = 0xF149F2CA.
constexpr uint32_t kKeyInvalidMax = float_key_host(0xF149F2CAu);

// out_idx[row][0] marker of the top-k paths: the row needs the exact radix path.
constexpr int32_t kFallbackFlag = (int32_t)0x80000000;

// Candidate (value bits, key) pairs of the fused indexer, read where its filter
// pass left them: key chunk s of row r holds min(count[r * nseg + s], cap)
// pairs from cand[(r * nseg + s) * cap] on, in key order; the row's packed
// position p is entry p - (pairs in chunks below s) of the chunk s holding it.
// A row goes back to the dense path (out_idx[row][0] = kFallbackFlag,
// plen[row] = -1) when a chunk overflowed, when the chunks hold more than ldc
// pairs, or when thr[row] is finite and fewer than k pairs reached it; every
// other row gets plen[row] = its pair count.  pval / pidx (ldc per row) receive
// the packed pairs of the rows the register top-k hands to the radix kernel.
constexpr int kCandMaxSeg = 8;
struct CandSegments {
  const u32x2* cand;
  const int32_t* count;
  const float* thr;
  int nseg, cap, ldc;
  float* pval;
  int32_t* pidx;
  int32_t* plen;
  // Counters (zeroed by an earlier launch on the stream, or null): rows handed
  // to the radix kernel on their packed candidates, and rows sent back to their
  // dense logits.  The passes behind read them and skip their work at zero.
  int32_t* nspill;
  int32_t* nback;
};

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Inclusive prefix sum across the 64 lanes of a wave.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    uint32_t t = __shfl_up(v, o, kWave);
    if (lane >= o) v += t;
  }
  return v;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2 r;
  r.x = (__bf16)a;
  r.y = (__bf16)b;
  return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

}  // namespace dsa
