// Per-row activation quantiser: the producer of the indexer's low-precision q / k.
//
//   amax  = max(max_j |x[r, j]|, 1e-4)
//   scale = amax / QMAX                       (round_scale: 2^ceil(log2(amax / QMAX)))
//   y     = cvt(clamp(x / scale, -QMAX, QMAX))
//
// QMAX = 127 with round-half-to-even to int8 (examples/deepseek_v4/act_quant.py:33-92 kernel,
// :118-142 golden), or 448 with round-to-nearest-even to OCP fp8 e4m3fn (the same recipe for
// the fp8 indexer inputs).  One wave per row: a pass for the absolute maximum (16-byte loads,
// a cross-lane max), then a pass that scales, converts and stores (the second read of the row
// hits L2).  HBM bound: (input bytes + 1) per element, plus 4 B of scale per row.
#include "common.hpp"

namespace dsa {

enum QuantIn : int { kQInBf16 = 1, kQInFp16 = 2, kQInFp32 = 3 };
enum QuantOut : int { kQOutFp8 = 0, kQOutInt8 = 4 };

template <int kIn>
struct QIn;
template <> struct QIn<kQInBf16> {
  typedef uint16_t T;
  static __device__ __forceinline__ float f(T v) { return __uint_as_float((uint32_t)v << 16); }
};
template <> struct QIn<kQInFp16> {
  typedef uint16_t T;
  static __device__ __forceinline__ float f(T v) { return (float)__builtin_bit_cast(_Float16, v); }
};
template <> struct QIn<kQInFp32> {
  typedef float T;
  static __device__ __forceinline__ float f(T v) { return v; }
};

// 2^ceil(log2(v)) for a positive normal v, from its bits (exponent + 1 unless the
// mantissa is zero): act_quant.py:96-109.
__device__ __forceinline__ float pow2_ceil(float v) {
  const uint32_t b = __float_as_uint(v);
  const int e = (int)((b >> 23) & 0xff) - 127 + ((b & 0x7fffff) ? 1 : 0);
  return __uint_as_float((uint32_t)(e + 127) << 23);
}

// One value to the output type: int8 after round-half-even, fp8 e4m3fn by the
// hardware conversion (round to nearest even; the input is already within +-448).
template <int kOut>
__device__ __forceinline__ uint8_t quant_one(float v) {
  if constexpr (kOut == kQOutInt8) {
    return (uint8_t)(int8_t)(int)__builtin_rintf(v);
  } else {
    return (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(v, 0.f, 0, false) & 0xff);
  }
}

template <int kIn, int kOut>
__global__ __launch_bounds__(256) void act_quant_kernel(const void* __restrict__ xv, int64_t rows, int n,
                                                        uint8_t* __restrict__ y, float* __restrict__ scales,
                                                        int round_scale) {
  typedef typename QIn<kIn>::T T;
  constexpr int kVec = 16 / sizeof(T);  // elements per 16-byte load
  constexpr float kQMax = kOut == kQOutInt8 ? 127.f : 448.f;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t r = (int64_t)blockIdx.x * (256 / kWave) + threadIdx.x / kWave;
  if (r >= rows) return;
  const T* x = static_cast<const T*>(xv) + r * n;
  uint8_t* yr = y + r * n;
  // 16-byte row loads (and 8- / 4-byte stores) when every row starts aligned.
  const bool vec = ((n * (int)sizeof(T)) & 15) == 0 && (reinterpret_cast<uintptr_t>(xv) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(y) & 7) == 0;
  const int nv = vec ? n / kVec : 0;  // whole 16-byte chunks

  float amax = 0.f;
  for (int c = lane; c < nv; c += kWave) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(x + (int64_t)c * kVec);
    const T* e = reinterpret_cast<const T*>(&w);
#pragma unroll
    for (int i = 0; i < kVec; ++i) amax = fmaxf(amax, fabsf(QIn<kIn>::f(e[i])));
  }
  for (int j = nv * kVec + lane; j < n; j += kWave) amax = fmaxf(amax, fabsf(QIn<kIn>::f(x[j])));
  amax = wave_max(amax);
  amax = fmaxf(amax, 1e-4f);
  float scale = amax / kQMax;
  if (round_scale) scale = pow2_ceil(scale);
  if (lane == 0) scales[r] = scale;

  for (int c = lane; c < nv; c += kWave) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(x + (int64_t)c * kVec);
    const T* e = reinterpret_cast<const T*>(&w);
    uint8_t q[kVec];
#pragma unroll
    for (int i = 0; i < kVec; ++i) q[i] = quant_one<kOut>(fminf(fmaxf(QIn<kIn>::f(e[i]) / scale, -kQMax), kQMax));
    if constexpr (kVec == 8) {
      *reinterpret_cast<uint2*>(yr + (int64_t)c * kVec) = *reinterpret_cast<const uint2*>(q);
    } else {
      *reinterpret_cast<uint32_t*>(yr + (int64_t)c * kVec) = *reinterpret_cast<const uint32_t*>(q);
    }
  }
  for (int j = nv * kVec + lane; j < n; j += kWave)
    yr[j] = quant_one<kOut>(fminf(fmaxf(QIn<kIn>::f(x[j]) / scale, -kQMax), kQMax));
}

template <int kIn>
static hipError_t launch_quant_in(int out_kind, const void* x, int64_t rows, int n, uint8_t* y, float* scales,
                                  int round_scale, hipStream_t stream) {
  const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  if (out_kind == kQOutInt8)
    hipLaunchKernelGGL((act_quant_kernel<kIn, kQOutInt8>), grid, block, 0, stream, x, rows, n, y, scales, round_scale);
  else
    hipLaunchKernelGGL((act_quant_kernel<kIn, kQOutFp8>), grid, block, 0, stream, x, rows, n, y, scales, round_scale);
  return hipGetLastError();
}

// Caller validated: in_kind in {bf16, fp16, fp32}, out_kind in {fp8, int8}, rows * n < 2^62, n < 2^31.
hipError_t launch_act_quant(int in_kind, const void* x, int64_t rows, int64_t n, int out_kind, void* y,
                            float* scales, int round_scale, hipStream_t stream) {
  if (rows == 0 || n == 0) return hipSuccess;
  uint8_t* yb = static_cast<uint8_t*>(y);
  switch (in_kind) {
    case kQInBf16: return launch_quant_in<kQInBf16>(out_kind, x, rows, (int)n, yb, scales, round_scale, stream);
    case kQInFp16: return launch_quant_in<kQInFp16>(out_kind, x, rows, (int)n, yb, scales, round_scale, stream);
    case kQInFp32: return launch_quant_in<kQInFp32>(out_kind, x, rows, (int)n, yb, scales, round_scale, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace dsa
