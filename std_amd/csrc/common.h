// Shared device helpers for the gfx950 kernels of libstdhip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "std_hip.h"

namespace stdhip {

constexpr int kHeadDim = 128;  // the only head_dim the kernels are built for

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef double f64x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

// bf16 is carried as its 16-bit pattern.
typedef uint16_t bf16_t;

__device__ __forceinline__ float bf16_to_f32(uint32_t bits) {
  return __uint_as_float(bits << 16);
}

// Round-to-nearest-even float -> bf16, quieting NaNs (same rounding as
// torch's float -> bfloat16 conversion). Both results are formed and one
// selected: a select, where an early return for NaN compiles to a branch
// that saves and restores the execution mask around each conversion.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t quiet = (u >> 16) | 0x40u;
  return (u & 0x7fffffffu) > 0x7f800000u ? quiet : rounded;
}

// fp16 is carried as the compiler's half type (its conversions from float
// round to nearest even, as torch's float -> float16 does).
typedef _Float16 f16_t;

template <typename T> __device__ __forceinline__ float to_f32(T x);
template <> __device__ __forceinline__ float to_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ float to_f32<bf16_t>(bf16_t x) { return bf16_to_f32(x); }
template <> __device__ __forceinline__ float to_f32<f16_t>(f16_t x) { return (float)x; }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) {
  return (bf16_t)f32_to_bf16(x);
}
template <> __device__ __forceinline__ f16_t from_f32<f16_t>(float x) { return (f16_t)x; }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// RMSNorm row statistic (modeling_qwen2_5_vl.py:192-197) in one fixed order,
// shared by the norm kernel and the projection that normalises its own input:
// over a block of 256 threads, thread t adds the squares of elements t,
// t + 256, t + 512, ... of the row in that order (fp32, each product and sum
// rounded), each wave adds its 64 partials by an xor butterfly, and the four
// wave sums combine as ((w0 + w1) + (w2 + w3)).
constexpr int kRmsBatch = 16;                  // elements a thread loads at once
constexpr int kRmsMaxOneBatch = 256 * kRmsBatch;

// This thread's kRmsBatch elements of a row of n from element i0; elements
// past the row re-read the last one and must not be used (a load under a
// condition would compile to a branch that waits for it before the next).
template <typename T>
__device__ __forceinline__ void rms_load(const T* __restrict__ src, T* dst, int i0, int n, int tid) {
#pragma unroll
  for (int j = 0; j < kRmsBatch; ++j) dst[j] = src[min(i0 + tid + 256 * j, n - 1)];
}

template <typename T>
__device__ __forceinline__ float rms_add_squares(float ss, const T* v, int i0, int n, int tid) {
#pragma unroll
  for (int j = 0; j < kRmsBatch; ++j)
    if (i0 + tid + 256 * j < n) {
      const float f = to_f32<T>(v[j]);
      ss = __fadd_rn(ss, __fmul_rn(f, f));
    }
  return ss;
}

__device__ __forceinline__ float rms_wave_sum(float ss) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
  return ss;
}

// 1 / sqrt(mean + eps) from the four wave sums.
__device__ __forceinline__ float rms_inv(const float* wave_sums, int n, float eps) {
  const float mean = ((wave_sums[0] + wave_sums[1]) + (wave_sums[2] + wave_sums[3])) * (1.0f / (float)n);
  return rsqrtf(__fadd_rn(mean, eps));
}

// dtype(weight * dtype(x * inv)), the normalised element as torch rounds it.
template <typename T>
__device__ __forceinline__ T rms_scale(T x, T weight, float inv) {
  const float n = to_f32<T>(from_f32<T>(__fmul_rn(to_f32<T>(x), inv)));
  return from_f32<T>(__fmul_rn(to_f32<T>(weight), n));
}

// Marks the device status word (optional) with a cache overflow; called by
// one thread per detection. A vector atomic, so concurrent markers need no
// ordering among themselves.
__device__ __forceinline__ void flag_overflow(int32_t* status) {
  if (status != nullptr) atomicOr(status, (int32_t)STD_STATUS_CACHE_OVERFLOW);
}

// Status of the most recent launch on this thread (0 or a positive hipError_t).
inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

inline size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

inline int dtype_size(int dtype) { return dtype == STD_F32 ? 4 : 2; }

}  // namespace stdhip
