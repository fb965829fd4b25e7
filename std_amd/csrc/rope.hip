// Rotary position embedding fused with the K/V cache append, at a device
// length and a device position: the per-step glue of a decode step whose
// lengths and positions never leave the GPU (so the step can be captured in a
// HIP graph and replayed every round).
//
// The arithmetic is the rotate-half embedding of modeling_qwen2_5_vl.py:690-732
// with the decoder's tables (inv_freq in fp32, angle = float(pos) * inv_freq,
// cos/sin of the angle rounded to the model dtype), evaluated op by op in the
// order torch evaluates q * cos + rotate_half(q) * sin: each product and the
// sum are rounded to the model dtype, with no fused multiply-add.
#include "common.h"

namespace stdhip {
namespace {

constexpr int D = kHeadDim;
constexpr int HALF = D / 2;

template <typename T>
__device__ __forceinline__ float rnd(float x) { return to_f32<T>(from_f32<T>(x)); }

// grid (n_rows, n_q + n_kv), block HALF: thread j rotates the pair (j, j + 64)
// of one head of one row. Query heads go to q_out [n_q][n_rows][D]; key heads
// are rotated into the cache row len + row, and the matching value row is
// copied there. Rows at or past the capacity are not written; they mark the
// status word.
template <typename T>
__global__ void __launch_bounds__(HALF)
rope_append_kernel(const T* __restrict__ qkv, long long qkv_rs, T* __restrict__ q_out, T* __restrict__ ck,
                   T* __restrict__ cv, int n_rows, int n_q, int n_kv, long long chs, int capacity,
                   const int32_t* __restrict__ len_dev, const int32_t* __restrict__ pos_dev, int pos_offset,
                   const float* __restrict__ inv_freq, int32_t* status) {
  // Every product is rounded to the dtype before the sum, as torch evaluates
  // it: plain operators (round to nearest even) with multiply-add
  // contraction off -- for fp16 the compiler would otherwise fuse x * cos
  // into the add and drop that rounding.
#pragma clang fp contract(off)
  const int row = blockIdx.x, head = blockIdx.y, j = threadIdx.x;
  const int pos = *pos_dev + pos_offset + row;
  const float ang = (float)pos * inv_freq[j];
  const float c = rnd<T>(cosf(ang)), s = rnd<T>(sinf(ang));
  const T* src = qkv + (long long)row * qkv_rs + (long long)head * D;
  const float x1 = to_f32<T>(src[j]), x2 = to_f32<T>(src[j + HALF]);
  const float lo = rnd<T>(rnd<T>(x1 * c) + rnd<T>(-x2 * s));
  const float hi = rnd<T>(rnd<T>(x2 * c) + rnd<T>(x1 * s));
  if (head < n_q) {
    T* dst = q_out + ((long long)head * n_rows + row) * D;
    dst[j] = from_f32<T>(lo);
    dst[j + HALF] = from_f32<T>(hi);
    return;
  }
  const int g = head - n_q;
  const int crow = *len_dev + row;
  if (crow < 0 || crow >= capacity) {
    if (g == 0 && j == 0) flag_overflow(status);
    return;
  }
  T* kd = ck + (long long)g * chs + (long long)crow * D;
  kd[j] = from_f32<T>(lo);
  kd[j + HALF] = from_f32<T>(hi);
  const T* vs = src + (long long)n_kv * D;
  T* vd = cv + (long long)g * chs + (long long)crow * D;
  vd[j] = vs[j];
  vd[j + HALF] = vs[j + HALF];
}

}  // namespace
}  // namespace stdhip

using namespace stdhip;

extern "C" int std_rope_append(const void* qkv, long long qkv_row_stride, void* q_out, void* cache_k, void* cache_v,
                               int n_rows, int n_q, int n_kv, int d, long long cache_head_stride, int capacity,
                               const int32_t* len_dev, const int32_t* pos_dev, int pos_offset,
                               const float* inv_freq, int dtype, int32_t* status, void* stream) {
  if (!qkv || !q_out || !cache_k || !cache_v || !len_dev || !pos_dev || !inv_freq) return STD_E_NULL;
  if (dtype != STD_F32 && dtype != STD_BF16 && dtype != STD_F16) return STD_E_DTYPE;
  if (d != D || n_rows < 1 || n_rows > 65535 || n_q < 1 || n_kv < 1 || n_q % n_kv != 0 || capacity < 1)
    return STD_E_SHAPE;
  if (qkv_row_stride < (long long)(n_q + 2 * n_kv) * D) return STD_E_SHAPE;
  if (n_kv > 1 && cache_head_stride < (long long)capacity * D) return STD_E_SHAPE;
  const dim3 grid(n_rows, n_q + n_kv);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == STD_BF16)
    hipLaunchKernelGGL(rope_append_kernel<bf16_t>, grid, dim3(HALF), 0, st, static_cast<const bf16_t*>(qkv),
                       qkv_row_stride, static_cast<bf16_t*>(q_out), static_cast<bf16_t*>(cache_k),
                       static_cast<bf16_t*>(cache_v), n_rows, n_q, n_kv, cache_head_stride, capacity, len_dev, pos_dev,
                       pos_offset, inv_freq, status);
  else if (dtype == STD_F16)
    hipLaunchKernelGGL(rope_append_kernel<f16_t>, grid, dim3(HALF), 0, st, static_cast<const f16_t*>(qkv),
                       qkv_row_stride, static_cast<f16_t*>(q_out), static_cast<f16_t*>(cache_k),
                       static_cast<f16_t*>(cache_v), n_rows, n_q, n_kv, cache_head_stride, capacity, len_dev, pos_dev,
                       pos_offset, inv_freq, status);
  else
    hipLaunchKernelGGL(rope_append_kernel<float>, grid, dim3(HALF), 0, st, static_cast<const float*>(qkv),
                       qkv_row_stride, static_cast<float*>(q_out), static_cast<float*>(cache_k),
                       static_cast<float*>(cache_v), n_rows, n_q, n_kv, cache_head_stride, capacity, len_dev, pos_dev,
                       pos_offset, inv_freq, status);
  return launch_status();
}
