// Greedy acceptance with device-side rollback, KV append at a device length,
// and the library-level entry points (status strings, version).
#include <climits>

#include "common.h"

namespace stdhip {
namespace {

constexpr int D = kHeadDim;
constexpr int AM_THREADS = 256;
constexpr int AM_PER_THREAD = 8;
constexpr int AM_CHUNK = AM_THREADS * AM_PER_THREAD;  // vocab entries per block
constexpr int kMaxRows = 64;

// Order-preserving key of a logit: larger value -> larger key; -0 == +0; every
// NaN is above +inf so that, like torch.argmax, the first NaN is the argmax.
__device__ __forceinline__ uint32_t order_key(float v) {
  if (v != v) return 0xffffffffu;
  const uint32_t b = __float_as_uint(v == 0.f ? 0.f : v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ bool better(uint32_t k1, int i1, uint32_t k0, int i0) {
  return k1 > k0 || (k1 == k0 && i1 < i0);
}

// grid (n_blocks, q_rows): partial argmax of logits[row][b*AM_CHUNK ...).
template <typename T>
__global__ void __launch_bounds__(AM_THREADS)
argmax_partial_kernel(const T* __restrict__ logits, long long row_stride, int vocab, int n_blocks,
                      uint2* __restrict__ part) {
  const int b = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  const T* x = logits + (long long)row * row_stride;
  const int start = b * AM_CHUNK, end = min(vocab, start + AM_CHUNK);
  // All of a thread's loads are issued before the first compare (indices past
  // the chunk re-read its last entry and are skipped): one memory round trip.
  T v[AM_PER_THREAD];
#pragma unroll
  for (int j = 0; j < AM_PER_THREAD; ++j) v[j] = x[min(start + tid + j * AM_THREADS, end - 1)];
  uint32_t bk = 0;
  int bi = INT_MAX;
#pragma unroll
  for (int j = 0; j < AM_PER_THREAD; ++j) {
    const int e = start + tid + j * AM_THREADS;
    const uint32_t k = order_key(to_f32<T>(v[j]));
    if (e < end && better(k, e, bk, bi)) { bk = k; bi = e; }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t ok = __shfl_xor(bk, off);
    const int oi = __shfl_xor(bi, off);
    if (better(ok, oi, bk, bi)) { bk = ok; bi = oi; }
  }
  __shared__ uint2 wbest[AM_THREADS / 64];
  if ((tid & 63) == 0) wbest[tid >> 6] = make_uint2(bk, (uint32_t)bi);
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < AM_THREADS / 64; ++w)
      if (better(wbest[w].x, (int)wbest[w].y, bk, bi)) { bk = wbest[w].x; bi = (int)wbest[w].y; }
    part[(long long)row * n_blocks + b] = make_uint2(bk, (uint32_t)bi);
  }
}

// The best (key, index) of one row's block partials, in every lane of the
// calling wave: lane l takes partials l, l + 64, ..., kFinalBatch of them per
// memory round trip (indices past the row re-read its last partial and are
// skipped), then a shuffle reduction. better() is a strict total order, so
// the result does not depend on the reduction order.
constexpr int kFinalBatch = 4;

__device__ __forceinline__ void row_best(const uint2* __restrict__ p, int n_blocks, int lane, uint32_t& bk, int& bi) {
  for (int b0 = 0; b0 < n_blocks; b0 += 64 * kFinalBatch) {
    uint2 v[kFinalBatch];
#pragma unroll
    for (int j = 0; j < kFinalBatch; ++j) v[j] = p[min(b0 + lane + 64 * j, n_blocks - 1)];
#pragma unroll
    for (int j = 0; j < kFinalBatch; ++j)
      if (b0 + lane + 64 * j < n_blocks && better(v[j].x, (int)v[j].y, bk, bi)) { bk = v[j].x; bi = (int)v[j].y; }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t ok = __shfl_xor(bk, off);
    const int oi = __shfl_xor(bi, off);
    if (better(ok, oi, bk, bi)) { bk = ok; bi = oi; }
  }
}

// One block of kFinalThreads: wave w reduces rows w, w + kFinalWaves, ...
// (row_best), then thread 0 forms the greedy prefix, the bonus and the rollback.
constexpr int kFinalThreads = 256;
constexpr int kFinalWaves = kFinalThreads / 64;

__global__ void __launch_bounds__(kFinalThreads)
accept_final_kernel(const uint2* __restrict__ part, int n_blocks, int q_rows, const int32_t* __restrict__ draft,
                    int n_draft, int has_pending, const int32_t* __restrict__ dense_next, int32_t* __restrict__ out,
                    int32_t* __restrict__ lens, int n_lens) {
  __shared__ int pred[kMaxRows + 1];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int row = w; row < q_rows; row += kFinalWaves) {
    uint32_t bk = 0;
    int bi = INT_MAX;
    row_best(part + (long long)row * n_blocks, n_blocks, lane, bk, bi);
    if (lane == 0) pred[row + (has_pending ? 0 : 1)] = bi;
  }
  if (tid == 0 && !has_pending) pred[0] = *dense_next;
  __syncthreads();
  if (tid == 0) {
    int a = 0;
    while (a < n_draft && draft[a] == pred[a]) ++a;
    out[0] = a;
    out[1] = pred[a];
    for (int i = 0; i <= n_draft; ++i) out[2 + i] = pred[i];
    for (int i = 0; i < n_lens; ++i) lens[i] -= n_draft - a;
  }
}

// Final step of the row argmax: one wave per row reduces its block partials
// (row_best) and writes the index as int64 (the token-id type of torch).
__global__ void __launch_bounds__(64)
argmax_final_kernel(const uint2* __restrict__ part, int n_blocks, long long* __restrict__ out) {
  const int r = blockIdx.x, lane = threadIdx.x;
  uint32_t bk = 0;
  int bi = INT_MAX;
  row_best(part + (long long)r * n_blocks, n_blocks, lane, bk, bi);
  if (lane == 0) out[r] = bi;
}

// One block per row: out = weight * dtype(x * rsqrt(mean(x^2) + eps)), the
// RMSNorm of modeling_qwen2_5_vl.py:192-197 with the products rounded to the
// dtype as torch evaluates them; squares and their sum are fp32 (the sum in
// this kernel's lane/wave order). No global staging, so it is safe to
// capture in a HIP graph.
//
// The row statistic follows the order of the rms_* helpers. A row of up to
// kRmsMaxOneBatch elements (3584: 14 a thread) is read with every load of x
// and of the weights issued before the first add -- one memory round trip --
// and kept in registers for the scaling pass; wider rows are read
// kRmsBatch elements a thread at a time, twice.
template <typename T>
__global__ void __launch_bounds__(256)
rms_norm_kernel(const T* __restrict__ x, const T* __restrict__ w, T* __restrict__ out, int hidden, long long x_rs,
                long long o_rs, float eps) {
  __shared__ float red[4];
  const int r = blockIdx.x, tid = threadIdx.x;
  const T* xr = x + (long long)r * x_rs;
  T* orow = out + (long long)r * o_rs;
  T xv[kRmsBatch], wv[kRmsBatch];
  auto inv_rms = [&](float ss) {
    ss = rms_wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    return rms_inv(red, hidden, eps);
  };
  auto scale = [&](float inv, int i0) {
#pragma unroll
    for (int j = 0; j < kRmsBatch; ++j) {
      const int i = i0 + tid + 256 * j;
      if (i < hidden) orow[i] = rms_scale<T>(xv[j], wv[j], inv);
    }
  };
  if (hidden <= kRmsMaxOneBatch) {
    rms_load<T>(xr, xv, 0, hidden, tid);
    rms_load<T>(w, wv, 0, hidden, tid);
    scale(inv_rms(rms_add_squares<T>(0.f, xv, 0, hidden, tid)), 0);
  } else {
    float ss = 0.f;
    for (int i0 = 0; i0 < hidden; i0 += kRmsMaxOneBatch) {
      rms_load<T>(xr, xv, i0, hidden, tid);
      ss = rms_add_squares<T>(ss, xv, i0, hidden, tid);
    }
    const float inv = inv_rms(ss);
    for (int i0 = 0; i0 < hidden; i0 += kRmsMaxOneBatch) {
      rms_load<T>(xr, xv, i0, hidden, tid);
      rms_load<T>(w, wv, i0, hidden, tid);
      scale(inv, i0);
    }
  }
}

__global__ void __launch_bounds__(256)
kv_append_kernel(char* __restrict__ ck, char* __restrict__ cv, const char* __restrict__ nk,
                 const char* __restrict__ nv, int rows, int row_bytes, long long chs_bytes, long long nhs_bytes,
                 long long nrs_bytes, int capacity, const int32_t* __restrict__ len_dev, int32_t* status) {
  const int g = blockIdx.y, kv = blockIdx.z;
  const int cpr = row_bytes / 16;
  const int c = blockIdx.x * 256 + threadIdx.x;
  const int s = c / cpr, col = c - s * cpr;
  if (s >= rows) return;
  const int pos = *len_dev + s;
  if (pos < 0 || pos >= capacity) {                     // not written: marks the status word
    if (g == 0 && kv == 0 && col == 0) flag_overflow(status);
    return;
  }
  const char* src = (kv ? nv : nk) + g * nhs_bytes + s * nrs_bytes + col * 16;
  char* dst = (kv ? cv : ck) + g * chs_bytes + (long long)pos * row_bytes + col * 16;
  *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
}

__global__ void __launch_bounds__(256) len_add_kernel(int32_t* len, int n, int delta) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) len[i] += delta;
}

int accept_blocks(int vocab) { return (vocab + AM_CHUNK - 1) / AM_CHUNK; }

}  // namespace
}  // namespace stdhip

using namespace stdhip;

extern "C" const char* std_status_string(int status) {
  switch (status) {
    case STD_OK: return "success";
    case STD_E_NULL: return "a required pointer is NULL";
    case STD_E_DTYPE: return "unsupported dtype";
    case STD_E_SHAPE: return "unsupported or inconsistent sizes";
    case STD_E_WORKSPACE: return "workspace smaller than required";
    case STD_E_ALIGN: return "pointer or stride not 16-byte aligned";
    case STD_E_RANGE: return "length or index past the cache capacity";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}

extern "C" int std_version(void) { return 0x000100; }

extern "C" size_t std_greedy_accept_workspace_bytes(int q_rows, int vocab) {
  if (q_rows < 1 || vocab < 1) return 0;
  return round_up((size_t)q_rows * accept_blocks(vocab) * sizeof(uint2), 256);
}

extern "C" int std_greedy_accept(const void* logits, long long logits_row_stride, int q_rows, int vocab, int dtype,
                                 const int32_t* draft, int n_draft, int has_pending, const int32_t* dense_next,
                                 int32_t* out, int32_t* rollback_lens, int n_lens, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  if (!logits || !draft || !out || !workspace) return STD_E_NULL;
  if (!has_pending && !dense_next) return STD_E_NULL;
  if (n_lens > 0 && !rollback_lens) return STD_E_NULL;
  if (dtype != STD_F32 && dtype != STD_BF16 && dtype != STD_F16) return STD_E_DTYPE;
  if (vocab < 1 || n_draft < 1 || n_lens < 0 || q_rows != n_draft + (has_pending ? 1 : 0) || q_rows > kMaxRows)
    return STD_E_SHAPE;
  if (logits_row_stride < vocab) return STD_E_SHAPE;
  if (workspace_bytes < std_greedy_accept_workspace_bytes(q_rows, vocab)) return STD_E_WORKSPACE;
  const int nb = accept_blocks(vocab);
  uint2* part = static_cast<uint2*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == STD_BF16)
    hipLaunchKernelGGL(argmax_partial_kernel<bf16_t>, dim3(nb, q_rows), dim3(AM_THREADS), 0, st,
                       static_cast<const bf16_t*>(logits), logits_row_stride, vocab, nb, part);
  else if (dtype == STD_F16)
    hipLaunchKernelGGL(argmax_partial_kernel<f16_t>, dim3(nb, q_rows), dim3(AM_THREADS), 0, st,
                       static_cast<const f16_t*>(logits), logits_row_stride, vocab, nb, part);
  else
    hipLaunchKernelGGL(argmax_partial_kernel<float>, dim3(nb, q_rows), dim3(AM_THREADS), 0, st,
                       static_cast<const float*>(logits), logits_row_stride, vocab, nb, part);
  int s = launch_status();
  if (s) return s;
  hipLaunchKernelGGL(accept_final_kernel, dim3(1), dim3(kFinalThreads), 0, st, part, nb, q_rows, draft, n_draft,
                     has_pending ? 1 : 0, dense_next, out, rollback_lens, n_lens);
  return launch_status();
}

extern "C" int std_kv_append(void* cache_k, void* cache_v, const void* new_k, const void* new_v, int n_kv, int rows,
                             int d, long long cache_head_stride, long long new_head_stride, long long new_row_stride,
                             int capacity, const int32_t* len_dev, int dtype, int32_t* status, void* stream) {
  if (!cache_k || !cache_v || !new_k || !new_v || !len_dev) return STD_E_NULL;
  if (dtype != STD_F32 && dtype != STD_BF16 && dtype != STD_F16) return STD_E_DTYPE;
  if (d != D || n_kv < 1 || rows < 1 || capacity < 1) return STD_E_SHAPE;
  const int es = dtype_size(dtype);
  if (!aligned16(cache_k) || !aligned16(cache_v) || !aligned16(new_k) || !aligned16(new_v)) return STD_E_ALIGN;
  if ((cache_head_stride * es) % 16 || (new_head_stride * es) % 16 || (new_row_stride * es) % 16) return STD_E_ALIGN;
  const int row_bytes = D * es, cpr = row_bytes / 16;
  hipLaunchKernelGGL(kv_append_kernel, dim3((rows * cpr + 255) / 256, n_kv, 2), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<char*>(cache_k), static_cast<char*>(cache_v),
                     static_cast<const char*>(new_k), static_cast<const char*>(new_v), rows, row_bytes,
                     cache_head_stride * es, new_head_stride * es, new_row_stride * es, capacity, len_dev, status);
  return launch_status();
}

extern "C" int std_len_add(int32_t* len_dev, int n, int delta, void* stream) {
  if (!len_dev) return STD_E_NULL;
  if (n < 1) return STD_E_SHAPE;
  hipLaunchKernelGGL(len_add_kernel, dim3((n + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream), len_dev, n,
                     delta);
  return launch_status();
}

extern "C" int std_argmax_rows(const void* logits, long long logits_row_stride, int rows, int vocab, int dtype,
                               long long* out, void* workspace, size_t workspace_bytes, void* stream) {
  if (!logits || !out || !workspace) return STD_E_NULL;
  if (dtype != STD_F32 && dtype != STD_BF16 && dtype != STD_F16) return STD_E_DTYPE;
  if (rows < 1 || rows > 65535 || vocab < 1 || logits_row_stride < vocab) return STD_E_SHAPE;
  if (workspace_bytes < std_greedy_accept_workspace_bytes(rows, vocab)) return STD_E_WORKSPACE;
  const int nb = accept_blocks(vocab);
  uint2* part = static_cast<uint2*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == STD_BF16)
    hipLaunchKernelGGL(argmax_partial_kernel<bf16_t>, dim3(nb, rows), dim3(AM_THREADS), 0, st,
                       static_cast<const bf16_t*>(logits), logits_row_stride, vocab, nb, part);
  else if (dtype == STD_F16)
    hipLaunchKernelGGL(argmax_partial_kernel<f16_t>, dim3(nb, rows), dim3(AM_THREADS), 0, st,
                       static_cast<const f16_t*>(logits), logits_row_stride, vocab, nb, part);
  else
    hipLaunchKernelGGL(argmax_partial_kernel<float>, dim3(nb, rows), dim3(AM_THREADS), 0, st,
                       static_cast<const float*>(logits), logits_row_stride, vocab, nb, part);
  int s = launch_status();
  if (s) return s;
  hipLaunchKernelGGL(argmax_final_kernel, dim3(rows), dim3(64), 0, st, part, nb, out);
  return launch_status();
}

extern "C" int std_rms_norm(const void* x, long long x_row_stride, const void* weight, void* out,
                            long long out_row_stride, int rows, int hidden, float eps, int dtype, void* stream) {
  if (!x || !weight || !out) return STD_E_NULL;
  if (dtype != STD_F32 && dtype != STD_BF16 && dtype != STD_F16) return STD_E_DTYPE;
  if (rows < 1 || hidden < 1 || x_row_stride < hidden || out_row_stride < hidden) return STD_E_SHAPE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == STD_BF16)
    hipLaunchKernelGGL(rms_norm_kernel<bf16_t>, dim3(rows), dim3(256), 0, st, static_cast<const bf16_t*>(x),
                       static_cast<const bf16_t*>(weight), static_cast<bf16_t*>(out), hidden, x_row_stride,
                       out_row_stride, eps);
  else if (dtype == STD_F16)
    hipLaunchKernelGGL(rms_norm_kernel<f16_t>, dim3(rows), dim3(256), 0, st, static_cast<const f16_t*>(x),
                       static_cast<const f16_t*>(weight), static_cast<f16_t*>(out), hidden, x_row_stride,
                       out_row_stride, eps);
  else
    hipLaunchKernelGGL(rms_norm_kernel<float>, dim3(rows), dim3(256), 0, st, static_cast<const float*>(x),
                       static_cast<const float*>(weight), static_cast<float*>(out), hidden, x_row_stride,
                       out_row_stride, eps);
  return launch_status();
}
