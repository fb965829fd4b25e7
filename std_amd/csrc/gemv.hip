// Weight-streaming projection for decode and verify rows: y[m][n] =
// sum_k x[m][k] * W[n][k] (+ b[n]) for M <= 16 rows, bf16 in, fp32
// accumulation, bf16 out (torch.nn.functional.linear of the decoder layers
// at batch 1). The bound is HBM: every weight byte is read once.
//
// A workgroup owns 16 output columns n; each of its waves walks one K range
// with v_mfma_f32_16x16x32_bf16: A = 16 weight rows x 32 k (lane (ln, lg)
// loads 16 contiguous bytes of row n0 + ln at k + 8 lg), B = the activation
// rows transposed (lane (ln, lg) loads x[ln][k + 8 lg .. +8], zero for
// ln >= M), so D[n][m] = sum_k W[n][k] x[m][k] lands as lane (ln, lg)
// element i = D[4 lg + i][ln]. The activations are a few KB and stay in L2.
// Splitting K over the workgroup's waves (rather than over workgroups with a
// second reduction launch) keeps one launch per projection and enough waves
// per CU to keep the weight stream in flight; the waves' partial tiles are
// added through LDS in wave order, so the result is deterministic.
#include "common.h"

namespace stdhip {
namespace {

constexpr int kUnroll = 8;                     // MFMAs (32 k each) per step
constexpr int kStepK = 32 * kUnroll;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ bf16x8_t ld16(const bf16_t* p) {
  return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(p));
}

// grid (ceil(N / 16)): a workgroup owns 16 output columns and its WK waves
// split K into WK contiguous ranges (multiples of 32); the waves' 16 x M fp32
// results are added in wave order through LDS by wave 0, which adds the bias
// and writes bf16. One launch, deterministic, no workspace.
template <int WK>
__global__ void __launch_bounds__(64 * WK)
gemv_bf16_kernel(const bf16_t* __restrict__ w, long long w_rs, const bf16_t* __restrict__ x, long long x_rs,
                 const bf16_t* __restrict__ bias, bf16_t* __restrict__ y, long long y_rs, int M, int N, int K) {
  __shared__ f32x4 red[WK][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int kw = (((K + WK - 1) / WK) + 31) / 32 * 32;        // this wave's K range
  const int k_begin = min(K, wave * kw), k_end = min(K, k_begin + kw);
  const bf16_t* wr = w + (long long)min(n0 + ln, N - 1) * w_rs + 8 * lg;
  const bool xm = ln < M;
  const bf16_t* xr = x + (long long)(xm ? ln : 0) * x_rs + 8 * lg;
  const bf16x8_t zero = {};
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  int k = k_begin;
  // Two steps of loads in flight: the next step's weights are requested
  // before the current step's MFMAs consume theirs.
  bf16x8_t a[kUnroll], b[kUnroll];
  auto load = [&](int kk, bf16x8_t* aa, bf16x8_t* bb) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      aa[u] = ld16(wr + kk + 32 * u);
      bb[u] = xm ? ld16(xr + kk + 32 * u) : zero;
    }
  };
  if (k + kStepK <= k_end) load(k, a, b);
  for (; k + kStepK <= k_end; k += kStepK) {
    bf16x8_t an[kUnroll], bn[kUnroll];
    const bool more = k + 2 * kStepK <= k_end;
    if (more) load(k + kStepK, an, bn);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[u], b[u], acc, 0, 0, 0);
    if (more) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) { a[u] = an[u]; b[u] = bn[u]; }
    }
  }
  for (; k < k_end; k += 32) {                 // K is a multiple of 32
    const bf16x8_t av = ld16(wr + k), bv = xm ? ld16(xr + k) : zero;
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc, 0, 0, 0);
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave != 0 || !xm) return;
  f32x4 t = red[0][lane];
#pragma unroll
  for (int i = 1; i < WK; ++i) t += red[i][lane];
  const int n = n0 + 4 * lg;                   // this lane's 4 columns of row m = ln
  bf16_t* dst = y + (long long)ln * y_rs + n;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (n + i < N) {
      const float v = bias ? t[i] + to_f32<bf16_t>(bias[n + i]) : t[i];
      dst[i] = from_f32<bf16_t>(v);
    }
}

}  // namespace
}  // namespace stdhip

using namespace stdhip;

extern "C" size_t std_gemv_workspace_bytes(int M, int N, int K) {
  (void)M;
  (void)N;
  (void)K;
  return 0;
}

extern "C" int std_gemv(const void* x, long long x_row_stride, const void* w, long long w_row_stride,
                        const void* bias, void* y, long long y_row_stride, int M, int N, int K, int dtype,
                        void* workspace, size_t workspace_bytes, void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  if (!x || !w || !y) return STD_E_NULL;
  if (dtype != STD_BF16) return STD_E_DTYPE;
  if (M < 1 || M > 16 || N < 1 || K < 32 || K % 32 != 0) return STD_E_SHAPE;
  if (x_row_stride < K || w_row_stride < K || y_row_stride < N) return STD_E_SHAPE;
  if (!aligned16(x) || !aligned16(w) || (x_row_stride * 2) % 16 || (w_row_stride * 2) % 16) return STD_E_ALIGN;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((N + 15) / 16);
  // K per wave: about 512-2400 k (eight waves once K is large)
  if (K > 4096)
    hipLaunchKernelGGL(gemv_bf16_kernel<8>, grid, dim3(512), 0, st, static_cast<const bf16_t*>(w), w_row_stride,
                       static_cast<const bf16_t*>(x), x_row_stride, static_cast<const bf16_t*>(bias),
                       static_cast<bf16_t*>(y), y_row_stride, M, N, K);
  else
    hipLaunchKernelGGL(gemv_bf16_kernel<4>, grid, dim3(256), 0, st, static_cast<const bf16_t*>(w), w_row_stride,
                       static_cast<const bf16_t*>(x), x_row_stride, static_cast<const bf16_t*>(bias),
                       static_cast<bf16_t*>(y), y_row_stride, M, N, K);
  return launch_status();
}
