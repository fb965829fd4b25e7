// Weight-streaming projection for decode and verify rows: y[m][n] =
// sum_k x[m][k] * W[n][k] (+ b[n]) for M <= 16 rows, bf16 in, fp32
// accumulation, bf16 out (torch.nn.functional.linear of the decoder layers
// at batch 1). The bound is HBM: every weight byte is read once.
//
// A wave owns 16 output columns n and walks its K range with
// v_mfma_f32_16x16x32_bf16: A = 16 weight rows x 32 k (lane (ln, lg) loads 16
// contiguous bytes of row n0 + ln at k + 8 lg), B = the activation rows
// transposed (lane (ln, lg) loads x[ln][k + 8 lg .. +8], zero for ln >= M),
// so D[n][m] = sum_k W[n][k] x[m][k] lands as lane (ln, lg) element i =
// D[4 lg + i][ln]. The activations are a few KB and stay in L2; no LDS. When
// there are too few column tiles to fill the chip, K is split over
// workgroups and a second kernel adds the fp32 partials in split order (so
// the result is deterministic and graph-replay safe).
#include "common.h"

namespace stdhip {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kUnroll = 8;                     // MFMAs (32 k each) per step
constexpr int kStepK = 32 * kUnroll;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ bf16x8_t ld16(const bf16_t* p) {
  return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(p));
}

// grid (ceil(N / (16 kWaves)), n_split). Split s covers k in
// [s * k_split, min(K, (s + 1) * k_split)); k_split is a multiple of kStepK.
__global__ void __launch_bounds__(kThreads)
gemv_bf16_kernel(const bf16_t* __restrict__ w, long long w_rs, const bf16_t* __restrict__ x, long long x_rs,
                 const bf16_t* __restrict__ bias, bf16_t* __restrict__ y, long long y_rs, float* __restrict__ part,
                 int M, int N, int K, int k_split) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  const int n0 = (blockIdx.x * kWaves + wave) * 16;
  if (n0 >= N) return;
  const int split = blockIdx.y, n_split = gridDim.y;
  const int k_begin = split * k_split, k_end = min(K, k_begin + k_split);
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
    const bf16x8_t a = ld16(wr + k), b = xm ? ld16(xr + k) : zero;
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  }
  if (!xm) return;
  const int n = n0 + 4 * lg;                   // this lane's 4 columns of row m = ln
  if (n_split == 1) {
    bf16_t* dst = y + (long long)ln * y_rs + n;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (n + i < N) {
        const float v = bias ? acc[i] + to_f32<bf16_t>(bias[n + i]) : acc[i];
        dst[i] = from_f32<bf16_t>(v);
      }
  } else {
    float* dst = part + ((long long)split * M + ln) * N + n;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (n + i < N) dst[i] = acc[i];
  }
}

// y[m][n] = bf16(sum over splits in order + bias), grid (ceil(M N / 256)).
__global__ void __launch_bounds__(256)
gemv_reduce_kernel(const float* __restrict__ part, int n_split, const bf16_t* __restrict__ bias,
                   bf16_t* __restrict__ y, long long y_rs, int M, int N) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long long)M * N) return;
  const int m = (int)(i / N), n = (int)(i - (long long)m * N);
  float s = 0.f;
  for (int sp = 0; sp < n_split; ++sp) s += part[((long long)sp * M + m) * N + n];
  if (bias) s += to_f32<bf16_t>(bias[n]);
  y[(long long)m * y_rs + n] = from_f32<bf16_t>(s);
}

struct GemvPlan {
  int n_split, k_split;
};

// One column tile per wave; K is split into pieces of at most 2048 (short
// waves balance over the CUs better than a few long ones) and further until
// about 1024 waves (four per SIMD) are resident, keeping at least 512 k per
// split. Measured on the 7B projection shapes at one row: 4.2-5.9 TB/s for
// the 136 MB-1.09 GB matrices, against 3.0-5.1 TB/s for a single split.
GemvPlan plan_gemv(int N, int K) {
  const int tiles = (N + 15) / 16;
  int n_split = (1024 + tiles - 1) / tiles;
  if (n_split < (K + 2047) / 2048) n_split = (K + 2047) / 2048;
  const int max_split = K / 512 > 0 ? K / 512 : 1;
  if (n_split > max_split) n_split = max_split;
  if (n_split < 1) n_split = 1;
  int k_split = (int)round_up((size_t)((K + n_split - 1) / n_split), kStepK);
  n_split = (K + k_split - 1) / k_split;
  return GemvPlan{n_split, k_split};
}

}  // namespace
}  // namespace stdhip

using namespace stdhip;

extern "C" size_t std_gemv_workspace_bytes(int M, int N, int K) {
  if (M < 1 || M > 16 || N < 1 || K < 32) return 0;
  const GemvPlan p = plan_gemv(N, K);
  return p.n_split > 1 ? round_up((size_t)p.n_split * M * N * sizeof(float), 256) : 0;
}

extern "C" int std_gemv(const void* x, long long x_row_stride, const void* w, long long w_row_stride,
                        const void* bias, void* y, long long y_row_stride, int M, int N, int K, int dtype,
                        void* workspace, size_t workspace_bytes, void* stream) {
  if (!x || !w || !y) return STD_E_NULL;
  if (dtype != STD_BF16) return STD_E_DTYPE;
  if (M < 1 || M > 16 || N < 1 || K < 32 || K % 32 != 0) return STD_E_SHAPE;
  if (x_row_stride < K || w_row_stride < K || y_row_stride < N) return STD_E_SHAPE;
  if (!aligned16(x) || !aligned16(w) || (x_row_stride * 2) % 16 || (w_row_stride * 2) % 16) return STD_E_ALIGN;
  const GemvPlan p = plan_gemv(N, K);
  const size_t need = std_gemv_workspace_bytes(M, N, K);
  if (need > 0 && (!workspace || workspace_bytes < need)) return STD_E_WORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int tiles = (N + 15) / 16;
  const dim3 grid((tiles + kWaves - 1) / kWaves, p.n_split);
  float* part = static_cast<float*>(workspace);
  hipLaunchKernelGGL(gemv_bf16_kernel, grid, dim3(kThreads), 0, st, static_cast<const bf16_t*>(w), w_row_stride,
                     static_cast<const bf16_t*>(x), x_row_stride, static_cast<const bf16_t*>(bias),
                     static_cast<bf16_t*>(y), y_row_stride, part, M, N, K, p.k_split);
  int s = launch_status();
  if (s || p.n_split == 1) return s;
  hipLaunchKernelGGL(gemv_reduce_kernel, dim3((unsigned)(((long long)M * N + 255) / 256)), dim3(256), 0, st, part,
                     p.n_split, static_cast<const bf16_t*>(bias), static_cast<bf16_t*>(y), y_row_stride, M, N);
  return launch_status();
}
