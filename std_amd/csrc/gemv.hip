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
// added through LDS in wave order, so the result is deterministic. The
// epilogue can also add the decoder's residual or apply the MLP's
// silu(gate) * up, so those elementwise ops cost no launch of their own.
#include "common.h"
#include "lds_dma.h"

namespace stdhip {
namespace {

constexpr int kUnroll = 8;                     // MFMAs (32 k each) per step

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ bf16x8_t ld16(const bf16_t* p) {
  return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(p));
}

// grid (ceil(N / 16)): a workgroup owns 16 output columns and its WK waves
// split K into WK contiguous ranges (multiples of 32); the waves' 16 x M fp32
// results are added in wave order through LDS by wave 0, which runs the
// epilogue and writes bf16. One launch, deterministic, no workspace.
//
// GATED (the MLP's gate/up projection, W = [gate rows; up rows], N = the
// intermediate size): the workgroup accumulates gate row n and up row N + n
// side by side and writes act[m][n] = silu(g) * u with g, u the projections
// rounded to bf16 -- torch.nn.functional.silu(gate) * up on the bf16 output
// of the [2N, K] linear, each op rounded to bf16 -- so the activation needs
// no launch of its own. residual (may be NULL): y = residual + round(x W^T +
// bias), the decoder's residual add rounded as torch rounds it.
__device__ __forceinline__ float round_bf16(float v) { return to_f32<bf16_t>(from_f32<bf16_t>(v)); }

// The waves' 16 x M partial tiles are added in wave order through LDS by wave
// 0, which applies the epilogue (bias, the gated activation, the residual)
// and writes bf16 rows m < M.
template <int WK, bool GATED, int COLS>
__device__ __forceinline__ void gemv_finish(f32x4 (*red)[WK][64], const f32x4* acc, int wave, int lane, int n0,
                                            const bf16_t* __restrict__ bias, const bf16_t* __restrict__ residual,
                                            long long r_rs, bf16_t* __restrict__ y, long long y_rs, int M, int N) {
  constexpr int kMat = GATED ? 2 : 1;
  const int ln = lane & 15, lg = lane >> 4;
  const bool xm = ln < M;
#pragma unroll
  for (int j = 0; j < kMat; ++j) red[j][wave][lane] = acc[j];
  __syncthreads();
  if (wave != 0 || !xm || 4 * lg >= COLS) return;
  f32x4 t[kMat];
#pragma unroll
  for (int j = 0; j < kMat; ++j) {
    t[j] = red[j][0][lane];
#pragma unroll
    for (int i = 1; i < WK; ++i) t[j] += red[j][i][lane];
  }
  const int n = n0 + 4 * lg;                   // this lane's 4 columns of row m = ln
  bf16_t* dst = y + (long long)ln * y_rs + n;
  const bf16_t* res = residual ? residual + (long long)ln * r_rs + n : nullptr;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (n + i < N) {
      float v = round_bf16(bias ? t[0][i] + to_f32<bf16_t>(bias[n + i]) : t[0][i]);
      if constexpr (GATED) {
        const float u = round_bf16(bias ? t[kMat - 1][i] + to_f32<bf16_t>(bias[N + n + i]) : t[kMat - 1][i]);
        const float s = round_bf16(__fdiv_rn(v, __fadd_rn(1.0f, expf(-v))));   // silu(g) in fp32, rounded
        v = round_bf16(s * u);
      }
      if (res) v = __fadd_rn(to_f32<bf16_t>(res[i]), v);
      dst[i] = from_f32<bf16_t>(v);
    }
}


// Steps of loads kept in flight per wave by the streaming kernel: a ring of
// kRing register buffers, refilled kRing - 1 steps ahead of the MFMAs (3 steps
// = 24 KB per wave; 2 and 3 ring slots measured slower at one row).
constexpr int kRing = 4;

// Weight lanes of columns past N load column N - 1 (D[n][m] depends only on
// weight row n and activation row m, and columns n >= N are not written);
// activation lanes of rows m >= M load nothing and hold zeros.
template <int WK, bool GATED>
__global__ void __launch_bounds__(64 * WK)
gemv_bf16_kernel(const bf16_t* __restrict__ w, long long w_rs, const bf16_t* __restrict__ x, long long x_rs,
                 const bf16_t* __restrict__ bias, const bf16_t* __restrict__ residual, long long r_rs,
                 bf16_t* __restrict__ y, long long y_rs, int M, int N, int K) {
  constexpr int kMat = GATED ? 2 : 1;          // weight row sets streamed per step
  constexpr int kU = kUnroll / kMat;           // k-steps of 32 per step (8 loads of 16 B per lane either way)
  constexpr int kStep = 32 * kU;
  __shared__ f32x4 red[kMat][WK][64];
  const int lane = threadIdx.x & 63;
  // Wave-uniform, so the step loop below is scalar control flow.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ln = lane & 15, lg = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int kw = (((K + WK - 1) / WK) + 31) / 32 * 32;        // this wave's K range
  const int k_begin = min(K, wave * kw), k_end = min(K, k_begin + kw);
  const int nsteps = (k_end - k_begin) / kStep;
  const bf16_t* wr[kMat];
  wr[0] = w + (long long)min(n0 + ln, N - 1) * w_rs + k_begin + 8 * lg;
  if constexpr (GATED) wr[kMat - 1] = wr[0] + (long long)N * w_rs;
  const bool xm = ln < M;
  const bf16_t* xr = x + (long long)(xm ? ln : 0) * x_rs + k_begin + 8 * lg;
  f32x4 acc[kMat];
#pragma unroll
  for (int j = 0; j < kMat; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Ring slot r holds step t with t % kRing == r. The ring is indexed by
  // compile-time constants only (the step loop is unrolled by kRing), so no
  // register copy ever waits on a load that is still in flight. Every slot
  // load is issued whatever the step count -- steps past the last one re-read
  // the last step, which is still in cache -- so the number of weight loads
  // issued after any slot is fixed and each MFMA waits only for its own slot
  // (a skipped slot behind a scalar branch makes the compiler wait for all).
  bf16x8_t a[kRing][kMat][kU], b[kRing][kU];
  auto load = [&](int t, int r) {
    const int kk = min(t, nsteps - 1) * kStep;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
#pragma unroll
      for (int j = 0; j < kMat; ++j) a[r][j][u] = ld16(wr[j] + kk + 32 * u);
      b[r][u] = xm ? ld16(xr + kk + 32 * u) : bf16x8_t{};
    }
  };
  auto mma = [&](int r) {
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
      for (int j = 0; j < kMat; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[r][j][u], b[r][u], acc[j], 0, 0, 0);
  };
  if (nsteps > 0) {
#pragma unroll
    for (int r = 0; r < kRing - 1; ++r) load(r, r);
    int t = 0;
    for (; t + kRing <= nsteps; t += kRing) {
#pragma unroll
      for (int r = 0; r < kRing; ++r) {
        load(t + r + kRing - 1, (r + kRing - 1) % kRing);
        mma(r);
      }
    }
#pragma unroll
    for (int r = 0; r < kRing - 1; ++r)        // the last nsteps % kRing steps, already loaded
      if (t + r < nsteps) mma(r);
  }
  for (int k = nsteps * kStep; k < k_end - k_begin; k += 32) {   // K is a multiple of 32
    const bf16x8_t bv = xm ? ld16(xr + k) : bf16x8_t{};
#pragma unroll
    for (int j = 0; j < kMat; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ld16(wr[j] + k), bv, acc[j], 0, 0, 0);
  }
  gemv_finish<WK, GATED, 16>(red, acc, wave, lane, n0, bias, residual, r_rs, y, y_rs, M, N);
}

// Weight streaming through LDS for one activation row and large weights (the
// decode steps' gate/up, down and lm_head): each wave streams its K range of
// the workgroup's 16 (gated: 2 x 16) weight rows HBM -> LDS through a private
// ring of global_load_lds_dwordx4 with the non-temporal policy. The register
// kernels' 16-byte lanes fetch each 128-byte line of a row in two load
// instructions; a DMA instruction here moves whole lines of several rows, and
// the stream read once leaves the caches to the data read again. No wave
// waits for another until the epilogue: each issues, waits for and reads only
// its own stages. Where the register kernels run four waves (gate/up,
// lm_head) this kernel keeps their K split, MFMA order and epilogue and equals
// them bit for bit; where they run two (down: 224 column blocks), two waves
// per CU could not keep enough bytes in flight (33 us against 27.6 us even
// with seven 4 KiB stages each), so eight waves split K here instead.
// Measured at one row, graph-replayed on the 7B shapes: gate/up 50.7 -> 43.6
// us, down 27.6 -> 24.0 us, lm_head 179 -> 161 us (a plain 271 MB read
// through this kind of ring: 39.6-40.3 us).
//
// Stage: 16 rows x KS k (2 KS bytes per row) per weight row set; a DMA
// instruction covers 1 KiB = 64 / C rows of C 16-byte chunks (C = KS / 8); the
// chunk c of row r lives at chunk c ^ (r % C), so that the MFMA operand reads
// (row ln, chunk 4u + lg) spread over the banks. NSTG ring slots per wave keep
// NSTG - 1 stages in flight. The wave's slice of the activation row goes to
// LDS by DMA ahead of the first stages.
template <int WK> struct DmaCfg;
template <> struct DmaCfg<4> { static constexpr int KS = 64, NSTG = 4; };
template <> struct DmaCfg<8> { static constexpr int KS = 128, NSTG = 3; };

// The activation slices of the WK waves (dynamic LDS; the rings are static).
inline int gemv_dma_xs_bytes(int WK, int K) {
  const int kw = (((K + WK - 1) / WK) + 31) / 32 * 32;
  return WK * ((kw * 2 + 1023) / 1024) * 1024;
}

// The input RMSNorm in the launch (NORM, one row): rows up to kGemvNormMaxK
// elements, one load batch of rms_norm_kernel's 256-thread layout, whose
// 256 kRmsBatch elements the activation region then holds.
constexpr int kGemvNormMaxK = 3584;
constexpr int kNormXsBytes = 256 * kRmsBatch * 2;
inline int gemv_dma_lds_bytes(int WK, int K, bool norm) {
  const int b = gemv_dma_xs_bytes(WK, K);
  return norm && b < kNormXsBytes ? kNormXsBytes : b;
}

// s_waitcnt until at most n * PER vector-memory operations are outstanding
// (n < MAXN, a run-time count turned into the instruction's immediate).
template <int PER, int MAXN>
__device__ __forceinline__ void wait_vm_stages(int n) {
  if constexpr (MAXN > 0) {
    if (n >= MAXN - 1) {
      __builtin_amdgcn_s_waitcnt(waitcnt_vm((MAXN - 1) * PER));
      return;
    }
    wait_vm_stages<PER, MAXN - 1>(n);
  } else {
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  }
}

// NORM (one row, K <= kGemvNormMaxK): x is a decoder layer's hidden state
// before its RMSNorm (weight nw, epsilon eps), normalised in the launch as
// rms_norm_kernel normalises it, bit for bit. The x row and the norm weight
// come by DMA ahead of the first stages -- the x row's 1 KiB pieces into the
// ring slot each wave fills last (piece q in wave q % WK's), the norm weight
// into the activation region -- and the first four waves (rms_norm_kernel's
// 256-thread layout) form the statistic and write the normalised row whole
// to the activation region, element i at byte 2 i, from which each wave reads
// its K range. The barriers are bare (the stages stay in flight); both
// stagings are read before the first overwrite (the normalised row after the
// second barrier, the ring slot by the stage issued after the third).
template <int WK, bool GATED, bool NORM = false>
__global__ void __launch_bounds__(64 * WK)
gemv_dma_kernel(const bf16_t* __restrict__ w, long long w_rs, const bf16_t* __restrict__ x,
                const bf16_t* __restrict__ bias, const bf16_t* __restrict__ residual, long long r_rs,
                bf16_t* __restrict__ y, int N, int K, const bf16_t* __restrict__ nw = nullptr, float eps = 0.f) {
  constexpr int KS = DmaCfg<WK>::KS, NSTG = DmaCfg<WK>::NSTG;
  constexpr int C = KS / 8;                      // 16-byte chunks per row of a stage
  constexpr int RPI = 64 / C;                    // rows per DMA instruction
  constexpr int IPM = 16 / RPI;                  // DMA instructions per row set and stage
  constexpr int kMat = GATED ? 2 : 1;
  constexpr int kMatB = 16 * KS * 2;
  constexpr int kStageB = kMat * kMatB;
  constexpr int kPer = kMat * IPM;               // DMA instructions per stage
  constexpr int kRowPieces = (kGemvNormMaxK * 2 + 1023) / 1024;
  static_assert(!NORM || kStageB >= (kRowPieces + WK - 1) / WK * 1024, "the x row fits the last ring slots");
  static_assert(!NORM || (WK >= 4 && kGemvNormMaxK <= 256 * kRmsBatch), "four statistic waves, one batch");
  __shared__ __align__(16) char rings[WK * NSTG * kStageB];
  extern __shared__ __align__(16) char xs_all[];
  __shared__ f32x4 red[kMat][WK][64];
  // the norm's four wave sums, in the epilogue's exchange buffer (first used
  // after the loop): the gated launch takes exactly half a CU's 160 KiB of
  // LDS, and 16 bytes more would leave one workgroup a CU
  float* rms_red = reinterpret_cast<float*>(&red[0][0][0]);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ln = lane & 15, lg = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int kw = (((K + WK - 1) / WK) + 31) / 32 * 32;
  const int k_begin = min(K, wave * kw), k_end = min(K, k_begin + kw);
  const int nk = k_end - k_begin;               // a multiple of 32
  const int nst = (nk + KS - 1) / KS;
  const int xs_b = ((kw * 2 + 1023) / 1024) * 1024;
  char* ring = rings + wave * NSTG * kStageB;
  char* xs = NORM ? xs_all + k_begin * 2 : xs_all + wave * xs_b;
  // the ring slot filled last, where wave q % WK keeps x row piece q
  auto x_piece = [&](int q) { return rings + (q % WK) * NSTG * kStageB + (NSTG - 1) * kStageB + (q / WK) * 1024; };
  // DMA lane roles: instruction i of a row set covers rows RPI i + lane / C;
  // the lane's 16 bytes are physical chunk lane % C of that row, i.e. logical
  // chunk lc[i] = (lane % C) ^ (row % C) (k 8 lc .. 8 lc + 7 of the stage);
  // rows past N re-read row N - 1.
  int row_b[IPM], lc[IPM];
#pragma unroll
  for (int i = 0; i < IPM; ++i) {
    const int r = RPI * i + lane / C;
    lc[i] = (lane % C) ^ (r % C);
    row_b[i] = (min(n0 + r, N - 1) - n0) * (int)(w_rs * 2);
  }
  const char* wb = reinterpret_cast<const char*>(w + (long long)n0 * w_rs + k_begin);
  auto issue = [&](int s) {
    const uint32_t dst = lds_addr(ring + (s % NSTG) * kStageB);
#pragma unroll
    for (int j = 0; j < kMat; ++j)
#pragma unroll
      for (int i = 0; i < IPM; ++i) {
        // k positions past the wave's range re-read its last 8 k (never used)
        const int kk = min(s * KS + 8 * lc[i], nk - 8);
        lds_dma16_sbase<true>(wb + (long long)j * N * w_rs * 2, (uint32_t)(row_b[i] + kk * 2),
                              dst + j * kMatB + i * 1024);
      }
  };
  if constexpr (NORM) {
    // the x row and the norm weight, 1 KiB pieces spread over the waves
    const int np = (K * 2 + 1023) / 1024;
    for (int q = wave; q < 2 * np; q += WK) {
      const bool is_x = q < np;
      const int b = (is_x ? q : q - np) * 1024;
      lds_dma16_sbase<false>(is_x ? x : nw, (uint32_t)min(b + lane * 16, K * 2 - 16),
                             lds_addr(is_x ? x_piece(q) : xs_all + b));
    }
  } else if (nk > 0) {
    // the activation slice [k_begin, k_end) of row 0, in 1 KiB DMA pieces
    const char* xb = reinterpret_cast<const char*>(x + k_begin);
    for (int b = 0; b < xs_b; b += 1024)
      lds_dma16_sbase<false>(xb, (uint32_t)min(b + lane * 16, nk * 2 - 16), lds_addr(xs + b));
  }
  f32x4 acc[kMat];
#pragma unroll
  for (int j = 0; j < kMat; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int pre = min(NSTG - 1, nst);
  for (int s = 0; s < pre; ++s) issue(s);
  if constexpr (NORM) {
    wait_vm_stages<kPer, NSTG>(pre);            // this wave's pieces have landed, its stages may not
    wg_barrier();
    const bool stat = threadIdx.x < 256;        // wave-uniform
    bf16_t nx[kRmsBatch], ng[kRmsBatch];
    if (stat) {
      // element e = tid + 256 j: x piece j / 2, norm weight byte 2 e (elements
      // past K read what the regions hold there and are never used)
#pragma unroll
      for (int j = 0; j < kRmsBatch; ++j) {
        nx[j] = *reinterpret_cast<const bf16_t*>(x_piece(j >> 1) + ((j & 1) * 256 + threadIdx.x) * 2);
        ng[j] = *reinterpret_cast<const bf16_t*>(xs_all + (threadIdx.x + 256 * j) * 2);
      }
      const float ss = rms_wave_sum(rms_add_squares<bf16_t>(0.f, nx, 0, K, threadIdx.x));
      if (lane == 0) rms_red[wave] = ss;
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_lgkm0());
    wg_barrier();
    if (stat) {
      const float inv = rms_inv(rms_red, K, eps);
#pragma unroll
      for (int j = 0; j < kRmsBatch; ++j)
        *reinterpret_cast<bf16_t*>(xs_all + (threadIdx.x + 256 * j) * 2) = rms_scale<bf16_t>(nx[j], ng[j], inv);
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_lgkm0());
    wg_barrier();
  }
  for (int s = 0; s < nst; ++s) {
    // stages issued: 0 .. min(s + NSTG - 2, nst - 1); stage s must have landed
    wait_vm_stages<kPer, NSTG - 1>(min(NSTG - 2, nst - 1 - s));
    // slot (s + NSTG - 1) % NSTG last held stage s - 1, whose operands are in registers
    if (s + NSTG - 1 < nst) issue(s + NSTG - 1);
    const char* st = ring + (s % NSTG) * kStageB;
#pragma unroll
    for (int u = 0; u < KS / 32; ++u) {
      const int kk = s * KS + 32 * u;
      if (kk < nk) {
        const bf16x8_t b = ln == 0 ? *reinterpret_cast<const bf16x8_t*>(xs + (kk + 8 * lg) * 2) : bf16x8_t{};
#pragma unroll
        for (int j = 0; j < kMat; ++j) {
          const bf16x8_t a =
              *reinterpret_cast<const bf16x8_t*>(st + j * kMatB + ln * (KS * 2) + (((4 * u + lg) ^ (ln % C)) << 4));
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[j], 0, 0, 0);
        }
      }
    }
  }
  gemv_finish<WK, GATED, 16>(red, acc, wave, lane, n0, bias, residual, r_rs, y, 0, 1, N);
}

// Two to sixteen activation rows over a large weight (the ten-row verify
// step): gemv_dma_kernel's ring, with each stage carrying, beside the weight
// rows, a 16-row slab of the activation rows' same K range (rows past M
// re-read row M - 1 and meet zero MFMA operands). The rows fill the MFMA's
// 16 columns, so M costs no extra matrix work; the slab comes by DMA with the
// default cache policy (every workgroup reads it), the weight non-temporally.
// 64-k stages, three slots per wave (four for a plain projection at four
// waves); eight waves where gemv_waves would run two (o, down).
template <int WK, bool GATED>
struct DmaRowsCfg {
  static constexpr int KS = 64, NSTG = (GATED || WK == 8) ? 3 : 4;
};

template <int WK, bool GATED>
__global__ void __launch_bounds__(64 * WK)
gemv_dma_rows_kernel(const bf16_t* __restrict__ w, long long w_rs, const bf16_t* __restrict__ x, long long x_rs,
                     const bf16_t* __restrict__ bias, const bf16_t* __restrict__ residual, long long r_rs,
                     bf16_t* __restrict__ y, long long y_rs, int M, int N, int K) {
  constexpr int KS = DmaRowsCfg<WK, GATED>::KS, NSTG = DmaRowsCfg<WK, GATED>::NSTG;
  constexpr int C = KS / 8, RPI = 64 / C, IPM = 16 / RPI;
  constexpr int kMat = GATED ? 2 : 1;
  constexpr int kMatB = 16 * KS * 2;
  constexpr int kStageB = (kMat + 1) * kMatB;    // the weight row sets, then the activation slab
  constexpr int kPer = (kMat + 1) * IPM;         // DMA instructions per stage
  __shared__ __align__(16) char rings[WK * NSTG * kStageB];
  __shared__ f32x4 red[kMat][WK][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ln = lane & 15, lg = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int kw = (((K + WK - 1) / WK) + 31) / 32 * 32;
  const int k_begin = min(K, wave * kw), k_end = min(K, k_begin + kw);
  const int nk = k_end - k_begin;               // a multiple of 32
  const int nst = (nk + KS - 1) / KS;
  char* ring = rings + wave * NSTG * kStageB;
  // DMA lane roles as in gemv_dma_kernel: instruction i covers rows
  // RPI i + lane / C of a row set (weight rows past N re-read row N - 1,
  // activation rows past M row M - 1), logical chunk lc[i]
  int row_b[IPM], xrow_b[IPM], lc[IPM];
#pragma unroll
  for (int i = 0; i < IPM; ++i) {
    const int r = RPI * i + lane / C;
    lc[i] = (lane % C) ^ (r % C);
    row_b[i] = (min(n0 + r, N - 1) - n0) * (int)(w_rs * 2);
    xrow_b[i] = min(r, M - 1) * (int)(x_rs * 2);
  }
  const char* wb = reinterpret_cast<const char*>(w + (long long)n0 * w_rs + k_begin);
  const char* xb = reinterpret_cast<const char*>(x + k_begin);
  auto issue = [&](int s) {
    const uint32_t dst = lds_addr(ring + (s % NSTG) * kStageB);
#pragma unroll
    for (int i = 0; i < IPM; ++i) {
      const int kk = min(s * KS + 8 * lc[i], nk - 8);
#pragma unroll
      for (int j = 0; j < kMat; ++j)
        lds_dma16_sbase<true>(wb + (long long)j * N * w_rs * 2, (uint32_t)(row_b[i] + kk * 2),
                              dst + j * kMatB + i * 1024);
      lds_dma16_sbase<false>(xb, (uint32_t)(xrow_b[i] + kk * 2), dst + kMat * kMatB + i * 1024);
    }
  };
  f32x4 acc[kMat];
#pragma unroll
  for (int j = 0; j < kMat; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < NSTG - 1 && s < nst; ++s) issue(s);
  const bool xm = ln < M;
  for (int s = 0; s < nst; ++s) {
    wait_vm_stages<kPer, NSTG - 1>(min(NSTG - 2, nst - 1 - s));
    if (s + NSTG - 1 < nst) issue(s + NSTG - 1);
    const char* st = ring + (s % NSTG) * kStageB;
#pragma unroll
    for (int u = 0; u < KS / 32; ++u) {
      if (s * KS + 32 * u < nk) {
        const int off = ln * (KS * 2) + (((4 * u + lg) ^ (ln % C)) << 4);
        const bf16x8_t b = xm ? *reinterpret_cast<const bf16x8_t*>(st + kMat * kMatB + off) : bf16x8_t{};
#pragma unroll
        for (int j = 0; j < kMat; ++j) {
          const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(st + j * kMatB + off);
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[j], 0, 0, 0);
        }
      }
    }
  }
  gemv_finish<WK, GATED, 16>(red, acc, wave, lane, n0, bias, residual, r_rs, y, y_rs, M, N);
}

// The gated projection at more than four rows (the ten-row verify step): one
// wave per workgroup walks all of K, requesting the next step's loads before
// the current step's MFMAs and draining them after (the copy into the
// current step's registers waits for them). Measured 53.4 us at ten rows on
// the 7B gate/up against 57-65 us for the ring kernel at one to four waves.
__global__ void __launch_bounds__(64)
gemv_gated_rows_kernel(const bf16_t* __restrict__ w, long long w_rs, const bf16_t* __restrict__ x, long long x_rs,
                       const bf16_t* __restrict__ bias, const bf16_t* __restrict__ residual, long long r_rs,
                       bf16_t* __restrict__ y, long long y_rs, int M, int N, int K) {
  constexpr int kU = kUnroll / 2;
  constexpr int kStep = 32 * kU;
  __shared__ f32x4 red[2][1][64];
  const int lane = threadIdx.x;
  const int ln = lane & 15, lg = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const bf16_t* wr[2];
  wr[0] = w + (long long)min(n0 + ln, N - 1) * w_rs + 8 * lg;
  wr[1] = wr[0] + (long long)N * w_rs;
  const bool xm = ln < M;
  const bf16_t* xr = x + (long long)(xm ? ln : 0) * x_rs + 8 * lg;
  f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  bf16x8_t a[2][kU], b[kU];
  auto load = [&](int kk, bf16x8_t (*aa)[kU], bf16x8_t* bb) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
#pragma unroll
      for (int j = 0; j < 2; ++j) aa[j][u] = ld16(wr[j] + kk + 32 * u);
      bb[u] = xm ? ld16(xr + kk + 32 * u) : bf16x8_t{};
    }
  };
  int k = 0;
  if (k + kStep <= K) load(k, a, b);
  for (; k + kStep <= K; k += kStep) {
    bf16x8_t an[2][kU], bn[kU];
    const bool more = k + 2 * kStep <= K;
    if (more) load(k + kStep, an, bn);
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j][u], b[u], acc[j], 0, 0, 0);
    if (more) {
#pragma unroll
      for (int u = 0; u < kU; ++u) {
#pragma unroll
        for (int j = 0; j < 2; ++j) a[j][u] = an[j][u];
        b[u] = bn[u];
      }
    }
  }
  for (; k < K; k += 32) {                     // K is a multiple of 32
    const bf16x8_t bv = xm ? ld16(xr + k) : bf16x8_t{};
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ld16(wr[j] + k), bv, acc[j], 0, 0, 0);
  }
  gemv_finish<1, true, 16>(red, acc, 0, lane, n0, bias, residual, r_rs, y, y_rs, M, N);
}

// Short K ranges at up to kShortRows rows (the q/k/v and lm_head projections
// of a decode step): every wave issues all of its weight
// loads at once -- one memory round trip instead of a stream of dependent
// steps -- and stages its slice of the activation rows in LDS meanwhile
// (the wave reads back only what it wrote), then runs its MFMAs.
constexpr int kShortSteps = 32;     // MFMA steps of 32 k per wave (128 VGPRs of weights)
constexpr int kShortRows = 4;
constexpr int kShortMaxK = 4096;

template <int WK, bool GATED, int COLS>
__global__ void __launch_bounds__(64 * WK)
gemv_short_kernel(const bf16_t* __restrict__ w, long long w_rs, const bf16_t* __restrict__ x, long long x_rs,
                  const bf16_t* __restrict__ bias, const bf16_t* __restrict__ residual, long long r_rs,
                  bf16_t* __restrict__ y, long long y_rs, int M, int N, int K) {
  constexpr int kMat = GATED ? 2 : 1;
  constexpr int NS = kShortSteps / kMat;
  __shared__ f32x4 red[kMat][WK][64];
  __shared__ __align__(16) bf16_t xs[kShortRows * kShortMaxK];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  const int n0 = blockIdx.x * COLS;
  const bool aw = ln < COLS;            // lanes past COLS carry zero weight rows
  const int kw = (((K + WK - 1) / WK) + 31) / 32 * 32;
  const int k_begin = min(K, wave * kw), k_end = min(K, k_begin + kw);
  const int nsteps = (k_end - k_begin) / 32;   // <= NS (checked on the host)
  const bf16_t* wr[kMat];
  wr[0] = w + (long long)min(n0 + ln, N - 1) * w_rs + k_begin + 8 * lg;
  if constexpr (GATED) wr[kMat - 1] = wr[0] + (long long)N * w_rs;
  bf16x8_t a[kMat][NS];
#pragma unroll
  for (int u = 0; u < NS; ++u)
    if (u < nsteps)
#pragma unroll
      for (int j = 0; j < kMat; ++j) a[j][u] = aw ? ld16(wr[j] + 32 * u) : bf16x8_t{};
  const int cpr = (k_end - k_begin) / 8;       // 16-byte chunks per activation row
  for (int c = lane; c < M * cpr; c += 64) {
    const int m = c / cpr, kk = k_begin + (c - m * cpr) * 8;
    *reinterpret_cast<uint4*>(xs + m * K + kk) = *reinterpret_cast<const uint4*>(x + (long long)m * x_rs + kk);
  }
  const bool xm = ln < M;
  const bf16_t* xl = xs + (xm ? ln : 0) * K + k_begin + 8 * lg;
  const bf16x8_t zero = {};
  f32x4 acc[kMat];
#pragma unroll
  for (int j = 0; j < kMat; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < NS; ++u)
    if (u < nsteps) {
      const bf16x8_t bv = xm ? ld16(xl + 32 * u) : zero;
#pragma unroll
      for (int j = 0; j < kMat; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j][u], bv, acc[j], 0, 0, 0);
    }
  gemv_finish<WK, GATED, COLS>(red, acc, wave, lane, n0, bias, residual, r_rs, y, y_rs, M, N);
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

namespace stdhip {
namespace {

// The fused q|k|v projection of up to kShortRows decode rows followed by the
// rotary embedding and the K/V cache append of rope.hip (one launch instead of
// two). The rotary embedding pairs columns j and j + 64 of a head, so a
// workgroup owns four pairs of one head -- output columns p..p+3 and
// p+64..p+67, p = 4 (block % 16), head = block / 16 -- and lanes lg = 0 and 1
// hold the two halves of the same pairs (exchanged with a lane shuffle). The
// projection itself is gemv_short_kernel's with eight columns: four waves split
// K, every weight load of a wave issued at once, the activation slice staged in
// LDS. The epilogue repeats rope_append_kernel's arithmetic op for op: the
// projection rounded to bf16 (bias added first), angle = float(pos) *
// inv_freq[j], cos / sin rounded to bf16, lo = x1 c - x2 s and hi = x2 c + x1 s
// with each product and the sum rounded. Query heads go to q_out
// [n_q][M][128]; key heads, rotated, and value heads, as projected, go to cache
// row len + m of their KV head (rows at or past the capacity are not written;
// they mark the status word).
//
// NORM (one row, K <= kQkvNormMaxK): x is the layer's input before its
// RMSNorm (weight nw): the workgroup forms the row statistic in the order of
// the rms_* helpers and writes the normalised row -- rms_norm_kernel's output
// bit for bit -- to LDS, where the MFMAs read it. The weight registers are
// sized to kQkvNormMaxK / 4 / 32 steps so the kernel keeps three workgroups a CU
// (all of a 7B q/k/v launch in one wave of workgroups).
constexpr int kQkvNormMaxK = 3584;

struct RopeArgs {
  bf16_t* q_out;
  bf16_t* ck;
  bf16_t* cv;
  long long chs;                  // cache head stride (elements)
  int n_q, n_kv, capacity, pos_offset;
  int32_t* status;                // optional device status word (cache overflow)
};

// Where columns p..p+3 of half `half` (half 0: columns p.., half 1: p + 64..)
// of head `head`, row m of M, go: query heads to q_out [n_q][M][128]; key and
// value heads to cache row len + m of their KV head (len: the cache length).
// nullptr for a cache row at or past the capacity (not written; it marks the
// status word).
__device__ __forceinline__ bf16_t* qkv_dest(int head, int half, int p, int m, int M, const RopeArgs& ra, int len) {
  const int kv_head = head - ra.n_q;
  bf16_t* dst;
  if (head < ra.n_q) {
    dst = ra.q_out + ((long long)head * M + m) * kHeadDim;
  } else {
    const int crow = len + m;
    if (crow < 0 || crow >= ra.capacity) {
      flag_overflow(ra.status);
      return nullptr;
    }
    dst = (kv_head < ra.n_kv ? ra.ck + (long long)kv_head * ra.chs : ra.cv + (long long)(kv_head - ra.n_kv) * ra.chs) +
          (long long)crow * kHeadDim;
  }
  return dst + half * (kHeadDim / 2) + p;
}

// rope_append_kernel's rotation factors at position pos and frequency freq:
// angle = float(pos) * freq, cos and sin each rounded to bf16.
__device__ __forceinline__ float2 rope_factors(int pos, float freq) {
  const float ang = __fmul_rn((float)pos, freq);
  return make_float2(round_bf16(cosf(ang)), round_bf16(sinf(ang)));
}

// The rotated element of half `half` of the pair (x1, x2) (the first and the
// second half's column), each product and the sum rounded to bf16:
// lo = x1 c - x2 s, hi = x2 c + x1 s.
__device__ __forceinline__ float rope_rotate(float x1, float x2, float2 f, int half) {
  return half ? round_bf16(__fadd_rn(round_bf16(__fmul_rn(x2, f.x)), round_bf16(__fmul_rn(x1, f.y))))
              : round_bf16(__fadd_rn(round_bf16(__fmul_rn(x1, f.x)), round_bf16(__fmul_rn(-x2, f.y))));
}

// The register kernel's epilogue: v holds columns p..p+3 of half `half` of
// row m (bias added, rounded to bf16), partner the same columns of the other
// half; query and key heads are rotated, value heads stored as projected.
__device__ __forceinline__ void qkv_rope_store(const float* v, const float* partner, int head, int half, int p, int m,
                                               int M, const RopeArgs& ra, const int32_t* __restrict__ len_dev,
                                               const int32_t* __restrict__ pos_dev,
                                               const float* __restrict__ inv_freq) {
  bf16_t* dst = qkv_dest(head, half, p, m, M, ra, *len_dev);
  if (!dst) return;
  if (head - ra.n_q >= ra.n_kv) {              // value heads: the projection as is
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = from_f32<bf16_t>(v[i]);
    return;
  }
  const int pos = *pos_dev + ra.pos_offset + m;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    dst[i] = from_f32<bf16_t>(rope_rotate(half ? partner[i] : v[i], half ? v[i] : partner[i],
                                          rope_factors(pos, inv_freq[p + i]), half));
}

template <bool NORM>
__global__ void __launch_bounds__(256, 3)    // three waves a SIMD: a 7B q/k/v launch in one wave of workgroups
gemv_qkv_rope_kernel(const bf16_t* __restrict__ w, long long w_rs, const bf16_t* __restrict__ x, long long x_rs,
                     const bf16_t* __restrict__ bias, int M, int K, RopeArgs ra, const int32_t* __restrict__ len_dev,
                     const int32_t* __restrict__ pos_dev, const float* __restrict__ inv_freq,
                     const bf16_t* __restrict__ nw, float eps) {
  constexpr int WK = 4, NS = NORM ? kQkvNormMaxK / 4 / 32 : kShortSteps, HALF = kHeadDim / 2;
  static_assert(kQkvNormMaxK <= kRmsMaxOneBatch && kQkvNormMaxK % 128 == 0, "one load batch, whole steps");
  __shared__ f32x4 red[WK][64];
  __shared__ __align__(16) bf16_t xs[kShortRows * kShortMaxK];
  __shared__ float rms_red[4];
  bf16_t nx[NORM ? kRmsBatch : 1], ng[NORM ? kRmsBatch : 1];
  if constexpr (NORM) {                        // issued first: the statistic's wait leaves the weights in flight
    rms_load<bf16_t>(x, nx, 0, K, threadIdx.x);
    rms_load<bf16_t>(nw, ng, 0, K, threadIdx.x);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  const int head = blockIdx.x / 16, p = (blockIdx.x % 16) * 4;
  const bool aw = ln < 8;                      // lanes past eight carry zero weight rows
  const int kw = (((K + WK - 1) / WK) + 31) / 32 * 32;
  const int k_begin = min(K, wave * kw), k_end = min(K, k_begin + kw);
  const int nsteps = (k_end - k_begin) / 32;   // <= NS (checked on the host)
  // weight row of lane ln: pair p + (ln & 3), first (ln < 4) or second half
  const bf16_t* wr = w + (long long)(head * kHeadDim + (ln >> 2 & 1) * HALF + p + (ln & 3)) * w_rs + k_begin + 8 * lg;
  bf16x8_t a[NS];
#pragma unroll
  for (int u = 0; u < NS; ++u)
    if (u < nsteps) a[u] = aw ? ld16(wr + 32 * u) : bf16x8_t{};
  if constexpr (NORM) {
    const float ss = rms_wave_sum(rms_add_squares<bf16_t>(0.f, nx, 0, K, threadIdx.x));
    if (lane == 0) rms_red[wave] = ss;
    __syncthreads();
    const float inv = rms_inv(rms_red, K, eps);
#pragma unroll
    for (int j = 0; j < kRmsBatch; ++j) {
      const int i = threadIdx.x + 256 * j;
      if (i < K) xs[i] = rms_scale<bf16_t>(nx[j], ng[j], inv);
    }
    __syncthreads();
  } else {
    const int cpr = (k_end - k_begin) / 8;     // 16-byte chunks per activation row
    for (int c = lane; c < M * cpr; c += 64) {
      const int m = c / cpr, kk = k_begin + (c - m * cpr) * 8;
      *reinterpret_cast<uint4*>(xs + m * K + kk) = *reinterpret_cast<const uint4*>(x + (long long)m * x_rs + kk);
    }
  }
  const bool xm = ln < M;
  const bf16_t* xl = xs + (xm ? ln : 0) * K + k_begin + 8 * lg;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < NS; ++u)
    if (u < nsteps) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[u], xm ? ld16(xl + 32 * u) : bf16x8_t{}, acc, 0, 0, 0);
  red[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  f32x4 t = red[0][lane];
#pragma unroll
  for (int i = 1; i < WK; ++i) t += red[i][lane];
  // lane (ln, lg < 2): row m = ln, pairs p + i, half lg
  const int half = lg & 1;
  const int col = head * kHeadDim + half * HALF + p;
  float v[4], partner[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = round_bf16(bias ? t[i] + to_f32<bf16_t>(bias[col + i]) : t[i]);
#pragma unroll
  for (int i = 0; i < 4; ++i) partner[i] = __shfl_xor(v[i], 16);
  if (!xm || lg >= 2) return;
  qkv_rope_store(v, partner, head, half, p, ln, M, ra, len_dev, pos_dev, inv_freq);
}

// One decode row over a q|k|v weight of at least kDmaMinBytes (the 7B q/k/v,
// 33 MB): the weight streams HBM -> LDS through gemv_dma_kernel's four-wave
// ring (non-temporal whole-line DMA, 64-k stages, four slots per wave), with
// its K split and MFMA order, so the sums equal gemv_dma_kernel<4, false>'s
// and gemv_short_kernel's bit for bit. A workgroup owns 16 weight rows: eight
// rotary pairs p..p+7 of one head, p = 8 (block % 8), head = block / 8, tile
// row r holding column p + (r & 7) of half r / 8; the two halves of a pair
// meet 32 lanes apart. Nothing the ring has in flight is waited for before its
// turn: what the kernel reads besides the weight arrives by DMA ahead of the
// first stages (the activation slices; with NORM the x row and the norm
// weight; wave 0 the workgroup's bias) or by scalar loads after the first
// stages (the cache length, the position and the frequencies, whose rotation
// factors lanes 0 and 1 of each wave form while those stages are in flight,
// one pair a lane), and the norm's barriers are bare
// (__syncthreads would wait for every load in flight). With NORM the
// workgroup forms the RMSNorm row from LDS in the order of the rms_* helpers
// (rms_norm_kernel's output bit for bit) and writes it whole to LDS.
// Measured at the 7B shape, weights cold, graph-replayed: 8.7 us without the
// norm (the plain projection: 8.5 us) and 10.1 us with it, against 10.6 and
// 12.7 us with the rotation factors formed in the epilogue, the scalar loads
// ahead of the first stages and the norm's plain loads and __syncthreads
// draining the ring (13.8 us in the register kernel). Six ring slots instead
// of four measured slower with the norm (10.6 us).
template <bool NORM>
__global__ void __launch_bounds__(256)
gemv_qkv_rope_dma_kernel(const bf16_t* __restrict__ w, long long w_rs, const bf16_t* __restrict__ x,
                         const bf16_t* __restrict__ bias, int K, RopeArgs ra, const int32_t* __restrict__ len_dev,
                         const int32_t* __restrict__ pos_dev, const float* __restrict__ inv_freq,
                         const bf16_t* __restrict__ nw, float eps) {
  constexpr int WK = 4, KS = DmaCfg<WK>::KS, NSTG = DmaCfg<WK>::NSTG, HALF = kHeadDim / 2;
  constexpr int C = KS / 8, RPI = 64 / C, IPM = 16 / RPI;
  constexpr int kStageB = 16 * KS * 2;
  constexpr int kXsB = ((kShortMaxK / WK) * 2 + 1023) / 1024 * 1024;   // one wave's slice region
  constexpr int kRowB = NORM ? kQkvNormMaxK * 2 : 16;                   // the x row, the norm weight
  static_assert(!NORM || (kQkvNormMaxK <= kRmsMaxOneBatch && kRowB % 1024 == 0), "one load batch, whole pieces");
  __shared__ __align__(16) char rings[WK * NSTG * kStageB];
  __shared__ __align__(16) char xs_all[WK * kXsB];
  __shared__ __align__(16) char rows[2][kRowB];
  __shared__ __align__(16) char bias_s[1024];
  __shared__ f32x4 red[WK][64];
  __shared__ float rms_red[WK];
  __shared__ float2 cs[8];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ln = lane & 15, lg = lane >> 4;
  const int head = blockIdx.x / 8, p = (blockIdx.x % 8) * 8;
  const bool rotated = head < ra.n_q + ra.n_kv;          // query and key heads
  const int kw = (((K + WK - 1) / WK) + 31) / 32 * 32;   // <= kShortMaxK / WK (checked on the host)
  const int k_begin = min(K, wave * kw), k_end = min(K, k_begin + kw);
  const int nk = k_end - k_begin;
  const int nst = (nk + KS - 1) / KS;
  char* ring = rings + wave * NSTG * kStageB;
  // without NORM each wave's slice arrives in whole 1 KiB DMA pieces, so the
  // waves' regions are padded to whole pieces; with NORM the normalised row is
  // written whole, element i at byte 2 i, and each wave reads its K range of it
  char* xs = NORM ? xs_all + k_begin * 2 : xs_all + wave * kXsB;
  int row_b[IPM], lc[IPM];
#pragma unroll
  for (int i = 0; i < IPM; ++i) {
    const int r = RPI * i + lane / C;
    lc[i] = (lane % C) ^ (r % C);
    row_b[i] = ((r >> 3) * HALF + (r & 7)) * (int)(w_rs * 2);
  }
  const char* wb = reinterpret_cast<const char*>(w + (long long)(head * kHeadDim + p) * w_rs + k_begin);
  auto issue = [&](int s) {
    const uint32_t dst = lds_addr(ring + (s % NSTG) * kStageB);
#pragma unroll
    for (int i = 0; i < IPM; ++i) {
      const int kk = min(s * KS + 8 * lc[i], nk - 8);
      lds_dma16_sbase<true>(wb, (uint32_t)(row_b[i] + kk * 2), dst + i * 1024);
    }
  };
  // bias columns p..p+7 and p+64..p+71: two 16-byte pieces (lanes past 1 re-read the second)
  if (bias && wave == 0)
    lds_dma16_sbase<false>(bias + head * kHeadDim + p, (uint32_t)(min(lane, 1) * HALF * 2), lds_addr(bias_s));
  if constexpr (NORM) {                          // the rows' 1 KiB pieces, spread over the waves
    const int np = (K * 2 + 1023) / 1024;
    for (int q = wave; q < 2 * np; q += WK) {
      const int r = q >= np ? 1 : 0, b = (q - r * np) * 1024;
      lds_dma16_sbase<false>(r ? nw : x, (uint32_t)min(b + lane * 16, K * 2 - 16), lds_addr(rows[r] + b));
    }
  } else if (nk > 0) {                           // the wave's activation slice
    const char* xb = reinterpret_cast<const char*>(x + k_begin);
    for (int b = 0; b < nk * 2; b += 1024)
      lds_dma16_sbase<false>(xb, (uint32_t)min(b + lane * 16, nk * 2 - 16), lds_addr(xs + b));
  }
  const int pre = min(NSTG - 1, nst);
  for (int s = 0; s < pre; ++s) issue(s);
  // The cache length, the position and the frequencies are uniform: read as
  // constant memory they are scalar loads, counted apart from the ring's
  // vector-memory operations, and read after the first stages are issued, since
  // waiting for any scalar load waits for all of them.
  typedef const __attribute__((address_space(4))) int32_t* cint_p;
  typedef const __attribute__((address_space(4))) float* cfloat_p;
  const int len = head >= ra.n_q ? *(cint_p)len_dev : 0;
  if (rotated) {
    const int pos = *(cint_p)pos_dev + ra.pos_offset;
    const float f0 = ((cfloat_p)inv_freq)[p + 2 * wave], f1 = ((cfloat_p)inv_freq)[p + 2 * wave + 1];
    if (lane < 2) cs[2 * wave + lane] = rope_factors(pos, lane ? f1 : f0);
  }
  if constexpr (NORM) {
    wait_vm_stages<IPM, NSTG>(pre);              // this wave's row pieces have landed, its stages may not
    wg_barrier();
    bf16_t nx[kRmsBatch], ng[kRmsBatch];
    rms_load<bf16_t>(reinterpret_cast<const bf16_t*>(rows[0]), nx, 0, K, threadIdx.x);
    rms_load<bf16_t>(reinterpret_cast<const bf16_t*>(rows[1]), ng, 0, K, threadIdx.x);
    const float ss = rms_wave_sum(rms_add_squares<bf16_t>(0.f, nx, 0, K, threadIdx.x));
    if (lane == 0) rms_red[wave] = ss;
    __builtin_amdgcn_s_waitcnt(waitcnt_lgkm0());
    wg_barrier();
    const float inv = rms_inv(rms_red, K, eps);
    // all kRmsBatch elements, those past K too (never read): 256 kRmsBatch
    // elements fill the slice regions exactly
    static_assert(256 * kRmsBatch * 2 == WK * kXsB, "the batch fits the slice regions");
#pragma unroll
    for (int j = 0; j < kRmsBatch; ++j)
      *reinterpret_cast<bf16_t*>(xs_all + (threadIdx.x + 256 * j) * 2) = rms_scale<bf16_t>(nx[j], ng[j], inv);
    __builtin_amdgcn_s_waitcnt(waitcnt_lgkm0());
    wg_barrier();
  }
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < nst; ++s) {
    wait_vm_stages<IPM, NSTG - 1>(min(NSTG - 2, nst - 1 - s));
    if (s + NSTG - 1 < nst) issue(s + NSTG - 1);
    const char* st = ring + (s % NSTG) * kStageB;
#pragma unroll
    for (int u = 0; u < KS / 32; ++u) {
      const int kk = s * KS + 32 * u;
      if (kk < nk) {
        const bf16x8_t b = ln == 0 ? *reinterpret_cast<const bf16x8_t*>(xs + (kk + 8 * lg) * 2) : bf16x8_t{};
        const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(st + ln * (KS * 2) + (((4 * u + lg) ^ (ln % C)) << 4));
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));     // wave 0's bias piece (older than every stage; a no-op)
  red[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  f32x4 t = red[0][lane];
#pragma unroll
  for (int i = 1; i < WK; ++i) t += red[i][lane];
  // lane (0, lg): tile rows 4 lg .. 4 lg + 3 = columns pp .. pp + 3 of half lg / 2
  const int half = lg >> 1, q4 = 4 * (lg & 1), pp = p + q4;
  const bf16_t* bl = reinterpret_cast<const bf16_t*>(bias_s + half * 16) + q4;
  float v[4], partner[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = round_bf16(bias ? t[i] + to_f32<bf16_t>(bl[i]) : t[i]);
#pragma unroll
  for (int i = 0; i < 4; ++i) partner[i] = __shfl_xor(v[i], 32);
  if (ln != 0) return;
  bf16_t* dst = qkv_dest(head, half, pp, 0, 1, ra, len);
  if (!dst) return;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    dst[i] = from_f32<bf16_t>(rotated ? rope_rotate(half ? partner[i] : v[i], half ? v[i] : partner[i], cs[q4 + i], half)
                                      : v[i]);
}

// Waves per workgroup (the K split). The register kernels below serve the
// weights under kDmaMinBytes -- every 7B projection streams through the LDS
// ring kernels instead, which take four waves where this picks four and eight
// otherwise. The rule was fitted on the register kernels' durations at one and
// ten rows on the 7B shapes (16-column blocks: q/k/v 288, o and down 224,
// gate/up 1184 of 2368 stacked, lm_head 9504), the figures below. The split is
// chosen from the non-gated projection of all N_rows weight rows, so a gated
// launch adds exactly the sums of the plain projection of its stacked
// [gate; up] weight:
//  - up to kShortRows rows, K <= kShortMaxK and >= 256 blocks: four waves
//    (a K range of at most 1024 = kShortSteps steps per wave) -- the short
//    kernel, eight-column workgroups below 1024 blocks so the work spreads
//    over every CU (q/k/v 11.3 us; lm_head 171 us against 179 us streaming);
//    gated, the ring kernel (gate/up 48.5 us against 50.3 us at one wave);
//  - other shapes up to kShortRows rows: two waves, ring kernel (o 7.6 us
//    against 8.6 us on the short path; down 25.7 us);
//  - more rows: one wave (at ten rows o 9.0 us, down 32.3 us; gate/up 53.4 us
//    in gemv_gated_rows_kernel against 57-65 us for the ring kernel).
inline int gemv_waves(int M, int n_rows, int K) {
  if (M > kShortRows) return 1;
  return K <= kShortMaxK && (n_rows + 15) / 16 >= 256 ? 4 : 2;
}

// One row over a weight of at least kDmaMinBytes goes through the LDS ring
// (gemv_dma_kernel, four waves where gemv_waves picks four, else eight; two to
// sixteen rows through gemv_dma_rows_kernel): every projection of a 7B decode
// step -- q/k/v (33 MB: 8.5 us against 11.6 us in the short kernel), o (26 MB:
// 7.4 against 7.9 us), gate/up (271 MB), down (136 MB) and lm_head (1.09 GB)
// -- and of the ten-row verify step. Smaller weights keep the register kernels,
// whose single load round trip suits a launch of a few microseconds. The
// waves' activation slices must fit the dynamic LDS, and a wave's slice pieces
// plus its stages in flight the 63 outstanding vector-memory operations it can
// count.
constexpr long long kDmaMinBytes = 16ll << 20;
inline bool use_dma(int n_rows, int K, int wk, bool gated) {
  if (wk == 2 && gated) return false;          // eight waves of two row sets would crowd the LDS
  const int dk = wk == 4 ? 4 : 8;
  const int kw = (((K + dk - 1) / dk) + 31) / 32 * 32;
  const int in_flight = dk == 4 ? (DmaCfg<4>::NSTG - 1) * (gated ? 2 : 1) * 2 : (DmaCfg<8>::NSTG - 1) * 4;
  return (long long)n_rows * K * 2 >= kDmaMinBytes && gemv_dma_xs_bytes(dk, K) <= (48 << 10) &&
         (kw * 2 + 1023) / 1024 + in_flight <= 63;
}

// One row through gemv_dma_kernel at dk waves (a gated launch at four only).
template <bool GATED, bool NORM>
int launch_dma(int dk, const void* x, const void* w, long long w_rs, const void* bias, const void* residual,
               long long r_rs, void* y, int N, int K, const void* nw, float eps, hipStream_t st) {
  void (*kern)(const bf16_t*, long long, const bf16_t*, const bf16_t*, const bf16_t*, long long, bf16_t*, int, int,
               const bf16_t*, float);
  if constexpr (GATED) kern = gemv_dma_kernel<4, true, NORM>;
  else kern = dk == 4 ? gemv_dma_kernel<4, false, NORM> : gemv_dma_kernel<8, false, NORM>;
  if (GATED) dk = 4;
  hipLaunchKernelGGL(kern, dim3((N + 15) / 16), dim3(64 * dk), gemv_dma_lds_bytes(dk, K, NORM), st,
                     static_cast<const bf16_t*>(w), w_rs, static_cast<const bf16_t*>(x),
                     static_cast<const bf16_t*>(bias), static_cast<const bf16_t*>(residual), r_rs,
                     static_cast<bf16_t*>(y), N, K, static_cast<const bf16_t*>(nw), eps);
  return launch_status();
}

template <bool GATED>
int launch_gemv(const void* x, long long x_rs, const void* w, long long w_rs, const void* bias, const void* residual,
                long long r_rs, void* y, long long y_rs, int M, int N, int K, hipStream_t st) {
  const int blocks = (N + 15) / 16;
  const int wk = gemv_waves(M, GATED ? 2 * N : N, K);
  auto launch = [&](auto kern, int grid, int waves) {
    hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * waves), 0, st, static_cast<const bf16_t*>(w), w_rs,
                       static_cast<const bf16_t*>(x), x_rs, static_cast<const bf16_t*>(bias),
                       static_cast<const bf16_t*>(residual), r_rs, static_cast<bf16_t*>(y), y_rs, M, N, K);
  };
  static_assert((kShortMaxK / 4) / 32 <= kShortSteps, "four waves cover K in kShortSteps steps each");
  if (M == 1 && use_dma(GATED ? 2 * N : N, K, wk, GATED))
    return launch_dma<GATED, false>(wk == 4 ? 4 : 8, x, w, w_rs, bias, residual, r_rs, y, N, K, nullptr, 0.f, st);
  if (M > 1 && (long long)(GATED ? 2 * N : N) * K * 2 >= kDmaMinBytes) {
    // several rows: the ring with per-stage activation slabs, four waves
    // where gemv_waves picks four at up to four rows (and for every gated
    // launch), else eight
    const bool four = GATED || gemv_waves(1, N, K) == 4;
    void (*kern)(const bf16_t*, long long, const bf16_t*, long long, const bf16_t*, const bf16_t*, long long,
                 bf16_t*, long long, int, int, int);
    if constexpr (GATED) kern = gemv_dma_rows_kernel<4, true>;
    else kern = four ? gemv_dma_rows_kernel<4, false> : gemv_dma_rows_kernel<8, false>;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(four ? 256 : 512), 0, st, static_cast<const bf16_t*>(w), w_rs,
                       static_cast<const bf16_t*>(x), x_rs, static_cast<const bf16_t*>(bias),
                       static_cast<const bf16_t*>(residual), r_rs, static_cast<bf16_t*>(y), y_rs, M, N, K);
    return launch_status();
  }
  if constexpr (GATED) {
    if (wk == 4) launch(gemv_bf16_kernel<4, true>, blocks, 4);
    else if (wk == 2) launch(gemv_bf16_kernel<2, true>, blocks, 2);
    else launch(gemv_gated_rows_kernel, blocks, 1);
  } else {
    if (wk == 4) {
      if (blocks < 1024) launch(gemv_short_kernel<4, false, 8>, (N + 7) / 8, 4);
      else launch(gemv_short_kernel<4, false, 16>, blocks, 4);
    } else if (wk == 2) {
      launch(gemv_bf16_kernel<2, false>, blocks, 2);
    } else {
      launch(gemv_bf16_kernel<1, false>, blocks, 1);
    }
  }
  return launch_status();
}

int gemv_entry(const void* x, long long x_rs, const void* w, long long w_rs, const void* bias, const void* residual,
               long long r_rs, void* y, long long y_rs, int M, int N, int K, int dtype, bool gated, void* stream) {
  if (!x || !w || !y) return STD_E_NULL;
  if (dtype != STD_BF16) return STD_E_DTYPE;
  if (M < 1 || M > 16 || N < 1 || K < 32 || K % 32 != 0) return STD_E_SHAPE;
  if (x_rs < K || w_rs < K || y_rs < N) return STD_E_SHAPE;
  if (residual && r_rs < N) return STD_E_SHAPE;
  if (!aligned16(x) || !aligned16(w) || (x_rs * 2) % 16 || (w_rs * 2) % 16) return STD_E_ALIGN;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return gated ? launch_gemv<true>(x, x_rs, w, w_rs, bias, residual, r_rs, y, y_rs, M, N, K, st)
               : launch_gemv<false>(x, x_rs, w, w_rs, bias, residual, r_rs, y, y_rs, M, N, K, st);
}

}  // namespace
}  // namespace stdhip

extern "C" int std_gemv(const void* x, long long x_row_stride, const void* w, long long w_row_stride,
                        const void* bias, void* y, long long y_row_stride, int M, int N, int K, int dtype,
                        void* workspace, size_t workspace_bytes, void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  return gemv_entry(x, x_row_stride, w, w_row_stride, bias, nullptr, 0, y, y_row_stride, M, N, K, dtype, false,
                    stream);
}

extern "C" int std_gemv_ex(const void* x, long long x_row_stride, const void* w, long long w_row_stride,
                           const void* bias, const void* residual, long long residual_row_stride, void* y,
                           long long y_row_stride, int M, int N, int K, int gated, int dtype, void* stream) {
  return gemv_entry(x, x_row_stride, w, w_row_stride, bias, residual, residual_row_stride, y, y_row_stride, M, N, K,
                    dtype, gated != 0, stream);
}

extern "C" int std_gemv_norm(const void* x, const void* norm_weight, float eps, const void* w,
                             long long w_row_stride, const void* bias, const void* residual, void* y, int N, int K,
                             int gated, int dtype, void* stream) {
  if (!x || !norm_weight || !w || !y) return STD_E_NULL;
  if (dtype != STD_BF16) return STD_E_DTYPE;
  if (N < 1 || K < 32 || K % 32 != 0 || K > kGemvNormMaxK || w_row_stride < K) return STD_E_SHAPE;
  if (!aligned16(x) || !aligned16(norm_weight) || !aligned16(w) || (w_row_stride * 2) % 16) return STD_E_ALIGN;
  // the split std_gemv_ex's ring launch would use for this shape: four waves
  // where gemv_waves picks four (and for every gated launch), else eight
  const int dk = gated || gemv_waves(1, N, K) == 4 ? 4 : 8;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return gated ? launch_dma<true, true>(dk, x, w, w_row_stride, bias, residual, 0, y, N, K, norm_weight, eps, st)
               : launch_dma<false, true>(dk, x, w, w_row_stride, bias, residual, 0, y, N, K, norm_weight, eps, st);
}

extern "C" int std_qkv_rope_append(const void* x, long long x_row_stride, int n_rows, int K, const void* w,
                                   long long w_row_stride, const void* bias, int n_q, int n_kv, int d, void* q_out,
                                   void* cache_k, void* cache_v, long long cache_head_stride, int capacity,
                                   const int32_t* len_dev, const int32_t* pos_dev, int pos_offset,
                                   const float* inv_freq, const void* norm_weight, float eps, int dtype,
                                   int32_t* status, void* stream) {
  if (!x || !w || !q_out || !cache_k || !cache_v || !len_dev || !pos_dev || !inv_freq) return STD_E_NULL;
  if (norm_weight && (n_rows != 1 || K > kQkvNormMaxK)) return STD_E_SHAPE;
  if (dtype != STD_BF16) return STD_E_DTYPE;
  if (d != kHeadDim || n_rows < 1 || n_rows > kShortRows || n_q < 1 || n_kv < 1 || n_q % n_kv != 0 || capacity < 1)
    return STD_E_SHAPE;
  if (K < 32 || K % 32 != 0 || K > kShortMaxK || x_row_stride < K || w_row_stride < K) return STD_E_SHAPE;
  if (n_kv > 1 && cache_head_stride < (long long)capacity * kHeadDim) return STD_E_SHAPE;
  if (!aligned16(x) || !aligned16(w) || (x_row_stride * 2) % 16 || (w_row_stride * 2) % 16) return STD_E_ALIGN;
  static_assert((kShortMaxK / 4) / 32 <= kShortSteps, "four waves cover K in kShortSteps steps each");
  const RopeArgs ra{static_cast<bf16_t*>(q_out), static_cast<bf16_t*>(cache_k), static_cast<bf16_t*>(cache_v),
                    cache_head_stride, n_q, n_kv, capacity, pos_offset, status};
  if (n_rows == 1 && (long long)(n_q + 2 * n_kv) * kHeadDim * K * 2 >= kDmaMinBytes &&
      (!bias || aligned16(bias)) && (!norm_weight || aligned16(norm_weight))) {
    auto kern = norm_weight ? gemv_qkv_rope_dma_kernel<true> : gemv_qkv_rope_dma_kernel<false>;
    hipLaunchKernelGGL(kern, dim3((n_q + 2 * n_kv) * 8), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const bf16_t*>(w), w_row_stride, static_cast<const bf16_t*>(x),
                       static_cast<const bf16_t*>(bias), K, ra, len_dev, pos_dev, inv_freq,
                       static_cast<const bf16_t*>(norm_weight), eps);
    return launch_status();
  }
  auto kern = norm_weight ? gemv_qkv_rope_kernel<true> : gemv_qkv_rope_kernel<false>;
  hipLaunchKernelGGL(kern, dim3((n_q + 2 * n_kv) * 16), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const bf16_t*>(w), w_row_stride, static_cast<const bf16_t*>(x), x_row_stride,
                     static_cast<const bf16_t*>(bias), n_rows, K, ra, len_dev, pos_dev, inv_freq,
                     static_cast<const bf16_t*>(norm_weight), eps);
  return launch_status();
}
