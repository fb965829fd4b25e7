// Text-to-video top-K selection and sparse-cache compaction.
//
// Score of key j for KV head g (the reference sums the selection prefill's
// attention probabilities over the group's query heads and the text rows,
// src/std_repro/std_qwen25vl.py:204-218):
//     score[g][j] = sum_{h in g} sum_{i : j <= text_start + i} exp(s_hij - lse_hi)
//     s_hij = (q[h][i] . k[g][j]) * scale,  lse_hi = log sum_{j' <= text_start+i} exp(s_hij')
// Everything is fp64. A bf16*bf16 (or fp32*fp32) product is exact in fp64, so a
// 128-term fp64 dot product agrees with any other summation order to ~1e-16
// relative; the column scores of two platforms then differ by ~1e-15 relative,
// far below the gap between neighbouring scores, and the top-K index sets
// agree except on exact ties, which both sides break toward the lowest index.
// Every column is reduced by the same instruction sequence, so bit-identical
// key columns get bit-identical scores.
//
//   pass 1  sel_rowstats: per (row, key block) partial (max, sum exp)    MFMA f64
//   merge   sel_lse:      lse per row, blocks in fixed order
//   pass 2  sel_colsum:   per (row group, key) partial column sums       MFMA f64
//   keys    sel_keys:     column score of every visual position, row groups in order
//   select  sel_topk_*:   multi-block radix select of the k-th largest score
//                         (8 histogram passes), then per-block counts and an
//                         ordered emission of positions ascending (ties: lowest)
#include <cfloat>

#include "common.h"

namespace stdhip {
namespace {

constexpr int D = kHeadDim;

template <typename T> __device__ __forceinline__ double to_f64(T x) { return (double)to_f32<T>(x); }

__device__ __forceinline__ f64x4 mfma_f64(double a, double b, f64x4 c) {
  return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

// e^x in fp64 for the softmax terms here (x <= a few tens; x below -1000
// gives 0). Cody-Waite reduction x = n ln2 + r with ln2 split into a 42-bit
// head (n * head exact for |n| < 2^11) and a tail, |r| <= ln2/2; e^r by its
// degree-13 Taylor polynomial in Horner form (truncation < 5e-18 relative);
// exact scaling by 2^n. Worst error over a dense sample of [-745, 0] against a
// 60-digit reference: 0.81 ulp.
__device__ __forceinline__ double exp_f64(double x) {
  constexpr double kLog2e = 1.4426950408889634;
  constexpr double kLn2Hi = 0.6931471805598903;       // ln 2 cut to 42 significant bits
  constexpr double kLn2Lo = 5.497923018708371e-14;    // ln 2 - kLn2Hi
  x = fmax(x, -1000.0);
  const double n = rint(x * kLog2e);
  const double r = fma(-n, kLn2Lo, fma(-n, kLn2Hi, x));
  double p = 1.6059043836821613e-10;                  // 1/13!
  p = fma(p, r, 2.08767569878681e-09);                // 1/12!
  p = fma(p, r, 2.505210838544172e-08);               // 1/11!
  p = fma(p, r, 2.755731922398589e-07);               // 1/10!
  p = fma(p, r, 2.7557319223985893e-06);              // 1/9!
  p = fma(p, r, 2.48015873015873e-05);                // 1/8!
  p = fma(p, r, 0.0001984126984126984);               // 1/7!
  p = fma(p, r, 0.001388888888888889);                // 1/6!
  p = fma(p, r, 0.008333333333333333);                // 1/5!
  p = fma(p, r, 0.041666666666666664);                // 1/4!
  p = fma(p, r, 0.16666666666666666);                 // 1/3!
  p = fma(p, r, 0.5);
  p = fma(p, r, 1.0);
  p = fma(p, r, 1.0);
  return ldexp(p, (int)n);
}

// ---------------------------------------------------------------------------
// v_mfma_f64_16x16x4f64 operand layout (lane l = 16*lg + ln): A[m = ln][k = lg],
// B[k = lg][n = ln]; result element i of lane l is D[lg + 4*i][ln] (rows
// interleaved by 4, unlike the fp32-accumulator 16x16 forms whose element i is
// row 4*lg + i).
//
// Pass 1. grid (n_kb, n_kv, n_rg1), block 256 (4 waves x 2 row tiles of 16:
// 128 rows, so the 7 x 128 text rows of a GQA group need no padding).
// S^T tile = K Q^T: A[m = ln][k = lg] = K[key][4c + lg] from LDS (fp64),
// B[k = lg][n = ln] = Q[row][4c + lg] from registers; lane holds row ln and
// keys lg + 4i of the 16-key subtile. The next 64-key tile of K is loaded
// into registers (16-byte loads) while the current one is consumed.
constexpr int P1_RTW = 2;
constexpr int P1_WAVES = 4;
constexpr int P1_THREADS = 64 * P1_WAVES;
constexpr int P1_ROWS = P1_WAVES * P1_RTW * 16;  // 128 rows per workgroup
constexpr int P1_TK = 64;
constexpr int KROW64 = D + 1;                    // LDS pitch in doubles
constexpr double kMaxSlack = 32.0;               // natural-log units

template <typename T>
struct KTile {
  static constexpr int kPerChunk = 16 / (int)sizeof(T);           // elements per 16-byte load
  static constexpr int kChunksPerRow = D / kPerChunk;
  static constexpr int kPerThread = P1_TK * kChunksPerRow / P1_THREADS;
};

template <typename T>
__global__ void __launch_bounds__(P1_THREADS)
sel_rowstats_kernel(const T* __restrict__ q, const T* __restrict__ k, double2* __restrict__ part,
                    int group, int text_len, int prompt_len, int text_start, long long k_hs,
                    double scale, int keys_per_block, int n_kb) {
  using KT = KTile<T>;
  __shared__ double Ks[P1_TK * KROW64];
  const int kbk = blockIdx.x, g = blockIdx.y, rg = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, ln = lane & 15, lg = lane >> 4;
  const int R = group * text_len;

  float qf[P1_RTW][32];
  int lim[P1_RTW];
#pragma unroll
  for (int j = 0; j < P1_RTW; ++j) {
    const int r = (rg * P1_WAVES * P1_RTW + w * P1_RTW + j) * 16 + ln;
    if (r < R) {
      const int hl = r / text_len, i = r - hl * text_len;
      const T* row = q + ((long long)(g * group + hl) * text_len + i) * D;
#pragma unroll
      for (int c = 0; c < 32; ++c) qf[j][c] = to_f32<T>(row[4 * c + lg]);
      lim[j] = text_start + i;
    } else {
#pragma unroll
      for (int c = 0; c < 32; ++c) qf[j][c] = 0.f;
      lim[j] = -1;
    }
  }
  double m_run[P1_RTW], l_run[P1_RTW];
#pragma unroll
  for (int j = 0; j < P1_RTW; ++j) { m_run[j] = -DBL_MAX; l_run[j] = 0.0; }
  // smallest causal limit over the wave's rows (-1 if the wave has padding rows)
  int wave_lim = lim[0];
#pragma unroll
  for (int j = 1; j < P1_RTW; ++j) wave_lim = min(wave_lim, lim[j]);
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) wave_lim = min(wave_lim, __shfl_xor(wave_lim, off));

  const T* kh = k + (long long)g * k_hs;
  const int kbeg = kbk * keys_per_block;
  const int kend = min(prompt_len, kbeg + keys_per_block);
  // K tile staging: thread chunk e = tid + P1_THREADS * i is row e / kChunksPerRow,
  // 16 bytes at element (e % kChunksPerRow) * kPerChunk; rows past the block's
  // last key re-read that key and are stored as zeros.
  uint4 kpre[KT::kPerThread];
  auto load_tile = [&](int key0) {
#pragma unroll
    for (int i = 0; i < KT::kPerThread; ++i) {
      const int e = tid + P1_THREADS * i, kr = e / KT::kChunksPerRow;
      const int c0 = (e - kr * KT::kChunksPerRow) * KT::kPerChunk;
      const int key = min(key0 + kr, kend - 1);
      kpre[i] = *reinterpret_cast<const uint4*>(kh + (long long)key * D + c0);
    }
  };
  auto store_tile = [&](int key0) {
#pragma unroll
    for (int i = 0; i < KT::kPerThread; ++i) {
      const int e = tid + P1_THREADS * i, kr = e / KT::kChunksPerRow;
      const int c0 = (e - kr * KT::kChunksPerRow) * KT::kPerChunk;
      const bool ok = key0 + kr < kend;
      const T* v = reinterpret_cast<const T*>(&kpre[i]);
      double* dst = Ks + kr * KROW64 + c0;
#pragma unroll
      for (int j = 0; j < KT::kPerChunk; ++j) dst[j] = ok ? to_f64<T>(v[j]) : 0.0;
    }
  };
  load_tile(kbeg);
  for (int key0 = kbeg; key0 < kend; key0 += P1_TK) {
    __syncthreads();
    store_tile(key0);
    __syncthreads();
    if (key0 + P1_TK < kend) load_tile(key0 + P1_TK);
#pragma unroll 1
    for (int ks = 0; ks < P1_TK / 16; ++ks) {
      f64x4 acc[P1_RTW];
#pragma unroll
      for (int j = 0; j < P1_RTW; ++j) acc[j] = f64x4{0.0, 0.0, 0.0, 0.0};
      const double* arow = Ks + (ks * 16 + ln) * KROW64 + lg;
#pragma unroll
      for (int c = 0; c < 32; ++c) {
        const double a = arow[4 * c];
#pragma unroll
        for (int j = 0; j < P1_RTW; ++j) acc[j] = mfma_f64(a, (double)qf[j][c], acc[j]);
      }
      const int kb = key0 + ks * 16 + lg;
      // wave-uniform: every key of the subtile exists and every row of the
      // wave sees it, so no element needs its mask
      const bool full = key0 + ks * 16 + 16 <= min(kend, wave_lim + 1);
#pragma unroll
      for (int j = 0; j < P1_RTW; ++j) {
        double s[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) s[i] = acc[j][i] * scale;
        if (!full) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = kb + 4 * i;
            s[i] = (key < kend && key <= lim[j]) ? s[i] : -INFINITY;
          }
        }
        // The running max is raised (one wave-uniform branch) only when a
        // score exceeds it by more than kMaxSlack, so terms stay <= e^kMaxSlack.
        const double mt = fmax(fmax(s[0], s[1]), fmax(s[2], s[3]));
        if (__ballot(mt > m_run[j] + kMaxSlack)) {
          const double mn = fmax(m_run[j], mt);
          l_run[j] *= exp_f64(m_run[j] - mn);
          m_run[j] = mn;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) l_run[j] += exp_f64(s[i] - m_run[j]);
      }
    }
  }
  // combine the four lane groups (disjoint keys of the same row)
#pragma unroll
  for (int j = 0; j < P1_RTW; ++j) {
    double m = m_run[j], l = l_run[j];
#pragma unroll
    for (int off = 16; off <= 32; off <<= 1) {
      const double mo = __shfl_xor(m, off), lo = __shfl_xor(l, off);
      const double mm = fmax(m, mo);
      l = l * exp_f64(m - mm) + lo * exp_f64(mo - mm);
      m = mm;
    }
    const int r = (rg * P1_WAVES * P1_RTW + w * P1_RTW + j) * 16 + ln;
    if (lg == 0 && r < R) part[((long long)g * n_kb + kbk) * R + r] = make_double2(m, l);
  }
}

// lse[g][r] from the n_kb partials, in block order.
__global__ void __launch_bounds__(256)
sel_lse_kernel(const double2* __restrict__ part, double* __restrict__ lse, int R, int n_kb, int n_kv) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= n_kv * R) return;
  const int g = idx / R, r = idx - g * R;
  const double2* p = part + (long long)g * n_kb * R + r;
  double M = -DBL_MAX;
  for (int b = 0; b < n_kb; ++b) M = fmax(M, p[(long long)b * R].x);
  double L = 0.0;
  for (int b = 0; b < n_kb; ++b) {
    const double2 v = p[(long long)b * R];
    L += v.y * exp_f64(v.x - M);
  }
  lse[idx] = M + log(L);
}

// ---------------------------------------------------------------------------
// Pass 2. grid (n_kb2, n_kv, n_rg2), block 512. A row group of 128 rows is
// staged in LDS; each of the 8 waves takes 16-key column tiles, holds K^T in
// registers and walks the 8 row tiles: S tile = Q K^T, A[m = ln][k = lg] =
// Q[row][4c+lg], B[k = lg][n = ln] = K[key][4c + lg]; lane holds key ln and
// rows lg + 4i.
constexpr int P2_RT = 8;
constexpr int P2_ROWS = P2_RT * 16;
constexpr int P2_WAVES = 8;
constexpr int P2_THREADS = 64 * P2_WAVES;
constexpr int QROW = D + 4;

template <typename T>
__global__ void __launch_bounds__(P2_THREADS)
sel_colsum_kernel(const T* __restrict__ q, const T* __restrict__ k, const double* __restrict__ lse,
                  double* __restrict__ colpart, int group, int text_len, int prompt_len, int text_start,
                  long long k_hs, double scale, int keys_per_block, int n_kv) {
  __shared__ float Qs[P2_ROWS * QROW];
  __shared__ double Ls[P2_ROWS];
  __shared__ int Lim[P2_ROWS];
  const int kbk = blockIdx.x, g = blockIdx.y, rg = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, ln = lane & 15, lg = lane >> 4;
  const int R = group * text_len;
  for (int e = tid; e < P2_ROWS * D; e += P2_THREADS) {
    const int rr = e / D, d = e - rr * D, r = rg * P2_ROWS + rr;
    float v = 0.f;
    if (r < R) {
      const int hl = r / text_len, i = r - hl * text_len;
      v = to_f32<T>(q[((long long)(g * group + hl) * text_len + i) * D + d]);
    }
    Qs[rr * QROW + d] = v;
  }
  for (int e = tid; e < P2_ROWS; e += P2_THREADS) {
    const int r = rg * P2_ROWS + e;
    Ls[e] = r < R ? lse[(long long)g * R + r] : 0.0;
    Lim[e] = r < R ? text_start + (r % text_len) : -1;
  }
  __syncthreads();

  const T* kh = k + (long long)g * k_hs;
  const int kbeg = kbk * keys_per_block;
  const int kend = min(prompt_len, kbeg + keys_per_block);
  const bool rows_full = (rg + 1) * P2_ROWS <= R;   // no padding rows in this group
  for (int kt0 = kbeg + w * 16; kt0 < kend; kt0 += P2_WAVES * 16) {
    const int key = kt0 + ln;
    // every lane loads (a key past the block's end re-reads the last key), so
    // the 32 loads are in flight together; such columns are zeroed
    const T* krow = kh + (long long)min(key, kend - 1) * D + lg;
    double bk[32];
#pragma unroll
    for (int c = 0; c < 32; ++c) bk[c] = to_f64<T>(krow[4 * c]);
#pragma unroll
    for (int c = 0; c < 32; ++c) bk[c] = key < kend ? bk[c] : 0.0;
    // wave-uniform: all 16 keys exist and all rows of the group see them
    const bool full = rows_full && kt0 + 16 <= min(kend, text_start + 1);
    double colsum = 0.0;
#pragma unroll 1
    for (int rt = 0; rt < P2_RT; ++rt) {
      double lse_r[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) lse_r[i] = Ls[rt * 16 + lg + 4 * i];
      f64x4 acc = {0.0, 0.0, 0.0, 0.0};
      const float* arow = Qs + (rt * 16 + ln) * QROW + lg;
#pragma unroll
      for (int c = 0; c < 32; ++c) acc = mfma_f64((double)arow[4 * c], bk[c], acc);
      if (full) {
#pragma unroll
        for (int i = 0; i < 4; ++i) colsum += exp_f64(acc[i] * scale - lse_r[i]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const double e = exp_f64(acc[i] * scale - lse_r[i]);
          colsum += (key < kend && key <= Lim[rt * 16 + lg + 4 * i]) ? e : 0.0;
        }
      }
    }
    colsum += __shfl_xor(colsum, 16);
    colsum += __shfl_xor(colsum, 32);
    if (lg == 0 && key < kend) colpart[((long long)rg * n_kv + g) * prompt_len + key] = colsum;
  }
}

// Column score of each visual position as an order-preserving u64 key
// (scores are >= 0, so the IEEE bit pattern orders like the value), and the
// optional full score row; the first block of each head also clears that
// head's radix histograms. grid (ceil(max(n_vis, P) / 256), n_kv), block 256.
__global__ void __launch_bounds__(256)
sel_keys_kernel(const double* __restrict__ colpart, int n_rg2, int n_kv, int prompt_len,
                const int32_t* __restrict__ vis, int n_vis, unsigned long long* __restrict__ keys,
                double* __restrict__ scores_out, unsigned* __restrict__ hist) {
  const int g = blockIdx.y;
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (blockIdx.x == 0)
    for (int p = 0; p < 8; ++p) hist[((long long)p * n_kv + g) * 256 + threadIdx.x] = 0u;
  if (t < n_vis) {
    const int j = vis[t];
    double s = 0.0;
    if (j >= 0 && j < prompt_len)
      for (int rg = 0; rg < n_rg2; ++rg) s += colpart[((long long)rg * n_kv + g) * prompt_len + j];
    keys[(long long)g * n_vis + t] = (unsigned long long)__double_as_longlong(s);
  }
  if (scores_out != nullptr && t < prompt_len) {
    double s = 0.0;
    for (int rg = 0; rg < n_rg2; ++rg) s += colpart[((long long)rg * n_kv + g) * prompt_len + t];
    scores_out[(long long)g * prompt_len + t] = s;
  }
}

// ---------------------------------------------------------------------------
// Top-k by a multi-block radix select over the u64 keys, 8 bits per pass from
// the top. Pass p histograms digit p of the keys whose higher digits equal
// those of the k-th largest key (found from passes < p): every block adds its
// slice's histogram into hist[p][g][256] (zeroed by sel_keys_kernel) and
// re-derives the earlier digits from those histograms, so no state but the
// histograms passes between launches. sel_topk_count then counts, per block,
// the keys above the k-th largest key T and the keys equal to it, and
// sel_topk_emit writes every key above T and the kk lowest-position keys equal
// to T (kk = k minus the count above T), positions ascending.
constexpr int TOPK_THREADS = 256;
constexpr int TOPK_PER_THREAD = 16;
constexpr int TOPK_SLICE = TOPK_THREADS * TOPK_PER_THREAD;   // keys per block
constexpr int TOPK_PASSES = 8;

int topk_blocks(int n_vis) { return (n_vis + TOPK_SLICE - 1) / TOPK_SLICE; }

// Exclusive prefix sum over the block (TOPK_THREADS threads) in thread order;
// *total receives the block sum.
__device__ int block_exclusive_scan(int v, int* wave_tot, int* total) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  if (lane == 63) wave_tot[w] = x;
  __syncthreads();
  if (tid == 0) {
    int acc = 0;
    for (int i = 0; i < TOPK_THREADS / 64; ++i) {
      const int t = wave_tot[i];
      wave_tot[i] = acc;
      acc += t;
    }
    *total = acc;
  }
  __syncthreads();
  const int res = wave_tot[w] + x - v;
  __syncthreads();
  return res;
}

struct RadixState {
  unsigned long long prefix, mask;
  int kk;   // rank (from the top) of the k-th largest key among keys matching prefix
};

// The k-th largest key's digits of passes [0, n_pass) from the histograms;
// thread t examines digit 255 - t, so the exclusive scan counts larger digits.
__device__ RadixState radix_state(const unsigned* __restrict__ hist, int g, int n_kv, int n_pass, int k_sel,
                                  int* wave_tot, int* sh) {
  RadixState st{0ull, 0ull, k_sel};
  const int tid = threadIdx.x;
  for (int p = 0; p < n_pass; ++p) {
    const int digit = 255 - tid;
    const int c = (int)hist[((long long)p * n_kv + g) * 256 + digit];
    const int above = block_exclusive_scan(c, wave_tot, sh + 2);
    if (above < st.kk && st.kk <= above + c) {
      sh[0] = digit;
      sh[1] = st.kk - above;
    }
    __syncthreads();
    const int shift = 56 - 8 * p;
    st.prefix |= (unsigned long long)sh[0] << shift;
    st.mask |= 255ull << shift;
    st.kk = sh[1];
    __syncthreads();
  }
  return st;
}

// LDS histogram add with one atomic per wave when all active lanes share a bin
// (the common case in the first passes, where most keys share a digit).
__device__ __forceinline__ void wave_hist_add(unsigned* h, unsigned bin, bool act, int lane) {
  const unsigned long long a = __ballot(act);
  if (a == 0) return;
  const int leader = __ffsll((long long)a) - 1;
  const unsigned b0 = __shfl(bin, leader);
  if (__ballot(act && bin == b0) == a) {
    if (lane == leader) atomicAdd(&h[b0], (unsigned)__popcll(a));
  } else if (act) {
    atomicAdd(&h[bin], 1u);
  }
}

// grid (topk_blocks(n_vis), n_kv), block TOPK_THREADS.
__global__ void __launch_bounds__(TOPK_THREADS)
sel_topk_hist_kernel(const unsigned long long* __restrict__ keys_all, int n_vis, int k_sel, int n_kv,
                     unsigned* __restrict__ hist, int pass) {
  __shared__ unsigned h[256];
  __shared__ int wave_tot[TOPK_THREADS / 64];
  __shared__ int sh[3];
  const int g = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
  const RadixState st = radix_state(hist, g, n_kv, pass, k_sel, wave_tot, sh);
  h[tid] = 0;
  __syncthreads();
  const unsigned long long* keys = keys_all + (long long)g * n_vis;
  const int shift = 56 - 8 * pass, base = blockIdx.x * TOPK_SLICE;
#pragma unroll 4
  for (int i = 0; i < TOPK_PER_THREAD; ++i) {
    const int t = base + i * TOPK_THREADS + tid;
    bool act = false;
    unsigned bin = 0;
    if (t < n_vis) {
      const unsigned long long u = keys[t];
      act = (u & st.mask) == st.prefix;
      bin = (unsigned)(u >> shift) & 255u;
    }
    wave_hist_add(h, bin, act, lane);
  }
  __syncthreads();
  if (h[tid]) atomicAdd(&hist[((long long)pass * n_kv + g) * 256 + tid], h[tid]);
}

// Thread tid owns keys [base + tid * TOPK_PER_THREAD, +TOPK_PER_THREAD) of the
// block's slice (contiguous, so thread order is position order).
__device__ __forceinline__ void slice_range(int n_vis, int& t0, int& t1) {
  t0 = min(n_vis, blockIdx.x * TOPK_SLICE + (int)threadIdx.x * TOPK_PER_THREAD);
  t1 = min(n_vis, t0 + TOPK_PER_THREAD);
}

// grid (topk_blocks(n_vis), n_kv): counts[g][blk] = (keys > T, keys == T).
__global__ void __launch_bounds__(TOPK_THREADS)
sel_topk_count_kernel(const unsigned long long* __restrict__ keys_all, int n_vis, int k_sel, int n_kv,
                      const unsigned* __restrict__ hist, int2* __restrict__ counts, int n_tb) {
  __shared__ int wave_tot[TOPK_THREADS / 64];
  __shared__ int sh[3];
  __shared__ int s_gt;
  const int g = blockIdx.y;
  const RadixState st = radix_state(hist, g, n_kv, TOPK_PASSES, k_sel, wave_tot, sh);
  const unsigned long long* keys = keys_all + (long long)g * n_vis;
  int t0, t1, gt = 0, eq = 0;
  slice_range(n_vis, t0, t1);
  for (int t = t0; t < t1; ++t) {
    const unsigned long long u = keys[t];
    gt += u > st.prefix;
    eq += u == st.prefix;
  }
  block_exclusive_scan(gt, wave_tot, &s_gt);
  block_exclusive_scan(eq, wave_tot, sh + 2);
  if (threadIdx.x == 0) counts[(long long)g * n_tb + blockIdx.x] = make_int2(s_gt, sh[2]);
}

// grid (topk_blocks(n_vis), n_kv): emit the block's selected positions at
// their global ranks.
__global__ void __launch_bounds__(TOPK_THREADS)
sel_topk_emit_kernel(const unsigned long long* __restrict__ keys_all, const int32_t* __restrict__ vis, int n_vis,
                     int k_sel, int n_kv, const unsigned* __restrict__ hist, const int2* __restrict__ counts,
                     int32_t* __restrict__ topk_out, int n_tb) {
  __shared__ int wave_tot[TOPK_THREADS / 64];
  __shared__ int sh[3];
  __shared__ int s_before[2];
  const int g = blockIdx.y, tid = threadIdx.x;
  const RadixState st = radix_state(hist, g, n_kv, TOPK_PASSES, k_sel, wave_tot, sh);
  const unsigned long long T = st.prefix;
  const int kk = st.kk;
  if (tid == 0) {
    int eq_before = 0, sel_before = 0;
    for (int b = 0; b < (int)blockIdx.x; ++b) {
      const int2 c = counts[(long long)g * n_tb + b];
      sel_before += c.x + min(max(kk - eq_before, 0), c.y);
      eq_before += c.y;
    }
    s_before[0] = eq_before;
    s_before[1] = sel_before;
  }
  __syncthreads();
  const unsigned long long* keys = keys_all + (long long)g * n_vis;
  int t0, t1, n_eq = 0;
  slice_range(n_vis, t0, t1);
  for (int t = t0; t < t1; ++t) n_eq += keys[t] == T;
  int eq_rank = s_before[0] + block_exclusive_scan(n_eq, wave_tot, sh + 2);
  int n_sel = 0;
  {
    int r = eq_rank;
    for (int t = t0; t < t1; ++t) {
      const unsigned long long u = keys[t];
      if (u > T) ++n_sel;
      else if (u == T) { if (r < kk) ++n_sel; ++r; }
    }
  }
  int off = s_before[1] + block_exclusive_scan(n_sel, wave_tot, sh + 2);
  int32_t* out = topk_out + (long long)g * k_sel;
  for (int t = t0; t < t1; ++t) {
    const unsigned long long u = keys[t];
    bool take = false;
    if (u > T) take = true;
    else if (u == T) { take = eq_rank < kk; ++eq_rank; }
    if (take && off < k_sel) out[off++] = vis[t];
  }
}

// ---------------------------------------------------------------------------
// Compact index: sorted union of two disjoint sorted lists.
__device__ __forceinline__ int count_below(const int32_t* a, int n, int v) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (a[mid] < v) lo = mid + 1; else hi = mid;
  }
  return lo;
}

__global__ void __launch_bounds__(256)
compact_index_kernel(const int32_t* __restrict__ nonvis, int n_nv, const int32_t* __restrict__ topk, int k_sel,
                     int32_t* __restrict__ idx_out) {
  const int g = blockIdx.y;
  const int t = blockIdx.x * 256 + threadIdx.x;
  const int total = n_nv + k_sel;
  if (t >= total) return;
  const int32_t* tk = topk + (long long)g * k_sel;
  int32_t* out = idx_out + (long long)g * total;
  if (t < n_nv) {
    const int v = nonvis[t];
    out[t + count_below(tk, k_sel, v)] = v;
  } else {
    const int j = t - n_nv, v = tk[j];
    out[j + count_below(nonvis, n_nv, v)] = v;
  }
}

// Row gather / scatter in 16-byte chunks (element-type agnostic).
// grid (ceil(rows * cpr / 256), n_kv, 2 for K and V).
__global__ void __launch_bounds__(256)
compact_kv_kernel(const char* __restrict__ dk, const char* __restrict__ dv, char* __restrict__ sk,
                  char* __restrict__ sv, const int32_t* __restrict__ idx, int compact_len, int row_bytes,
                  long long dhs_bytes, int dense_rows, long long shs_bytes, int sparse_rows) {
  const int g = blockIdx.y, kv = blockIdx.z;
  const int cpr = row_bytes / 16;
  const int c = blockIdx.x * 256 + threadIdx.x;
  const int s = c / cpr, col = c - s * cpr;
  if (s >= compact_len || s >= sparse_rows) return;
  const int src_row = idx[(long long)g * compact_len + s];
  if (src_row < 0 || src_row >= dense_rows) return;
  const char* src = (kv ? dv : dk) + g * dhs_bytes + (long long)src_row * row_bytes + col * 16;
  char* dst = (kv ? sv : sk) + g * shs_bytes + (long long)s * row_bytes + col * 16;
  *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
}

// ---------------------------------------------------------------------------
struct SelectPlan {
  int R, n_rg1, n_kb, kpb1, n_rg2, n_kb2, kpb2, n_tb;
  size_t off_part, off_lse, off_col, off_keys, off_hist, off_cnt, total;
};

SelectPlan plan_select(int n_q, int n_kv, int text_len, int prompt_len, int n_vis) {
  SelectPlan p;
  p.R = (n_q / n_kv) * text_len;
  p.n_rg1 = (p.R + P1_ROWS - 1) / P1_ROWS;
  int per_kb = n_kv * p.n_rg1;
  p.n_kb = 512 / per_kb > 0 ? 512 / per_kb : 1;       // at most 2 workgroups per CU, one round
  p.kpb1 = (int)round_up((size_t)((prompt_len + p.n_kb - 1) / p.n_kb), P1_TK);
  p.n_kb = (prompt_len + p.kpb1 - 1) / p.kpb1;
  p.n_rg2 = (p.R + P2_ROWS - 1) / P2_ROWS;
  per_kb = n_kv * p.n_rg2;
  p.n_kb2 = 1024 / per_kb > 0 ? 1024 / per_kb : 1;    // at most two rounds of 2 workgroups per CU
  p.kpb2 = (int)round_up((size_t)((prompt_len + p.n_kb2 - 1) / p.n_kb2), P2_WAVES * 16);
  p.n_kb2 = (prompt_len + p.kpb2 - 1) / p.kpb2;
  p.off_part = 0;
  p.off_lse = round_up(p.off_part + (size_t)n_kv * p.n_kb * p.R * sizeof(double2), 256);
  p.off_col = round_up(p.off_lse + (size_t)n_kv * p.R * sizeof(double), 256);
  p.off_keys = round_up(p.off_col + (size_t)p.n_rg2 * n_kv * prompt_len * sizeof(double), 256);
  p.n_tb = topk_blocks(n_vis);
  p.off_hist = round_up(p.off_keys + (size_t)n_kv * n_vis * sizeof(unsigned long long), 256);
  p.off_cnt = round_up(p.off_hist + (size_t)TOPK_PASSES * n_kv * 256 * sizeof(unsigned), 256);
  p.total = round_up(p.off_cnt + (size_t)n_kv * p.n_tb * sizeof(int2), 256);
  return p;
}

bool select_shape_ok(int n_q, int n_kv, int text_len, int prompt_len, int text_start, int d, int n_vis, int k_sel) {
  if (d != D || n_q <= 0 || n_kv <= 0 || n_q % n_kv != 0) return false;
  if (text_len < 1 || text_start < 0 || prompt_len != text_start + text_len) return false;
  if (n_vis < 1 || n_vis > prompt_len || k_sel < 1 || k_sel > n_vis) return false;
  return true;
}

// From column partials colpart[rg][g][prompt_len] (fp64, n_rg row groups):
// the u64 keys of the visual columns, the radix passes, counts and the
// ordered emission of the k_sel selected positions per KV head.
int launch_topk(const double* colpart, int n_rg, int n_kv, int prompt_len, const int32_t* vis, int n_vis, int k_sel,
                int32_t* topk_out, double* scores_out, unsigned long long* keys, unsigned* hist, int2* counts,
                hipStream_t st) {
  const int n_cols = n_vis > prompt_len ? n_vis : prompt_len;
  hipLaunchKernelGGL(sel_keys_kernel, dim3((n_cols + 255) / 256, n_kv), dim3(256), 0, st, colpart, n_rg, n_kv,
                     prompt_len, vis, n_vis, keys, scores_out, hist);
  int s = launch_status();
  if (s) return s;
  const dim3 tgrid(topk_blocks(n_vis), n_kv);
  for (int pass = 0; pass < TOPK_PASSES; ++pass) {
    hipLaunchKernelGGL(sel_topk_hist_kernel, tgrid, dim3(TOPK_THREADS), 0, st, keys, n_vis, k_sel, n_kv, hist, pass);
    if ((s = launch_status())) return s;
  }
  hipLaunchKernelGGL(sel_topk_count_kernel, tgrid, dim3(TOPK_THREADS), 0, st, keys, n_vis, k_sel, n_kv, hist, counts,
                     (int)tgrid.x);
  if ((s = launch_status())) return s;
  hipLaunchKernelGGL(sel_topk_emit_kernel, tgrid, dim3(TOPK_THREADS), 0, st, keys, vis, n_vis, k_sel, n_kv, hist,
                     counts, topk_out, (int)tgrid.x);
  return launch_status();
}

// ---------------------------------------------------------------------------
// Selection from materialised attention probabilities, the reference's input
// (std_qwen25vl.py:175-231: per layer [1, n_q, T, P] probabilities of the text
// suffix's rows over the prompt, summed over the query heads of each KV head
// and the text rows, then top-k over the visual columns). colpart[rg][g][j] =
// the fp64 sum of column j over row group rg's probability rows (row r = head
// r / T of the group, text row r % T), rows in order; the keys stage adds the
// row groups in order. fp64 holds any sum of fp16 probabilities exactly, so
// the scores and the selected positions do not depend on the summation order.
// grid (ceil(P / 1024), n_kv, n_rg), block 256: thread t sums columns
// 4 (blockIdx.x * 256 + t) .. +3.
template <typename T>
__device__ __forceinline__ double prob_to_f64(T x);
template <> __device__ __forceinline__ double prob_to_f64<float>(float x) { return (double)x; }
template <> __device__ __forceinline__ double prob_to_f64<bf16_t>(bf16_t x) { return (double)bf16_to_f32(x); }
struct f16_bits {
  uint16_t v;
};
template <> __device__ __forceinline__ double prob_to_f64<f16_bits>(f16_bits x) {
  return (double)(float)__builtin_bit_cast(_Float16, x.v);
}

// VEC: four-column vector loads (rows 8-byte aligned for 16-bit types,
// 16-byte for fp32); otherwise element loads, for any prompt length and
// stride (the reference's contiguous [1, Hq, T, P] probabilities have row
// stride P, which is odd for most prompts).
template <typename T, bool VEC>
__global__ void __launch_bounds__(256)
probs_colsum_kernel(const T* __restrict__ probs, long long head_stride, long long row_stride, int group, int text_len,
                    int prompt_len, int rows_per_rg, double* __restrict__ colpart, int n_kv) {
  const int g = blockIdx.y, rg = blockIdx.z;
  const int j0 = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (j0 >= prompt_len) return;
  const int R = group * text_len;
  const int r0 = rg * rows_per_rg, r1 = min(R, r0 + rows_per_rg);
  const bool full = j0 + 4 <= prompt_len;
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll 8
  for (int r = r0; r < r1; ++r) {
    const int hl = r / text_len, t = r - hl * text_len;
    const T* row = probs + (long long)(g * group + hl) * head_stride + (long long)t * row_stride + j0;
    T x[4];
    if (VEC && full) {
      if constexpr (sizeof(T) == 2) {
        const uint2 u = *reinterpret_cast<const uint2*>(row);
        x[0] = __builtin_bit_cast(T, (uint16_t)(u.x & 0xffffu));
        x[1] = __builtin_bit_cast(T, (uint16_t)(u.x >> 16));
        x[2] = __builtin_bit_cast(T, (uint16_t)(u.y & 0xffffu));
        x[3] = __builtin_bit_cast(T, (uint16_t)(u.y >> 16));
      } else {
        const float4 u = *reinterpret_cast<const float4*>(row);
        x[0] = __builtin_bit_cast(T, u.x);
        x[1] = __builtin_bit_cast(T, u.y);
        x[2] = __builtin_bit_cast(T, u.z);
        x[3] = __builtin_bit_cast(T, u.w);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = row[min(e, prompt_len - 1 - j0)];   // in-row: columns past P re-read P - 1
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += prob_to_f64<T>(x[e]);
  }
  double* dst = colpart + ((long long)rg * n_kv + g) * prompt_len + j0;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (j0 + e < prompt_len) dst[e] = acc[e];
}

struct ProbsPlan {
  int n_rg, rows_per_rg, n_tb;
  size_t off_col, off_keys, off_hist, off_cnt, total;
};

ProbsPlan plan_probs(int n_q, int n_kv, int text_len, int prompt_len, int n_vis) {
  ProbsPlan p;
  const int R = (n_q / n_kv) * text_len;
  const int n_cb = (prompt_len + 1023) / 1024;
  int n_rg = 2048 / (n_cb * n_kv);                      // about 2048 workgroups (8 per CU)
  n_rg = n_rg < 1 ? 1 : n_rg > 64 ? 64 : n_rg;
  n_rg = n_rg > R ? R : n_rg;
  p.rows_per_rg = (R + n_rg - 1) / n_rg;
  p.n_rg = (R + p.rows_per_rg - 1) / p.rows_per_rg;
  p.n_tb = topk_blocks(n_vis);
  p.off_col = 0;
  p.off_keys = round_up((size_t)p.n_rg * n_kv * prompt_len * sizeof(double), 256);
  p.off_hist = round_up(p.off_keys + (size_t)n_kv * n_vis * sizeof(unsigned long long), 256);
  p.off_cnt = round_up(p.off_hist + (size_t)TOPK_PASSES * n_kv * 256 * sizeof(unsigned), 256);
  p.total = round_up(p.off_cnt + (size_t)n_kv * p.n_tb * sizeof(int2), 256);
  return p;
}

template <typename T>
int launch_select_probs(const void* probs, long long head_stride, long long row_stride, int n_q, int n_kv,
                        int text_len, int prompt_len, const int32_t* vis, int n_vis, int k_sel, int32_t* topk_out,
                        double* scores_out, void* ws, hipStream_t st) {
  const ProbsPlan p = plan_probs(n_q, n_kv, text_len, prompt_len, n_vis);
  char* base = static_cast<char*>(ws);
  double* colpart = reinterpret_cast<double*>(base + p.off_col);
  const size_t vb = 4 * sizeof(T);
  const bool vec = (uintptr_t)probs % vb == 0 && (row_stride * (long long)sizeof(T)) % vb == 0 &&
                   (head_stride * (long long)sizeof(T)) % vb == 0;
  auto kern = vec ? probs_colsum_kernel<T, true> : probs_colsum_kernel<T, false>;
  hipLaunchKernelGGL(kern, dim3((prompt_len + 1023) / 1024, n_kv, p.n_rg), dim3(256), 0, st,
                     static_cast<const T*>(probs), head_stride, row_stride, n_q / n_kv, text_len, prompt_len,
                     p.rows_per_rg, colpart, n_kv);
  const int s = launch_status();
  if (s) return s;
  return launch_topk(colpart, p.n_rg, n_kv, prompt_len, vis, n_vis, k_sel, topk_out, scores_out,
                     reinterpret_cast<unsigned long long*>(base + p.off_keys),
                     reinterpret_cast<unsigned*>(base + p.off_hist), reinterpret_cast<int2*>(base + p.off_cnt), st);
}

template <typename T>
int launch_select(const void* q_text, const void* k, int n_q, int n_kv, int text_len, int prompt_len, int text_start,
                  long long k_hs, const int32_t* vis, int n_vis, int k_sel, int32_t* topk_out, double* scores_out,
                  void* ws, hipStream_t st) {
  const SelectPlan p = plan_select(n_q, n_kv, text_len, prompt_len, n_vis);
  char* base = static_cast<char*>(ws);
  double2* part = reinterpret_cast<double2*>(base + p.off_part);
  double* lse = reinterpret_cast<double*>(base + p.off_lse);
  double* colpart = reinterpret_cast<double*>(base + p.off_col);
  unsigned long long* keys = reinterpret_cast<unsigned long long*>(base + p.off_keys);
  unsigned* hist = reinterpret_cast<unsigned*>(base + p.off_hist);
  int2* counts = reinterpret_cast<int2*>(base + p.off_cnt);
  const int group = n_q / n_kv;
  const double scale = 1.0 / sqrt((double)D);
  const T* qt = static_cast<const T*>(q_text);
  const T* kk = static_cast<const T*>(k);
  hipLaunchKernelGGL((sel_rowstats_kernel<T>), dim3(p.n_kb, n_kv, p.n_rg1), dim3(P1_THREADS), 0, st, qt, kk, part, group,
                     text_len, prompt_len, text_start, k_hs, scale, p.kpb1, p.n_kb);
  int s = launch_status();
  if (s) return s;
  hipLaunchKernelGGL(sel_lse_kernel, dim3((n_kv * p.R + 255) / 256), dim3(256), 0, st, part, lse, p.R, p.n_kb, n_kv);
  if ((s = launch_status())) return s;
  hipLaunchKernelGGL((sel_colsum_kernel<T>), dim3(p.n_kb2, n_kv, p.n_rg2), dim3(P2_THREADS), 0, st, qt, kk, lse, colpart,
                     group, text_len, prompt_len, text_start, k_hs, scale, p.kpb2, n_kv);
  if ((s = launch_status())) return s;
  return launch_topk(colpart, p.n_rg2, n_kv, prompt_len, vis, n_vis, k_sel, topk_out, scores_out, keys, hist, counts,
                     st);
}

}  // namespace
}  // namespace stdhip

using namespace stdhip;

extern "C" size_t std_select_topk_workspace_bytes(int n_q, int n_kv, int text_len, int prompt_len, int n_visual,
                                                  int d) {
  if (d != D || n_q <= 0 || n_kv <= 0 || n_q % n_kv != 0 || text_len < 1 || prompt_len < text_len || n_visual < 1)
    return 0;
  return plan_select(n_q, n_kv, text_len, prompt_len, n_visual).total;
}

extern "C" int std_select_topk(const void* q_text, const void* k, int n_q, int n_kv, int text_len, int prompt_len,
                               int text_start, int d, long long k_head_stride, int dtype, const int32_t* visual_pos,
                               int n_visual, int k_select, int32_t* topk_out, double* scores_out, void* workspace,
                               size_t workspace_bytes, void* stream) {
  if (!q_text || !k || !visual_pos || !topk_out || !workspace) return STD_E_NULL;
  if (dtype != STD_F32 && dtype != STD_BF16 && dtype != STD_F16) return STD_E_DTYPE;
  if (!select_shape_ok(n_q, n_kv, text_len, prompt_len, text_start, d, n_visual, k_select)) return STD_E_SHAPE;
  if (n_kv > 1 && k_head_stride < (long long)prompt_len * D) return STD_E_SHAPE;
  if (workspace_bytes < plan_select(n_q, n_kv, text_len, prompt_len, n_visual).total) return STD_E_WORKSPACE;
  if (!aligned16(workspace) || !aligned16(k)) return STD_E_ALIGN;
  if ((k_head_stride * dtype_size(dtype)) % 16) return STD_E_ALIGN;   // 16-byte K row loads
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == STD_BF16)
    return launch_select<bf16_t>(q_text, k, n_q, n_kv, text_len, prompt_len, text_start, k_head_stride, visual_pos,
                                 n_visual, k_select, topk_out, scores_out, workspace, st);
  if (dtype == STD_F16)
    return launch_select<f16_t>(q_text, k, n_q, n_kv, text_len, prompt_len, text_start, k_head_stride, visual_pos,
                                n_visual, k_select, topk_out, scores_out, workspace, st);
  return launch_select<float>(q_text, k, n_q, n_kv, text_len, prompt_len, text_start, k_head_stride, visual_pos,
                              n_visual, k_select, topk_out, scores_out, workspace, st);
}

extern "C" int std_build_compact_index(const int32_t* non_visual, int n_nonvisual, const int32_t* topk, int k_select,
                                       int n_kv, int32_t* idx_out, void* stream) {
  if (!topk || !idx_out || (n_nonvisual > 0 && !non_visual)) return STD_E_NULL;
  if (n_nonvisual < 0 || k_select < 1 || n_kv < 1) return STD_E_SHAPE;
  const int total = n_nonvisual + k_select;
  hipLaunchKernelGGL(compact_index_kernel, dim3((total + 255) / 256, n_kv), dim3(256), 0,
                     static_cast<hipStream_t>(stream), non_visual, n_nonvisual, topk, k_select, idx_out);
  return launch_status();
}

extern "C" int std_compact_kv(const void* dense_k, const void* dense_v, void* sparse_k, void* sparse_v,
                              const int32_t* idx, int n_kv, int compact_len, int d, long long dense_head_stride,
                              int dense_rows, long long sparse_head_stride, int sparse_rows, int dtype,
                              void* stream) {
  if (!dense_k || !dense_v || !sparse_k || !sparse_v || !idx) return STD_E_NULL;
  if (dtype != STD_F32 && dtype != STD_BF16 && dtype != STD_F16) return STD_E_DTYPE;
  if (d != D || n_kv < 1 || compact_len < 1 || dense_rows < 1 || sparse_rows < 1) return STD_E_SHAPE;
  if (compact_len > sparse_rows) return STD_E_RANGE;
  const int es = dtype_size(dtype);
  if (!aligned16(dense_k) || !aligned16(dense_v) || !aligned16(sparse_k) || !aligned16(sparse_v)) return STD_E_ALIGN;
  if ((dense_head_stride * es) % 16 || (sparse_head_stride * es) % 16) return STD_E_ALIGN;
  const int row_bytes = D * es, cpr = row_bytes / 16;
  const long long chunks = (long long)compact_len * cpr;
  hipLaunchKernelGGL(compact_kv_kernel, dim3((unsigned)((chunks + 255) / 256), n_kv, 2), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const char*>(dense_k),
                     static_cast<const char*>(dense_v), static_cast<char*>(sparse_k), static_cast<char*>(sparse_v),
                     idx, compact_len, row_bytes, dense_head_stride * es, dense_rows, sparse_head_stride * es,
                     sparse_rows);
  return launch_status();
}

extern "C" size_t std_select_topk_probs_workspace_bytes(int n_q, int n_kv, int text_len, int prompt_len,
                                                        int n_visual) {
  if (n_q <= 0 || n_kv <= 0 || n_q % n_kv != 0 || text_len < 1 || prompt_len < 1 || n_visual < 1) return 0;
  return plan_probs(n_q, n_kv, text_len, prompt_len, n_visual).total;
}

extern "C" int std_select_topk_probs(const void* probs, long long head_stride, long long row_stride, int dtype,
                                     int n_q, int n_kv, int text_len, int prompt_len, const int32_t* visual_pos,
                                     int n_visual, int k_select, int32_t* topk_out, double* scores_out,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  if (!probs || !visual_pos || !topk_out || !workspace) return STD_E_NULL;
  if (dtype != STD_F32 && dtype != STD_BF16 && dtype != STD_F16) return STD_E_DTYPE;
  if (n_q <= 0 || n_kv <= 0 || n_q % n_kv != 0 || text_len < 1 || prompt_len < 1) return STD_E_SHAPE;
  if (n_visual < 1 || n_visual > prompt_len || k_select < 1 || k_select > n_visual) return STD_E_SHAPE;
  if (row_stride < prompt_len || head_stride < row_stride * text_len) return STD_E_SHAPE;
  if (workspace_bytes < plan_probs(n_q, n_kv, text_len, prompt_len, n_visual).total) return STD_E_WORKSPACE;
  // element-aligned probabilities; rows aligned to four elements take vector loads
  const int es = dtype == STD_F32 ? 4 : 2;
  if (!aligned16(workspace) || ((uintptr_t)probs % es) != 0) return STD_E_ALIGN;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == STD_F16)
    return launch_select_probs<f16_bits>(probs, head_stride, row_stride, n_q, n_kv, text_len, prompt_len, visual_pos,
                                         n_visual, k_select, topk_out, scores_out, workspace, st);
  if (dtype == STD_BF16)
    return launch_select_probs<bf16_t>(probs, head_stride, row_stride, n_q, n_kv, text_len, prompt_len, visual_pos,
                                       n_visual, k_select, topk_out, scores_out, workspace, st);
  return launch_select_probs<float>(probs, head_stride, row_stride, n_q, n_kv, text_len, prompt_len, visual_pos,
                                    n_visual, k_select, topk_out, scores_out, workspace, st);
}
