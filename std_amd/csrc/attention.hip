// GQA attention over a strided KV cache for the STD decode loop.
//
// One split-K kernel serves both the sparse draft / dense AR decode
// (q_len = 1) and the dense verify (q_len = gamma + 1, offset-causal): the
// n_q/n_kv query heads of a KV head and their q_len positions form R <= 128
// query rows that are carried through the key stream together, so each K/V
// row is read from HBM exactly once per launch (no repeat_kv, no per-head
// re-reads).
//
// Workgroup = (split of the key range, KV head), 4 wavefronts. K/V tiles of
// 64 keys are loaded with coalesced 16-byte loads (16 lanes per 256-byte bf16
// row), staged in LDS with register double buffering, and wave w owns keys
// [16w, 16w+16) of every tile. Scores are computed transposed, S^T = K Q^T,
// on 16x16 MFMA tiles, so a lane holds one query row and four keys: the
// online-softmax row statistics stay in-lane (two cross-lane max steps per
// tile), and the probabilities are already laid out as the B operand of the
// O^T += V^T P^T MFMA. The four waves' partial states are merged in LDS; with
// more than one split per head, (m, l, O) partials go to the workspace and a
// second kernel merges them in split order (deterministic).
#include <climits>

#include "common.h"

namespace stdhip {
namespace {

constexpr int D = kHeadDim;
constexpr int TK = 64;              // keys per LDS tile
constexpr int WAVES = 4;            // wave w owns keys [16w, 16w + 16) of each tile
constexpr int NTHREADS = 64 * WAVES;
constexpr int LROW = D + 4;         // LDS row pitch (elements) of staged K/V rows
constexpr int OROW = D + 4;         // LDS row pitch (floats) of the output merge
constexpr int kMaxRows = 128;       // R = (n_q / n_kv) * q_len limit (8 row tiles)
constexpr int kTargetWorkgroups = 512;

// MFMA fragments -------------------------------------------------------------
// Lane l = 16*lg + ln. A 16x16 fp32 accumulator tile holds C[4*lg + i][ln] in
// element i. For S^T = K Q^T the M index is the key (16 keys of the wave) and
// N the query row; for O^T = V^T P^T the M index is the head-dim row and N
// the query row. The contraction slots of A and B are paired identically, so
// any d-to-slot assignment is valid as long as A and B use the same one.
template <typename T> struct Frag;

template <> struct Frag<bf16_t> {
  // 16x16x16 bf16: each lane supplies 4 contraction elements.
  struct QFrag { i16x4 c[8]; };   // q[16c + 4lg + j]
  struct KFrag { i16x4 c[8]; };   // K[key][16c + 4lg + j]
  struct VFrag { i16x4 t[8]; };   // V[kb + 4lg + j][16t + ln]

  static __device__ __forceinline__ void load_q(QFrag& f, const bf16_t* row, int lg) {
#pragma unroll
    for (int c = 0; c < 8; ++c) f.c[c] = *(const i16x4*)(row + 16 * c + 4 * lg);
  }
  static __device__ __forceinline__ void zero_q(QFrag& f) {
#pragma unroll
    for (int c = 0; c < 8; ++c) f.c[c] = i16x4{0, 0, 0, 0};
  }
  static __device__ __forceinline__ void load_k(KFrag& f, const bf16_t* lrow, int lg) {
#pragma unroll
    for (int c = 0; c < 8; ++c) f.c[c] = *(const i16x4*)(lrow + 16 * c + 4 * lg);
  }
  static __device__ __forceinline__ void load_v(VFrag& f, const bf16_t* vt, int kb, int ln, int lg) {
    const bf16_t* base = vt + (kb + 4 * lg) * LROW + ln;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      f.t[t] = i16x4{(short)base[16 * t], (short)base[LROW + 16 * t],
                     (short)base[2 * LROW + 16 * t], (short)base[3 * LROW + 16 * t]};
    }
  }
  static __device__ __forceinline__ f32x4 qk(const KFrag& k, const QFrag& q) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 8; ++c) acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(k.c[c], q.c[c], acc, 0, 0, 0);
    return acc;
  }
  static __device__ __forceinline__ void pv(f32x4* acc, const VFrag& v, const float* p) {
    const i16x4 b = {(short)f32_to_bf16(p[0]), (short)f32_to_bf16(p[1]),
                     (short)f32_to_bf16(p[2]), (short)f32_to_bf16(p[3])};
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v.t[t], b, acc[t], 0, 0, 0);
  }
};

template <> struct Frag<float> {
  // 16x16x4 fp32: each lane supplies 1 contraction element per step.
  struct QFrag { float c[32]; };    // q[4c + lg]
  struct KFrag { float c[32]; };    // K[key][4c + lg]
  struct VFrag { float t[8][4]; };  // V[kb + 4lg + j][16t + ln]

  static __device__ __forceinline__ void load_q(QFrag& f, const float* row, int lg) {
#pragma unroll
    for (int c = 0; c < 32; ++c) f.c[c] = row[4 * c + lg];
  }
  static __device__ __forceinline__ void zero_q(QFrag& f) {
#pragma unroll
    for (int c = 0; c < 32; ++c) f.c[c] = 0.f;
  }
  static __device__ __forceinline__ void load_k(KFrag& f, const float* lrow, int lg) {
#pragma unroll
    for (int c = 0; c < 32; ++c) f.c[c] = lrow[4 * c + lg];
  }
  static __device__ __forceinline__ void load_v(VFrag& f, const float* vt, int kb, int ln, int lg) {
    const float* base = vt + (kb + 4 * lg) * LROW + ln;
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) f.t[t][j] = base[j * LROW + 16 * t];
  }
  static __device__ __forceinline__ f32x4 qk(const KFrag& k, const QFrag& q) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 32; ++c) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(k.c[c], q.c[c], acc, 0, 0, 0);
    return acc;
  }
  static __device__ __forceinline__ void pv(f32x4* acc, const VFrag& v, const float* p) {
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(v.t[t][j], p[j], acc[t], 0, 0, 0);
  }
};

template <typename T, int NT>
struct SplitSmem {
  static constexpr int kTileElems = TK * LROW;
  static constexpr int kKVBytes = 2 * 2 * kTileElems * (int)sizeof(T);   // K,V x double buffer
  // Query rows live in LDS (not registers) once the accumulators of NT row
  // tiles crowd the register file; bf16 only, fp32 would not fit in LDS.
  static constexpr bool kQLds = sizeof(T) == 2 && NT > 2;
  static constexpr int kQBytes = kQLds ? NT * 16 * LROW * (int)sizeof(T) : 0;
  static constexpr int kOBytes = NT * 16 * OROW * 4;
  static constexpr int kMLOff = kKVBytes + kQBytes > kOBytes ? kKVBytes + kQBytes : kOBytes;
  static constexpr int kBytes = kMLOff + (WAVES + 1) * NT * 16 * 8;
};

// grid (n_split, n_kv), block NTHREADS.
template <typename T, int NT>
__global__ void __launch_bounds__(NTHREADS)
attn_split_kernel(const T* __restrict__ q, const T* __restrict__ kc, const T* __restrict__ vc,
                  T* __restrict__ out, float* __restrict__ ws_o, float2* __restrict__ ws_ml,
                  int q_len, int kv_len, int group, long long k_hs, long long v_hs,
                  float scale_log2, int tiles_per_split, int n_split, int causal_off) {
  using F = Frag<T>;
  using S = SplitSmem<T, NT>;
  constexpr int EPC = 16 / (int)sizeof(T);      // elements per 16-byte chunk
  constexpr int CPR = D / EPC;                  // chunks per K/V row
  constexpr int CPT = TK * CPR / NTHREADS;      // chunks per thread per tile
  __shared__ __align__(16) unsigned char smem[S::kBytes];
  T* Ks = reinterpret_cast<T*>(smem);
  T* Vs = Ks + 2 * S::kTileElems;

  const int g = blockIdx.y, split = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  const int R = group * q_len;
  const int key_begin = split * tiles_per_split * TK;
  const int key_end = min(kv_len, key_begin + tiles_per_split * TK);
  const int ntiles = (key_end - key_begin + TK - 1) / TK;
  const T* kh = kc + (long long)g * k_hs;
  const T* vh = vc + (long long)g * v_hs;

  T* Qs = reinterpret_cast<T*>(smem + S::kKVBytes);                // [NT*16][LROW] if kQLds
  typename F::QFrag qf[S::kQLds ? 1 : NT];
  int lim[NT];
#pragma unroll
  for (int rt = 0; rt < NT; ++rt) {
    const int r = rt * 16 + ln;
    const int hl = r / q_len, i = r - hl * q_len;
    lim[rt] = r < R ? causal_off + i : INT_MAX;
    if constexpr (!S::kQLds) {
      if (r < R) F::load_q(qf[rt], q + ((long long)(g * group + hl) * q_len + i) * D, lg);
      else F::zero_q(qf[rt]);
    }
  }
  if constexpr (S::kQLds) {
    for (int c = tid; c < NT * 16 * CPR; c += NTHREADS) {
      const int r = c / CPR, col = c - r * CPR;
      uint4 val = make_uint4(0, 0, 0, 0);
      if (r < R) {
        const int hl = r / q_len, i = r - hl * q_len;
        val = *reinterpret_cast<const uint4*>(q + ((long long)(g * group + hl) * q_len + i) * D + col * EPC);
      }
      uint2* dq = reinterpret_cast<uint2*>(Qs + r * LROW + col * EPC);
      dq[0] = make_uint2(val.x, val.y);
      dq[1] = make_uint2(val.z, val.w);
    }
  }

  float m_run[NT], l_run[NT];
  f32x4 acc[NT][8];
#pragma unroll
  for (int rt = 0; rt < NT; ++rt) {
    m_run[rt] = -1e30f;
    l_run[rt] = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  uint4 kreg[CPT], vreg[CPT];
  auto gload = [&](int t) {
    const int base = key_begin + t * TK;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int c = tid + j * NTHREADS;
      const int row = c / CPR, col = c - row * CPR;
      const int key = base + row;
      if (key < key_end) {
        kreg[j] = *reinterpret_cast<const uint4*>(kh + (long long)key * D + col * EPC);
        vreg[j] = *reinterpret_cast<const uint4*>(vh + (long long)key * D + col * EPC);
      } else {
        kreg[j] = make_uint4(0, 0, 0, 0);
        vreg[j] = make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto lstore = [&](int buf) {
    T* kd = Ks + buf * S::kTileElems;
    T* vd = Vs + buf * S::kTileElems;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int c = tid + j * NTHREADS;
      const int row = c / CPR, col = c - row * CPR;
      uint2* pk = reinterpret_cast<uint2*>(kd + row * LROW + col * EPC);
      uint2* pv = reinterpret_cast<uint2*>(vd + row * LROW + col * EPC);
      pk[0] = make_uint2(kreg[j].x, kreg[j].y);
      pk[1] = make_uint2(kreg[j].z, kreg[j].w);
      pv[0] = make_uint2(vreg[j].x, vreg[j].y);
      pv[1] = make_uint2(vreg[j].z, vreg[j].w);
    }
  };

  gload(0);
  lstore(0);
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) gload(t + 1);
    const T* Kt = Ks + buf * S::kTileElems;
    const T* Vt = Vs + buf * S::kTileElems;
    const int tile_base = key_begin + t * TK;
    const bool need_mask = (tile_base + TK > key_end) || (tile_base + TK - 1 > causal_off);
    typename F::KFrag kf;
    typename F::VFrag vf;
    F::load_k(kf, Kt + (w * 16 + ln) * LROW, lg);
    F::load_v(vf, Vt, w * 16, ln, lg);
    const int key0 = tile_base + w * 16 + 4 * lg;
#pragma unroll
    for (int rt = 0; rt < NT; ++rt) {
      f32x4 s;
      if constexpr (S::kQLds) {
        typename F::QFrag qt;
        F::load_q(qt, Qs + (rt * 16 + ln) * LROW, lg);
        s = F::qk(kf, qt);
      } else {
        s = F::qk(kf, qf[rt]);
      }
      float sv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[i] = s[i] * scale_log2;
      if (need_mask) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = key0 + i;
          if (key >= key_end || key > lim[rt]) sv[i] = -INFINITY;
        }
      }
      float mt = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
      mt = fmaxf(mt, __shfl_xor(mt, 16));
      mt = fmaxf(mt, __shfl_xor(mt, 32));
      const float m_new = fmaxf(m_run[rt], mt);
      const float alpha = fast_exp2(m_run[rt] - m_new);
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = fast_exp2(sv[i] - m_new);
      l_run[rt] = l_run[rt] * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
      m_run[rt] = m_new;
#pragma unroll
      for (int d = 0; d < 8; ++d) acc[rt][d] *= alpha;
      F::pv(acc[rt], vf, p);
    }
    if (t + 1 < ntiles) lstore(buf ^ 1);
    __syncthreads();
  }

  // ---- merge the four waves (each saw a different quarter of every tile) ----
#pragma unroll
  for (int rt = 0; rt < NT; ++rt) {
    l_run[rt] += __shfl_xor(l_run[rt], 16);
    l_run[rt] += __shfl_xor(l_run[rt], 32);
  }
  float* So = reinterpret_cast<float*>(smem);                       // [NT*16][OROW]
  float2* ml_w = reinterpret_cast<float2*>(smem + S::kMLOff);       // [WAVES][NT*16]
  float2* ml_f = ml_w + WAVES * NT * 16;                            // [NT*16]
  if (lg == 0) {
#pragma unroll
    for (int rt = 0; rt < NT; ++rt) ml_w[w * NT * 16 + rt * 16 + ln] = make_float2(m_run[rt], l_run[rt]);
  }
  __syncthreads();
  float scl[NT];
#pragma unroll
  for (int rt = 0; rt < NT; ++rt) {
    const int r = rt * 16 + ln;
    float M = ml_w[r].x;
#pragma unroll
    for (int ww = 1; ww < WAVES; ++ww) M = fmaxf(M, ml_w[ww * NT * 16 + r].x);
    float L = 0.f;
#pragma unroll
    for (int ww = 0; ww < WAVES; ++ww) {
      const float2 ml = ml_w[ww * NT * 16 + r];
      L += ml.y * fast_exp2(ml.x - M);
    }
    scl[rt] = fast_exp2(m_run[rt] - M);
    if (w == 0 && lg == 0) ml_f[r] = make_float2(M, L);
  }
#pragma unroll
  for (int ww = 0; ww < WAVES; ++ww) {
    if (w == ww) {
#pragma unroll
      for (int rt = 0; rt < NT; ++rt) {
#pragma unroll
        for (int d = 0; d < 8; ++d) {
          f32x4* dst = reinterpret_cast<f32x4*>(So + (rt * 16 + ln) * OROW + 16 * d + 4 * lg);
          const f32x4 o = acc[rt][d] * scl[rt];
          if (ww == 0) *dst = o; else *dst += o;
        }
      }
    }
    __syncthreads();
  }

  for (int idx = tid; idx < R * (D / 4); idx += NTHREADS) {
    const int r = idx / (D / 4), d4 = idx - r * (D / 4);
    const f32x4 o = *reinterpret_cast<const f32x4*>(So + r * OROW + 4 * d4);
    const float2 ml = ml_f[r];
    if (n_split == 1) {
      const int hl = r / q_len, i = r - hl * q_len;
      T* dst = out + ((long long)(g * group + hl) * q_len + i) * D + 4 * d4;
#pragma unroll
      for (int e = 0; e < 4; ++e) dst[e] = from_f32<T>(o[e] / ml.y);
    } else {
      const long long row = (long long)(g * n_split + split) * R + r;
      *reinterpret_cast<f32x4*>(ws_o + row * D + 4 * d4) = o;
      if (d4 == 0) ws_ml[row] = ml;
    }
  }
}

// grid (R, n_kv), block D: combine the split partials of one query row.
template <typename T>
__global__ void __launch_bounds__(D)
attn_merge_kernel(const float* __restrict__ ws_o, const float2* __restrict__ ws_ml, T* __restrict__ out,
                  int n_split, int q_len, int group) {
  const int r = blockIdx.x, g = blockIdx.y, d = threadIdx.x;
  const int R = group * q_len;
  const long long base = (long long)g * n_split * R + r;
  float M = -1e30f;
  for (int s = 0; s < n_split; ++s) M = fmaxf(M, ws_ml[base + (long long)s * R].x);
  float L = 0.f, o = 0.f;
  for (int s = 0; s < n_split; ++s) {
    const long long row = base + (long long)s * R;
    const float2 ml = ws_ml[row];
    const float e = fast_exp2(ml.x - M);
    L += ml.y * e;
    o += ws_o[row * D + d] * e;
  }
  const int hl = r / q_len, i = r - hl * q_len;
  out[((long long)(g * group + hl) * q_len + i) * D + d] = from_f32<T>(o / L);
}

struct SplitPlan {
  int tiles_per_split;
  int n_split;
};

SplitPlan plan_splits(int n_kv, int kv_len) {
  const int ntiles = (kv_len + TK - 1) / TK;
  const int target = (kTargetWorkgroups + n_kv - 1) / n_kv;
  int tps = (ntiles + target - 1) / target;
  if (tps < 1) tps = 1;
  SplitPlan p;
  p.tiles_per_split = tps;
  p.n_split = (ntiles + tps - 1) / tps;
  return p;
}

size_t attn_workspace_bytes(int n_kv, int rows, int kv_len) {
  const SplitPlan p = plan_splits(n_kv, kv_len);
  if (p.n_split <= 1) return 0;
  const size_t n = (size_t)n_kv * p.n_split * rows;
  return round_up(n * D * sizeof(float), 256) + n * sizeof(float2);
}

template <typename T, int NT>
int launch_attn_t(const void* q, const void* k, const void* v, void* out, int n_kv, int q_len, int kv_len,
                  int group, long long k_hs, long long v_hs, float scale, void* ws, hipStream_t st) {
  const int R = group * q_len;
  const SplitPlan p = plan_splits(n_kv, kv_len);
  const size_t n = (size_t)n_kv * p.n_split * R;
  float* ws_o = static_cast<float*>(ws);
  float2* ws_ml = reinterpret_cast<float2*>(static_cast<char*>(ws) + round_up(n * D * sizeof(float), 256));
  const float scale_log2 = scale * 1.4426950408889634f;
  hipLaunchKernelGGL((attn_split_kernel<T, NT>), dim3(p.n_split, n_kv), dim3(NTHREADS), 0, st,
                     static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                     static_cast<T*>(out), ws_o, ws_ml, q_len, kv_len, group, k_hs, v_hs, scale_log2,
                     p.tiles_per_split, p.n_split, kv_len - q_len);
  int st0 = launch_status();
  if (st0 != 0 || p.n_split == 1) return st0;
  hipLaunchKernelGGL((attn_merge_kernel<T>), dim3(R, n_kv), dim3(D), 0, st, ws_o, ws_ml,
                     static_cast<T*>(out), p.n_split, q_len, group);
  return launch_status();
}

template <typename T>
int launch_attn(const void* q, const void* k, const void* v, void* out, int n_kv, int q_len, int kv_len,
                int group, long long k_hs, long long v_hs, float scale, void* ws, hipStream_t st) {
  const int nt = (group * q_len + 15) / 16;
  switch (nt) {
    case 1: return launch_attn_t<T, 1>(q, k, v, out, n_kv, q_len, kv_len, group, k_hs, v_hs, scale, ws, st);
    case 2: return launch_attn_t<T, 2>(q, k, v, out, n_kv, q_len, kv_len, group, k_hs, v_hs, scale, ws, st);
    case 3: return launch_attn_t<T, 3>(q, k, v, out, n_kv, q_len, kv_len, group, k_hs, v_hs, scale, ws, st);
    case 4: return launch_attn_t<T, 4>(q, k, v, out, n_kv, q_len, kv_len, group, k_hs, v_hs, scale, ws, st);
    case 5: return launch_attn_t<T, 5>(q, k, v, out, n_kv, q_len, kv_len, group, k_hs, v_hs, scale, ws, st);
    case 6: return launch_attn_t<T, 6>(q, k, v, out, n_kv, q_len, kv_len, group, k_hs, v_hs, scale, ws, st);
    case 7: return launch_attn_t<T, 7>(q, k, v, out, n_kv, q_len, kv_len, group, k_hs, v_hs, scale, ws, st);
    case 8: return launch_attn_t<T, 8>(q, k, v, out, n_kv, q_len, kv_len, group, k_hs, v_hs, scale, ws, st);
    default: return STD_E_SHAPE;
  }
}

int attn_entry(const void* q, const void* k, const void* v, void* out, int n_q, int n_kv, int q_len,
               int kv_len, int d, long long k_hs, long long v_hs, float scale, int dtype, void* ws,
               size_t ws_bytes, void* stream) {
  if (!q || !k || !v || !out) return STD_E_NULL;
  if (dtype != STD_F32 && dtype != STD_BF16) return STD_E_DTYPE;
  if (d != D || n_q <= 0 || n_kv <= 0 || n_q % n_kv != 0 || q_len < 1 || kv_len < q_len) return STD_E_SHAPE;
  const int group = n_q / n_kv;
  if ((long long)group * q_len > kMaxRows) return STD_E_SHAPE;
  const int es = dtype_size(dtype);
  if (k_hs < (long long)kv_len * D || v_hs < (long long)kv_len * D) return STD_E_SHAPE;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out)) return STD_E_ALIGN;
  if ((k_hs * es) % 16 != 0 || (v_hs * es) % 16 != 0) return STD_E_ALIGN;
  const size_t need = attn_workspace_bytes(n_kv, group * q_len, kv_len);
  if (need > 0 && (ws == nullptr || ws_bytes < need)) return STD_E_WORKSPACE;
  if (need > 0 && !aligned16(ws)) return STD_E_ALIGN;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == STD_BF16)
    return launch_attn<bf16_t>(q, k, v, out, n_kv, q_len, kv_len, group, k_hs, v_hs, scale, ws, st);
  return launch_attn<float>(q, k, v, out, n_kv, q_len, kv_len, group, k_hs, v_hs, scale, ws, st);
}

}  // namespace
}  // namespace stdhip

using namespace stdhip;

extern "C" size_t std_gqa_decode_workspace_bytes(int n_q, int n_kv, int kv_len, int d) {
  if (n_q <= 0 || n_kv <= 0 || n_q % n_kv != 0 || kv_len < 1 || d != D) return 0;
  return attn_workspace_bytes(n_kv, n_q / n_kv, kv_len);
}

extern "C" int std_gqa_decode(const void* q, const void* k, const void* v, void* out, int n_q, int n_kv,
                              int kv_len, int d, long long k_head_stride, long long v_head_stride, float scale,
                              int dtype, void* workspace, size_t workspace_bytes, void* stream) {
  return attn_entry(q, k, v, out, n_q, n_kv, 1, kv_len, d, k_head_stride, v_head_stride, scale, dtype,
                    workspace, workspace_bytes, stream);
}

extern "C" size_t std_verify_attn_workspace_bytes(int n_q, int n_kv, int q_len, int kv_len, int d) {
  if (n_q <= 0 || n_kv <= 0 || n_q % n_kv != 0 || q_len < 1 || kv_len < q_len || d != D) return 0;
  return attn_workspace_bytes(n_kv, (n_q / n_kv) * q_len, kv_len);
}

extern "C" int std_verify_attn(const void* q, const void* k, const void* v, void* out, int n_q, int n_kv,
                               int q_len, int kv_len, int d, long long k_head_stride, long long v_head_stride,
                               float scale, int dtype, void* workspace, size_t workspace_bytes, void* stream) {
  return attn_entry(q, k, v, out, n_q, n_kv, q_len, kv_len, d, k_head_stride, v_head_stride, scale, dtype,
                    workspace, workspace_bytes, stream);
}
