// GQA attention over a strided KV cache for the STD decode loop.
//
// One split-K design serves both the sparse draft / dense AR decode
// (q_len = 1) and the dense verify (q_len = gamma + 1, offset-causal): the
// n_q/n_kv query heads of a KV head and their q_len positions form R <= 96
// query rows that are carried through the key stream together, so each K/V
// row is read from HBM exactly once per launch (no repeat_kv, no per-head
// re-reads).
//
// Workgroup = (split of the key range, KV head). Four key-waves own keys
// [16w, 16w+16) of every 64-key tile; for verify-sized row counts a second
// group of four waves takes the other half of the row tiles, so that each
// SIMD runs two waves that hide each other's MFMA/LDS latency. Scores are computed transposed,
// S^T = K Q^T, on 16x16 MFMA tiles, so a lane holds one query row and four
// keys: the online-softmax row statistics stay in-lane, and the
// probabilities are already laid out as the B operand of O^T += V^T P^T.
//
// bf16 (the production path): K/V tiles stream HBM -> LDS through a 4-stage
// ring of global_load_lds_dwordx4 (no staging registers, three tiles in
// flight per workgroup). Rows are 256 bytes with their 16-byte chunks XOR
// swizzled so that the K operand reads (ds_read_b128, one key row per lane)
// and the V^T operand reads (ds_read_b64_tr_b16, four keys of one head-dim
// column per lane) are free of bank conflicts. QK^T uses 16x16x32 bf16 MFMA,
// PV 16x16x16 bf16 MFMA with fp32 accumulation.
// fp32: the same algorithm with register-staged LDS tiles and 16x16x4 fp32
// MFMA (exactness path for fp32 caches).
//
// Splits: the key tiles of a head are dealt round-robin to n_split workgroups;
// each merges its key-waves in LDS, then writes (m, l, O) partials that a
// merge kernel combines in split order, so results are deterministic. Merging
// inside the split launch was measured slower in every form tried (a
// last-arriving workgroup behind release fences, a grid barrier, merge
// workgroups appended to the grid reading agent-scope partials): carrying the
// partials across XCDs within a launch costs more than the second launch.
#include <algorithm>
#include <climits>
#include <mutex>
#include <type_traits>

#include "common.h"
#include "lds_dma.h"

// Timing build (STD_PHASE_STAMPS=1, a separate library that the measurement
// workload loads; the product library compiles none of this): each
// workgroup of the 16-bit attention kernels records s_memrealtime (a 100 MHz
// clock common to the whole chip) at its phases -- entry, first DMA issued,
// every tile barrier, loop end, end of its output stores -- and each merge
// block its entry and end.
#ifndef STD_PHASE_STAMPS
#define STD_PHASE_STAMPS 0
#endif
#if STD_PHASE_STAMPS
constexpr int kStampSlots = 48, kStampWgs = 2048, kStampMerge = 8192;
__device__ unsigned long long phase_stamps[kStampWgs * kStampSlots];
__device__ unsigned long long merge_stamps[kStampMerge * 2];
#endif

namespace stdhip {
namespace {

// Slots of a workgroup's stamp row: 0 entry, 1 first tiles issued, 2 + u the
// barrier of step u (u < 40), 43 compute loop done, 44/45 key-split waves'
// output stores begin/end, 46 the tile count, 47 row owners' output stores end.
__device__ __forceinline__ void stamp(int slot, unsigned long long v = 0) {
#if STD_PHASE_STAMPS
  const int wg = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
  if (wg < kStampWgs) phase_stamps[wg * kStampSlots + slot] = v ? v : __builtin_amdgcn_s_memrealtime();
#else
  (void)slot;
  (void)v;
#endif
}

constexpr int D = kHeadDim;
constexpr int TK = 64;              // keys per tile
constexpr int WAVES = 4;            // wave w owns keys [16w, 16w + 16) of each tile
constexpr int NTHREADS = 64 * WAVES;
constexpr int LROW = D + 4;         // LDS row pitch (elements) of register-staged K/V rows
constexpr int OROW = D + 4;         // LDS row pitch (floats) of the output merge
constexpr int OTILE_BYTES = 16 * OROW * 4;   // one 16-row tile of merged O
constexpr int kMaxRows = 96;        // R = (n_q / n_kv) * q_len limit (6 row tiles)
constexpr int kMaxSplit = 512;
constexpr float kRescaleSlack = 8.f; // bf16 path: raise the running max only past this (log2)

// ---------------------------------------------------------------------------
// Split plan and workspace layout (shared by host and device code).
struct SplitPlan {
  int ntiles;
  int n_split;
};

// Split-count model of the one-row-tile bf16 decode (fitted on MI355X to the
// key-split kernel, graph-replayed): a workgroup takes a 32 KiB tile step in
// 32 KiB / min(kCuGBs, kHbmGBs / workgroups) -- about 50 GB/s is what one
// such workgroup streams with a hundred others beside it (112 GB/s alone),
// and about 6.3 TB/s is shared by all -- and more than one split adds the
// merge launch with its partial round trip, kMergeUs.
constexpr double kCuGBs = 50.0;
constexpr double kHbmGBs = 6300.0;
constexpr double kMergeUs = 3.5;

// n_kv counts the launch's independent problems (KV heads x batch).
SplitPlan plan_splits(int n_kv, int rows, int kv_len, int dtype) {
  SplitPlan p;
  p.ntiles = (kv_len + TK - 1) / TK;
  const bool h16 = dtype == STD_BF16 || dtype == STD_F16;          // the 16-bit (bf16 / fp16) kernels
  const int target_wg = h16 ? 256 : 512;   // one LDS-heavy workgroup per CU
  int per_head = target_wg / n_kv;
  if (per_head < 1) per_head = 1;
  p.n_split = p.ntiles < per_head ? p.ntiles : per_head;
  // A decode over many problems (e.g. the 28 layers of one draft step in one
  // launch, 112 problems) or over few tiles streams each problem in one
  // workgroup when splitting saves less time than the merge costs.
  if (h16 && rows <= 16 && p.n_split > 1) {
    auto est_us = [&](int n) {
      const double rate = std::min(kCuGBs, kHbmGBs / ((double)n * n_kv));   // bytes per ns
      return (double)((p.ntiles + n - 1) / n) * (2.0 * TK * D * 2) / rate * 1e-3 + (n > 1 ? kMergeUs : 0.0);
    };
    if (est_us(1) <= est_us(p.n_split)) p.n_split = 1;
  }
  return p;
}

// Element strides between the independent problems of a batched launch
// (blockIdx.z); all zero for a single problem.
struct BatchStrides {
  long long q, k, v, o;
  long long w;          // partial rows per problem in the split workspace (set at launch)
};

// Index-addressed keys (decode, bf16): key j < n_idx of KV head g is row
// idx[g * idx_hs + j] of the dense cache (k, v with head strides k_hs, v_hs
// and dense_rows rows per head; an index outside [0, dense_rows) is clamped),
// keys j >= n_idx are rows j of the launch's own cache, as without indices.
// idx == nullptr: no gather. status: the optional device status word that a
// device length outside the launch's range marks (host side; the kernels
// receive GatherDev, with the index array as a separate argument).
struct GatherArgs {
  const int32_t* idx;
  long long idx_hs;
  int n_idx;
  int dense_rows;
  const bf16_t* k;
  const bf16_t* v;
  long long k_hs, v_hs;
  int32_t* status;
};

// The kernel-side auxiliary arguments of the non-collector kernels: the
// status word and GatherArgs' index parameters (same size as the index
// pointer it replaces: the argument block of these latency-bound launches
// stays at 248 bytes).
struct GatherDev {
  int32_t* status;
  long long idx_hs;
  int n_idx;
  int dense_rows;
  const bf16_t* k;
  const bf16_t* v;
  long long k_hs, v_hs;
};

// Visual-attention collector riding the verify pass (COLL): the group-mean
// query of each verify position, a softmax over the visual keys only, summed
// over the positions. The visual keys lie in [vis_begin, vis_end); with vmask
// == nullptr they are that whole range, otherwise key j is visual iff bit
// j % 32 of vmask[j / 32] is set (any ascending position set; vis_begin and
// vis_end are then its first position and last + 1). logits:
// [n_kv][n_vtiles][q_len][64] log2-domain scaled logits of the 64-key tiles
// that hold visual keys (tile vt = key / 64 - vis_begin / 64; -inf at
// non-visual keys), so that a split writes one contiguous block per tile;
// stats: [n_kv][n_split][q_len] per-split (max, sum of exp2(logit - max)).
// len_off: a device-length launch reads *len_dev + len_off cached keys (the
// positions before a chunk of verify rows, see verify_collect_entry).
struct CollArgs {
  float* logits;
  float2* stats;
  int n_vtiles;
  int vis_begin, vis_end;
  const uint32_t* vmask;
  int len_off;
  int32_t* status;
};

template <bool COLL>
using AuxArgs = typename std::conditional<COLL, CollArgs, GatherDev>::type;

struct WsLayout {
  size_t o_off, ml_off, total;
};

// part_bytes: 2 for scaled fp16 partials (bf16 launches with several row
// tiles), 4 for fp32 (part_bytes_of).
int part_bytes_of(int dtype, int rows) { return dtype == STD_BF16 && rows > 16 ? 2 : 4; }

WsLayout ws_layout(int n_kv, int rows, const SplitPlan& p, int part_bytes) {
  WsLayout l{0, 0, 0};
  if (p.n_split <= 1) return l;
  const size_t n = (size_t)n_kv * p.n_split * rows;
  l.o_off = 0;
  l.ml_off = round_up(l.o_off + n * D * part_bytes, 256);
  l.total = round_up(l.ml_off + n * sizeof(float2), 256);
  return l;
}

// A problem of at least kStreamTiles key tiles (4096 keys: 2 MiB of K and V
// per KV head) is read once per launch and not again before other data has
// passed through the caches -- a dense cache, or a compact cache of 4096 keys
// per head, whose 28 layers (235 MB) a model's weight stream evicts between
// two draft steps: its tiles are loaded non-temporally. Measured at 4096 keys
// (the 28-layer batched draft read cold): 42.3-42.9 -> 39.2-39.8 us; a round
// with nothing between its draft steps then loses the Infinity Cache's copy
// of that compact cache (3 % slower). The 1024-key compact cache (16 tiles)
// keeps the default policy.
constexpr int kStreamTiles = 64;
inline bool stream_keys(int ntiles) { return ntiles >= kStreamTiles; }

// Tiles are dealt to the splits of a head round-robin: split s streams tiles
// s, s + n_split, s + 2 n_split, ... so that at every step the workgroups of a
// head read neighbouring 16 KiB tiles, spread over the HBM channels. (One
// contiguous chunk per split puts 256 workgroups 512 KiB apart at 128k context;
// the same DMA ring then reads 10 % slower.)
__device__ __forceinline__ int split_ntiles(int split, int ntiles_total, int n_split) {
  return (ntiles_total - split + n_split - 1) / n_split;   // >= 0: split < n_split
}
__device__ __forceinline__ int tile_key0(int split, int tt, int n_split) { return (split + tt * n_split) * TK; }

// Device-length launch: the cache holds *len_dev rows plus this step's q_len
// new rows, and the grid was planned for kv_len (the launch's maximum). A
// length outside [0, kv_len - q_len] empties every split: nothing is read and
// the outputs become 0/0 = NaN.
__device__ __forceinline__ void device_length(const int32_t* len_dev, int q_len, int& kv_len, int& ntiles_total,
                                              int& causal_off, int len_off = 0) {
  const int len = *len_dev + len_off;
  kv_len = (len >= 0 && len <= kv_len - q_len) ? len + q_len : 0;
  ntiles_total = (kv_len + TK - 1) / TK;
  causal_off = kv_len - q_len;
}

// Fused append: cache rows [kv_len - n_new, kv_len) receive the n_new new
// rows (new_*[g][r], strides in elements). Each workgroup writes the rows of
// the tiles it streams, before it reads them (the caller puts a barrier
// between the two), so no other workgroup depends on these writes.
template <typename T>
__device__ void append_rows(T* __restrict__ kh, T* __restrict__ vh, const T* __restrict__ nk,
                            const T* __restrict__ nv, long long n_hs, long long n_rs, int g, int n_new, int kv_len,
                            int split, int n_split, int nthreads) {
  constexpr int EPC = 16 / (int)sizeof(T);
  constexpr int CPR = D / EPC;
  if (kv_len < n_new) return;
  const int first = kv_len - n_new;
  for (int idx = threadIdx.x; idx < n_new * CPR; idx += nthreads) {
    const int row = first + idx / CPR, col = idx % CPR;
    if ((row / TK) % n_split != split) continue;        // another split streams this tile
    const long long src = (long long)g * n_hs + (long long)(row - first) * n_rs + col * EPC;
    const uint4 k4 = *reinterpret_cast<const uint4*>(nk + src);
    const uint4 v4 = *reinterpret_cast<const uint4*>(nv + src);
    *reinterpret_cast<uint4*>(kh + (long long)row * D + col * EPC) = k4;
    *reinterpret_cast<uint4*>(vh + (long long)row * D + col * EPC) = v4;
  }
}

// ---------------------------------------------------------------------------
// Epilogue shared by both kernels: the key-waves' merged rows are in LDS
// (So(r) -> row r of O, unnormalised; ml_f[r] = (m, l), log2 domain).
template <typename T, typename OLoad>
__device__ void finish_split(OLoad load_o, const float2* ml_f, T* __restrict__ out, float* __restrict__ ws_o,
                             float2* __restrict__ ws_ml, int g, int split, int n_split, int q_len, int group,
                             int nthreads) {
  const int tid = threadIdx.x;
  const int R = group * q_len;
  const long long head_row0 = (long long)g * n_split * R;
  for (int idx = tid; idx < R * (D / 4); idx += nthreads) {
    const int r = idx / (D / 4), d4 = idx - r * (D / 4);
    const f32x4 o = load_o(r, d4);
    if (n_split == 1) {
      const float L = ml_f[r].y;
      const int hl = r / q_len, i = r - hl * q_len;
      T* dst = out + ((long long)(g * group + hl) * q_len + i) * D + 4 * d4;
#pragma unroll
      for (int e = 0; e < 4; ++e) dst[e] = from_f32<T>(o[e] / L);
    } else {
      const long long row = head_row0 + (long long)split * R + r;
      *reinterpret_cast<f32x4*>(ws_o + row * D + 4 * d4) = o;
      if (d4 == 0) ws_ml[row] = ml_f[r];
    }
  }
}

// Scaled fp16 partials (the bf16 kernels with several row tiles, i.e. verify):
// a split stores its unnormalised row O as P = O 2^-k in fp16, k chosen so
// that max|P| lies in [2^14, 2^15) (full fp16 precision, no overflow whatever
// the values), and (m, l) as (m + k, l 2^-k): weighted by 2^(m + k - M'), P
// contributes exactly what O contributes at 2^(m - M'), so the merge's
// arithmetic is the same as for fp32 partials, at half the bytes written and
// read back (128k verify: 9.3 -> 4.7 MB, 0.5 us less per layer). The decodes
// keep fp32 partials: their few partial bytes save nothing, and the row-max
// reduction lengthened the latency-bound launches (draft +0.35 us). fp16
// caches keep fp32 partials as well: their outputs have an fp16 partial's own
// precision, so its rounding would add up to half an output ulp.
typedef _Float16 half_t;
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int part_exp(float amax) {
  const int e = (int)((__float_as_uint(amax) >> 23) & 0xff) - 127;   // floor(log2 amax) for a normal amax
  return amax > 0.f ? min(max(e - 14, -100), 100) : 0;
}
__device__ __forceinline__ float exp2i(int k) { return __uint_as_float((uint32_t)(127 + k) << 23); }   // |k| <= 126

__device__ __forceinline__ f32x4 load_part(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ f32x4 load_part(const half_t* p) {
  return __builtin_convertvector(*reinterpret_cast<const half4_t*>(p), f32x4);
}

// Cross-lane max and sum of lanes l and l ^ 16 (xor16) or l and l ^ 32
// (xor32) through v_permlane16/32_swap: both lanes get (the value of the one
// with the bit clear) op (the value of the one with the bit set).
__device__ __forceinline__ float xor16_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
}
__device__ __forceinline__ float xor32_max(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
}
__device__ __forceinline__ float xor16_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}

// Merge, wave form (at most kWaveMergeMax splits: the draft's one-tile
// splits, short verifies): one wave per row. Lane (c, h) = (lane & 31,
// lane >> 5) owns columns 4c .. 4c + 3 and the splits h, h + 2, ..., h + 2(J-1)
// and issues all of their loads before the first use; loads past the last
// split fall outside a buffer resource bounded at it, which returns zeros
// without a memory access (re-reading the last split instead made the loads of
// one line wait on each other: 17 splits at J = 16 took the 1034-key draft from
// 7.4 to 7.8 us per layer). The two half-waves combine through one lane swap:
// no LDS, no barrier (1024-key draft, 16 splits: 7.19 -> 6.49 us per layer
// against the block form). Each half adds its splits in ascending order and
// the row is half 0's sum plus half 1's, so the result is deterministic.
constexpr int kWaveMergeMax = 32;
// J = splits per half-wave: ceil(n_split / 2) rounded up to an instantiated
// count (the draft's 1024-1033 keys give 16 or 17 splits: J = 8 or 9).
inline int merge_j(int n_split) {
  return n_split <= 8 ? 4 : n_split <= 16 ? 8 : n_split <= 18 ? 9 : n_split <= 24 ? 12 : 16;
}
constexpr int kBufWord3 = 0x00020000;     // raw buffer resource word 3 (gfx9 family)

template <typename T, typename PT, int J>
__device__ __forceinline__ void merge_row_wave(const PT* __restrict__ ws_o, const float2* __restrict__ ws_ml,
                                               T* __restrict__ out, int n_split, int q_len, int group,
                                               long long out_bs, int n_kv, int r, int g, int bz, int lane) {
  static_assert(2 * J <= kWaveMergeMax, "one pass covers every split");
  const int c = lane & 31, h = lane >> 5;
  const int R = group * q_len;
  out += bz * out_bs;
  const long long base = ((long long)bz * n_kv + g) * n_split * R + r;
  const uint32_t step_b = (uint32_t)(R * D * sizeof(PT));
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(ws_o + base * D), (short)0, (int)((n_split - 1) * step_b + D * sizeof(PT)), kBufWord3);
  const __amdgpu_buffer_rsrc_t rm = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(ws_ml + base), (short)0, (int)((n_split - 1) * R * 8 + 8), kBufWord3);
  float2 ml[J];
  f32x4 pv[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const uint32_t sp = h + 2 * j;
    ml[j] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rm, sp * R * 8, 0, 0));
    if constexpr (sizeof(PT) == 4)
      pv[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ro, sp * step_b + 16 * c, 0, 0));
    else
      pv[j] = __builtin_convertvector(
          __builtin_bit_cast(half4_t, __builtin_amdgcn_raw_buffer_load_b64(ro, sp * step_b + 8 * c, 0, 0)), f32x4);
  }
  float M = -1e30f, L = 0.f;
#pragma unroll
  for (int j = 0; j < J; ++j)
    if (h + 2 * j < n_split) M = fmaxf(M, ml[j].x);
  M = xor32_max(M);
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < J; ++j)
    if (h + 2 * j < n_split) {
      const float e = fast_exp2(ml[j].x - M);
      L += ml[j].y * e;
      o += pv[j] * e;
    }
  L = xor32_sum(L);
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = xor32_sum(o[e]);
  if (h == 0) {
    const int hl = r / q_len, i = r - hl * q_len;
    T* dst = out + ((long long)(g * group + hl) * q_len + i) * D + 4 * c;
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[e] = from_f32<T>(o[e] / L);
  }
}

// Merge, block form (more than kWaveMergeMax splits: long verifies and dense
// decodes): four waves per row, wave w taking the splits [w per, (w + 1) per)
// with per = ceil(n_split / 4), in passes of 16 laid out as in the wave form
// (buffer resources bounded at the wave's last split). Every wave first forms
// the row's maximum over all splits from one (m, l) load per lane and a
// 64-lane butterfly, so the four waves' sums share one scale; they are added
// in wave order through LDS after a single barrier. All of a wave's first
// pass goes out before the maximum is formed. (The previous form, eight split
// groups sharing weights through LDS with three barriers, spanned 3.1 us for
// the 128k verify's 280 rows.)
constexpr int kMergeThreads = 256;

template <typename T, typename PT>
__device__ __forceinline__ void merge_row_block(const PT* __restrict__ ws_o, const float2* __restrict__ ws_ml,
                                                T* __restrict__ out, int n_split, int q_len, int group,
                                                long long out_bs, int n_kv, int r, int g) {
  __shared__ f32x4 part[4][D / 4];
  __shared__ float lpart[4];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, h = lane >> 5;
  const int R = group * q_len;
  out += blockIdx.z * out_bs;
  const long long base = ((long long)blockIdx.z * n_kv + g) * n_split * R + r;
  const uint32_t step_b = (uint32_t)(R * D * sizeof(PT));
  const int per = (n_split + 3) / 4;
  const int s_beg = min(n_split, w * per), s_end = min(n_split, s_beg + per);
  const int n_w = s_end - s_beg;
  // this wave's splits (empty range: a resource of no records, every load zero)
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(ws_o + (base + (long long)s_beg * R) * D), (short)0,
      n_w > 0 ? (int)((n_w - 1) * step_b + D * sizeof(PT)) : 0, kBufWord3);
  const __amdgpu_buffer_rsrc_t rm = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(ws_ml + base + (long long)s_beg * R), (short)0, n_w > 0 ? (n_w - 1) * R * 8 + 8 : 0, kBufWord3);
  // all of the row's (m, l) pairs, for the maximum
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)(ws_ml + base), (short)0,
                                                                      (n_split - 1) * R * 8 + 8, kBufWord3);
  constexpr int J = 8;
  float2 ml[J];
  f32x4 pv[J];
  auto load = [&](int s0) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t sp = s0 + h + 2 * j;           // relative to s_beg
      ml[j] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rm, sp * R * 8, 0, 0));
      if constexpr (sizeof(PT) == 4)
        pv[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ro, sp * step_b + 16 * c, 0, 0));
      else
        pv[j] = __builtin_convertvector(
            __builtin_bit_cast(half4_t, __builtin_amdgcn_raw_buffer_load_b64(ro, sp * step_b + 8 * c, 0, 0)), f32x4);
    }
  };
  load(0);
  float M = -1e30f;
  for (int s = lane; s < n_split; s += 64)
    M = fmaxf(M, __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(ra, s * R * 8, 0, 0)).x);
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) M = fmaxf(M, __shfl_xor(M, off));
  M = xor32_max(xor16_max(M));
  float L = 0.f;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < n_w; s0 += 2 * J) {
    if (s0 > 0) load(s0);
#pragma unroll
    for (int j = 0; j < J; ++j)
      if (s0 + h + 2 * j < n_w) {
        const float e = fast_exp2(ml[j].x - M);
        L += ml[j].y * e;
        o += pv[j] * e;
      }
  }
  L = xor32_sum(L);
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = xor32_sum(o[e]);
  if (h == 0) part[w][c] = o;
  if (lane == 0) lpart[w] = L;
  __syncthreads();
  if (w == 0 && h == 0) {
    const f32x4 t = ((part[0][c] + part[1][c]) + part[2][c]) + part[3][c];
    const float Lt = ((lpart[0] + lpart[1]) + lpart[2]) + lpart[3];
    const int hl = r / q_len, i = r - hl * q_len;
    T* dst = out + ((long long)(g * group + hl) * q_len + i) * D + 4 * c;
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[e] = from_f32<T>(t[e] / Lt);
  }
}

// grid (R, n_kv, n_batch): block (r, g, b) merges row r of KV head g of
// problem b; J == 0: the block form (kMergeThreads threads), otherwise the
// wave form (one wave).
template <typename T, typename PT, int J>
__global__ void __launch_bounds__(J == 0 ? kMergeThreads : 64)
attn_merge_kernel(const PT* __restrict__ ws_o, const float2* __restrict__ ws_ml, T* __restrict__ out,
                  int n_split, int q_len, int group, long long out_bs, int n_kv) {
#if STD_PHASE_STAMPS
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
#endif
  if constexpr (J == 0)
    merge_row_block<T, PT>(ws_o, ws_ml, out, n_split, q_len, group, out_bs, n_kv, blockIdx.x, blockIdx.y);
  else
    merge_row_wave<T, PT, J>(ws_o, ws_ml, out, n_split, q_len, group, out_bs, n_kv, blockIdx.x, blockIdx.y,
                             blockIdx.z, threadIdx.x);
#if STD_PHASE_STAMPS
  const int b = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
  if (threadIdx.x == 0 && b < kStampMerge) {
    __builtin_amdgcn_s_waitcnt(0);
    merge_stamps[2 * b] = t0;
    merge_stamps[2 * b + 1] = __builtin_amdgcn_s_memrealtime();
  }
#endif
}

// Where the collector's per-key sums go: the visual keys' scores in position
// order (dynamic_selection.py:515 gathers key_states at visual_positions).
// vmask == nullptr: keys [vis_begin, vis_end), key j -> j - vis_begin;
// otherwise key j (bit j % 32 of vmask[j / 32] set) -> vrank[j / 32] + the
// set bits below it in its word; n_visual bounds every write. Keys at or past
// key_lim (the cached keys of a device-length launch) are never scored.
// accumulate: add to the scores instead of overwriting them (verify rows
// collected chunk by chunk, in row order).
struct CollOut {
  float* scores;
  long long score_hs;
  const uint32_t* vmask;
  const int32_t* vrank;
  int n_visual;
  const int32_t* len_dev;
  int len_off;
  int accumulate;
};

// Collector finish (the column sums of VerificationCollectorV3._hook,
// dynamic_selection.py:504-519), one 256-thread block per 16 visual tiles
// (1024 keys) of a KV head: thread t's four keys are columns 4 (t % 16) .. +3
// of visual tile 16 cb + t / 16. Every load is issued first: the thread's logits, then
// the split statistics of the rows its wave reduces (wave w: rows w, w + 4,
// ...; lane s: splits s, s + 64, ...). Each row's log-sum-exp is formed by a
// fixed butterfly, then the thread sums exp2(logit - lse) over the rows in
// row order.
__device__ __forceinline__ void coll_finish(const float* __restrict__ logits, const float2* __restrict__ stats,
                                            const CollOut co, int q_len, int n_split, int n_vtiles, int vis_begin,
                                            int vis_end, int cb, int g) {
  __shared__ float lse[16];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int vt = min(16 * cb + tid / 16, n_vtiles - 1), c = 4 * (tid % 16);
  const float* src = logits + ((long long)g * n_vtiles + vt) * q_len * TK + c;
  f32x4 z[16];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (i < q_len) z[i] = *reinterpret_cast<const f32x4*>(src + i * TK);
  float2 st[4][2];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int i = wv + 4 * r, sp = lane + 64 * h;
      st[r][h] = (i < q_len && sp < n_split) ? stats[((long long)g * n_split + sp) * q_len + i]
                                             : make_float2(-1e30f, 0.f);
    }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = wv + 4 * r;
    float m = fmaxf(st[r][0].x, st[r][1].x);
    float l = st[r][0].y * fast_exp2(st[r][0].x - m) + st[r][1].y * fast_exp2(st[r][1].x - m);
    for (int sp = lane + 128; sp < n_split; sp += 64) {       // more than 128 splits (fewer than 2 KV heads)
      const float2 v = stats[((long long)g * n_split + sp) * q_len + min(i, q_len - 1)];
      const float mm = fmaxf(m, v.x);
      l = l * fast_exp2(m - mm) + v.y * fast_exp2(v.x - mm);
      m = mm;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float mo = __shfl_xor(m, off), lo = __shfl_xor(l, off);
      const float mm = fmaxf(m, mo);
      l = l * fast_exp2(m - mm) + lo * fast_exp2(mo - mm);
      m = mm;
    }
    if (lane == 0 && i < q_len) lse[i] = m + __log2f(l);
  }
  __syncthreads();
  // The four keys' score slots (-1: not scored). They share one mask word.
  const bool live = 16 * cb + tid / 16 < n_vtiles;
  float* dst = co.scores + (long long)g * co.score_hs;
  const int key0 = (vis_begin / TK + vt) * TK + c;
  const int key_lim = co.len_dev != nullptr ? min(vis_end, *co.len_dev + co.len_off) : vis_end;
  uint32_t word = 0;
  int rank0 = 0;
  if (live && co.vmask != nullptr && key0 < vis_end) {
    word = co.vmask[key0 >> 5];
    rank0 = co.vrank[key0 >> 5];
  }
  int slot[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int key = key0 + e;
    int sl = key - vis_begin;
    if (co.vmask != nullptr) {
      const int bit = key & 31;
      sl = ((word >> bit) & 1u) ? rank0 + __popc(word & ((1u << bit) - 1u)) : -1;
    }
    slot[e] = (live && key >= vis_begin && key < key_lim && sl >= 0 && sl < co.n_visual) ? sl : -1;
  }
  // Sum over the rows in row order, continuing from the earlier chunks' sum
  // when accumulating (so chunked rows fold exactly as one pass would).
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (co.accumulate) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (slot[e] >= 0) acc[e] = dst[slot[e]];
  }
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (i < q_len) {
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] += fast_exp2(z[i][e] - lse[i]);
    }
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (slot[e] >= 0) dst[slot[e]] = acc[e];
}

// The verify merge and the collector finish in one launch: grid
// (n_row_blocks + n_col_blocks, n_kv). The first n_row_blocks blocks merge
// the attention rows (none when the verify ran as one split): one row per
// block in the block form (J == 0, n_row_blocks = n_rows), otherwise one per
// wave (n_row_blocks = (n_rows + 3) / 4, row 4x + w). The other blocks finish
// 1024 visual keys each.
template <typename T, typename PT, int J>
__global__ void __launch_bounds__(kMergeThreads)
merge_coll_kernel(const PT* __restrict__ ws_o, const float2* __restrict__ ws_ml, T* __restrict__ out,
                  int n_split, int q_len, int group, int n_rows, const float* __restrict__ logits,
                  const float2* __restrict__ stats, CollOut co, int n_vtiles, int vis_begin, int vis_end) {
  static_assert(kMergeThreads == 256, "the collector finish runs 256 threads");
#if STD_PHASE_STAMPS
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
#endif
  const int n_row_blocks = J == 0 ? n_rows : (n_rows + 3) / 4;
  if ((int)blockIdx.x < n_row_blocks) {
    if constexpr (J == 0) {
      merge_row_block<T, PT>(ws_o, ws_ml, out, n_split, q_len, group, 0LL, gridDim.y, blockIdx.x, blockIdx.y);
    } else {
      const int r = 4 * blockIdx.x + (threadIdx.x >> 6);
      if (r < n_rows)
        merge_row_wave<T, PT, J>(ws_o, ws_ml, out, n_split, q_len, group, 0LL, gridDim.y, r, blockIdx.y, 0,
                                 threadIdx.x & 63);
    }
  } else {
    coll_finish(logits, stats, co, q_len, n_split, n_vtiles, vis_begin, vis_end, blockIdx.x - n_row_blocks,
                blockIdx.y);
  }
#if STD_PHASE_STAMPS
  const int b = blockIdx.y * gridDim.x + blockIdx.x;
  if (threadIdx.x == 0 && b < kStampMerge) {
    __builtin_amdgcn_s_waitcnt(0);
    merge_stamps[2 * b] = t0;
    merge_stamps[2 * b + 1] = __builtin_amdgcn_s_memrealtime();
  }
#endif
}

// ===========================================================================
// bf16 kernel: DMA ring + swizzled LDS + MFMA.
constexpr int NSTAGE = 4;
constexpr int ROWB = D * 2;               // bytes per bf16 row
constexpr int TILEB = TK * ROWB;          // 16 KiB of K (or V) per tile
constexpr int STAGEB = 2 * TILEB;         // K then V

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef short i16x8 __attribute__((ext_vector_type(8)));

// 16-byte chunk c of row r lives at chunk c ^ swz(r): sixteen consecutive
// rows map one logical chunk to sixteen distinct positions (K reads), and
// four consecutive rows map a chunk pair to eight (V transpose reads).
__device__ __forceinline__ int swz(int row) { return ((row & 7) << 1) | ((row >> 3) & 1); }
__device__ __forceinline__ int sw_off(int row, int chunk) { return row * ROWB + ((chunk ^ swz(row)) << 4); }

// Four floats -> four bf16 (RNE); the two-wide conversions compile to
// v_cvt_pk_bf16_f32.
__device__ __forceinline__ i16x4 pack_bf16x4(float a, float b, float c, float d) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  const uint32_t lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
  const uint32_t hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{c, d}, bf16x2_t));
  return __builtin_bit_cast(i16x4, (uint64_t)lo | ((uint64_t)hi << 32));
}

// The 16-bit element arithmetic of the bf16 kernels, for bf16 (bf16_t) or
// fp16 (f16_t) caches: the MFMA operand vectors, QK^T / PV MFMAs of 32 and
// 16 contraction elements, the packing of four floats (probabilities, output
// rows; round to nearest even), the element 1.0, one element's bit pattern
// to fp32, and the split of an fp32 value into a 16-bit head and remainder.
// Storage is the 16-bit pattern either way, so loads, the DMA ring and the
// appends are shared.
template <typename E> struct Elem;
template <> struct Elem<bf16_t> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  typedef short v4 __attribute__((ext_vector_type(4)));
  static constexpr short kOne = 0x3f80;
  static __device__ __forceinline__ f32x4 mma32(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16(v4 a, v4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ i16x4 pack4(float a, float b, float c, float d) { return pack_bf16x4(a, b, c, d); }
  static __device__ __forceinline__ float to_f32(uint32_t bits) { return bf16_to_f32(bits); }
  static __device__ __forceinline__ void split(float m, short& hi, short& lo) {
    const uint32_t h = f32_to_bf16(m);
    hi = (short)h;
    lo = (short)f32_to_bf16(m - bf16_to_f32(h));
  }
};
template <> struct Elem<f16_t> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  typedef _Float16 v4 __attribute__((ext_vector_type(4)));
  static constexpr short kOne = 0x3c00;
  static __device__ __forceinline__ f32x4 mma32(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16(v4 a, v4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ i16x4 pack4(float a, float b, float c, float d) {
    return __builtin_bit_cast(i16x4, __builtin_convertvector(f32x4{a, b, c, d}, v4));
  }
  static __device__ __forceinline__ float to_f32(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
  }
  // The head comes from one conversion instruction (round toward zero) and
  // the remainder is taken against that same value. Written as two plain
  // fp16 roundings, the compiler formed the head twice, once from the fp32
  // product and once inside a mixed-precision FMA from the exact product, and
  // where the two differed head + remainder was off by a whole fp16 ulp.
  static __device__ __forceinline__ void split(float m, short& hi, short& lo) {
    const auto h2 = __builtin_amdgcn_cvt_pkrtz(m, 0.f);
    hi = __builtin_bit_cast(short, h2[0]);
    lo = __builtin_bit_cast(short, (_Float16)(m - (float)h2[0]));
  }
};


// Row-owner layout: compute wave w < NT owns query rows [16w, 16w + 16) of the
// launch's R rows and processes all 64 keys of every tile, so at the end of
// its key range a wave holds complete row statistics and output rows and
// writes them straight from registers (no cross-wave merge, no LDS epilogue).
// Waves w >= NT only help issue the DMA ring. Decode (NT == 1) runs four
// waves, verify eight. KS (key split, NT == 1 only) instead lets all four
// waves compute, each on its own 16 keys of every tile, and merges them at
// the end; it pays once a workgroup streams several tiles.
template <int NT>
struct Bf16Cfg {
  static constexpr int kWaves = NT == 1 ? 4 : 8;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kSegsPerWave = 16 / kWaves;       // 1 KiB K segments (and V) per wave per tile
  static constexpr int kLoadsPerTile = 2 * kSegsPerWave;
};

// Split partials: scaled fp16 for the bf16 launches with several row tiles
// (verify), whose 8-bit outputs are far coarser than an fp16 partial; fp32
// otherwise -- the decodes, and fp16 caches, whose outputs carry as many
// significand bits as an fp16 partial would.
template <int NT, typename E>
using PartT = typename std::conditional<(NT > 1) && std::is_same<E, bf16_t>::value, half_t, float>::type;

template <int NT, bool KS, bool GA, bool COLL = false, typename E = bf16_t, bool STREAM = false>
__global__ void __launch_bounds__(NT == 1 ? 256 : 512)
attn_bf16_kernel(const bf16_t* __restrict__ q, bf16_t* __restrict__ kc, bf16_t* __restrict__ vc,
                 bf16_t* __restrict__ out, PartT<NT, E>* __restrict__ ws_o, float2* __restrict__ ws_ml, int q_len,
                 int kv_len, int group, long long k_hs, long long v_hs, float scale_log2, int ntiles_total,
                 int n_split, int causal_off, const bf16_t* __restrict__ new_k, const bf16_t* __restrict__ new_v,
                 long long n_hs, long long n_rs, int n_new, BatchStrides bs, const int32_t* __restrict__ len_dev,
                 AuxArgs<COLL> ga, const int32_t* __restrict__ gidx) {
  using C = Bf16Cfg<NT>;
  using EL = Elem<E>;
  using v8 = typename EL::v8;                    // 8 elements: the 16x16x32 MFMA operands
  using v4 = typename EL::v4;                    // 4 elements: the 16x16x16 MFMA operands
  __shared__ __align__(16) char ring[NSTAGE * STAGEB];
  // With the collector the query rows are staged in LDS by the ring's DMA
  // (its group means read every row of the group): 1.7 us less per 128k
  // verify than loading them through registers; without it the rows are read
  // once and go straight to registers.
  constexpr bool kQLds = COLL;
  __shared__ __align__(16) char qs[kQLds ? 16 * NT * ROWB : 16];
  // Collector: the group-mean query rows, 16-bit heads (rows 0..15) then
  // remainders (rows 16..31), in the swizzled row layout of qs.
  __shared__ __align__(16) char qm[COLL ? 2 * 16 * ROWB : 16];

#if STD_PHASE_STAMPS
  const unsigned long long t_entry = __builtin_amdgcn_s_memrealtime();
#endif
  const int g = blockIdx.y, split = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
#if STD_PHASE_STAMPS
  if (tid == 0) stamp(0, t_entry);
#endif
  // Wave roles. Key split (KS, one row tile): every wave computes, on its own
  // 16 keys of each tile. Otherwise waves w < NT own one 16-row tile each
  // (row owners) and the rest only help issue the DMA ring -- except with
  // five row tiles (HYB, the 70-row verify), where waves 0-3 own row tiles
  // 0-3 and waves 4-7, one per SIMD, share row tile 4 by keys as in the key
  // split, so that no SIMD carries two row tiles.
  static_assert(!KS || NT == 1, "the key split serves one row tile");
  static_assert(!COLL || (NT == 5 && !KS && !GA), "the collector rides the five-row-tile verify layout");
  constexpr bool HYB = NT == 5 && !KS;
  constexpr int kOwners = HYB ? 4 : NT;
  const bool computes = !KS && w < kOwners;     // row owner (wave-uniform)
  const bool ksw = KS || (HYB && w >= 4);       // key-split wave (wave-uniform)
  const int ks_sub = KS ? w : w - 4;            // its 16 keys of each tile: 16 ks_sub ...
  const int ln = lane & 15, lg = lane >> 4;
  const int R = group * q_len;
  {
    const long long b = blockIdx.z;
    q += b * bs.q;
    kc += b * bs.k;
    vc += b * bs.v;
    out += b * bs.o;
    if (n_split > 1) {
      ws_o += b * bs.w * D;
      ws_ml += b * bs.w;
    }
  }
  if (len_dev != nullptr) {
    if constexpr (COLL)
      device_length(len_dev, q_len, kv_len, ntiles_total, causal_off, ga.len_off);
    else
      device_length(len_dev, q_len, kv_len, ntiles_total, causal_off);
    if (kv_len == 0 && tid == 0 && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0) flag_overflow(ga.status);
  }
  const int ntiles = split_ntiles(split, ntiles_total, n_split);
  bf16_t* kh = kc + (long long)g * k_hs;
  bf16_t* vh = vc + (long long)g * v_hs;
  if (n_new > 0) {
    append_rows<bf16_t>(kh, vh, new_k, new_v, n_hs, n_rs, g, n_new, kv_len, split, n_split, C::kThreads);
    __syncthreads();
  }

  // Each issuing wave DMAs kSegs 1 KiB segments (4 rows) of K and of V per
  // tile. Lane l fills row 4*seg + l/16 at physical chunk l%16, i.e. logical
  // chunk (l%16) ^ swz(row). Rows past the cache's last key re-read that key
  // (their scores are masked), so no read leaves the valid range.
  // With the collector, only waves 0-3 issue the ring (four segments each):
  // the key-split waves then keep no loads of the ring in flight, so their
  // logit stores never enter a ring wait count, and they need no ring wait at
  // all (the barrier that follows the issuing waves' waits orders each tile).
  constexpr int kDmaWaves = COLL ? 4 : C::kWaves;
  constexpr int kSegs = 16 / kDmaWaves;
  constexpr int kLoads = 2 * kSegs;
  const bool dma_wave = w < kDmaWaves;
  int dma_row[kSegs], dma_chunk[kSegs];
#pragma unroll
  for (int j = 0; j < kSegs; ++j) {
    const int seg = w * kSegs + j;
    dma_row[j] = seg * 4 + (lane >> 4);
    dma_chunk[j] = ((lane & 15) ^ swz(dma_row[j])) * 16;
  }
  auto issue = [&](int tt, char* stage) {
    if (!dma_wave) return;
    const int key0 = tile_key0(split, tt, n_split);
    const int last = min(kv_len - key0, TK) - 1;       // wave-uniform
    if constexpr (GA) {
      static_assert(NT == 1, "gathered keys serve the single-row decode");
      if (key0 < ga.n_idx) {                             // wave-uniform: a tile with gathered keys
        // This wave's DMA rows are 4 kSegs consecutive rows from wrow0;
        // their indices come through scalar loads (gidx is read-only and not
        // aliased, so the compiler can use them; they are counted apart from
        // the ring's vector-memory count), then each lane copies from its row's
        // own address: gathered dense row or own-cache row.
        constexpr int kRows = 4 * kSegs;
        const int wrow0 = w * kRows;
        int sidx[kRows];
        if (key0 + wrow0 < ga.n_idx) {
          const int4* ip = reinterpret_cast<const int4*>(gidx + g * ga.idx_hs + key0 + wrow0);
#pragma unroll
          for (int i = 0; i < kRows / 4; ++i) {
            const int4 v4 = ip[i];
            sidx[4 * i] = v4.x;
            sidx[4 * i + 1] = v4.y;
            sidx[4 * i + 2] = v4.z;
            sidx[4 * i + 3] = v4.w;
          }
        } else {
#pragma unroll
          for (int i = 0; i < kRows; ++i) sidx[i] = 0;
        }
        const char* gkh = reinterpret_cast<const char*>(ga.k + g * ga.k_hs);
        const char* gvh = reinterpret_cast<const char*>(ga.v + g * ga.v_hs);
        // Rows past the cache's last key re-read that key from where it really
        // lives (a gathered dense row or an own-cache row), as the compacted
        // cache would: own-cache rows below n_idx are never written.
        const int klast = key0 + last;
        const char *lk, *lv;
        if (klast < ga.n_idx) {
          const int il = min(max(gidx[g * ga.idx_hs + klast], 0), ga.dense_rows - 1);
          lk = gkh + (long long)il * ROWB;
          lv = gvh + (long long)il * ROWB;
        } else {
          lk = reinterpret_cast<const char*>(kh + (long long)klast * D);
          lv = reinterpret_cast<const char*>(vh + (long long)klast * D);
        }
        const int sel = lane >> 4;
#pragma unroll
        for (int j = 0; j < kSegs; ++j) {
          const int r = dma_row[j];
          const int key = key0 + r;
          int ix = sel == 0 ? sidx[4 * j] : sel == 1 ? sidx[4 * j + 1] : sel == 2 ? sidx[4 * j + 2] : sidx[4 * j + 3];
          ix = min(max(ix, 0), ga.dense_rows - 1);
          const char *ka, *va;
          if (r > last) {
            ka = lk;
            va = lv;
          } else if (key < ga.n_idx) {
            ka = gkh + (long long)ix * ROWB;
            va = gvh + (long long)ix * ROWB;
          } else {
            ka = reinterpret_cast<const char*>(kh + (long long)key * D);
            va = reinterpret_cast<const char*>(vh + (long long)key * D);
          }
          const uint32_t dst = lds_addr(stage) + (w * kSegs + j) * 1024;
          lds_dma16_vaddr(ka + dma_chunk[j], dst);
          lds_dma16_vaddr(va + dma_chunk[j], dst + TILEB);
        }
        return;
      }
    }
    const bf16_t* kt = kh + (long long)key0 * D;
    const bf16_t* vt = vh + (long long)key0 * D;
#pragma unroll
    for (int j = 0; j < kSegs; ++j) {
      const uint32_t off = (uint32_t)(min(dma_row[j], last) * ROWB + dma_chunk[j]);
      const uint32_t dst = lds_addr(stage) + (w * kSegs + j) * 1024;
      lds_dma16_sbase<STREAM>(kt, off, dst);
      lds_dma16_sbase<STREAM>(vt, off, dst + TILEB);
    }
  };

  // The first two tiles are in flight while the query rows are loaded. With
  // kQLds the rows go to LDS by DMA ahead of the tiles, and the wait below
  // covers only them (loads complete in issue order), so that the collector's
  // group means are formed while tiles 0 and 1 are still in flight; waiting
  // for tile 0 as well put that work between the tile's arrival and the next
  // DMA issue (first tile at the barrier 7.2-8.2 us instead of 3.9 us, 128k
  // keys).
  auto stage = [&](int u) { return ring + (u & (NSTAGE - 1)) * STAGEB; };
  if (kQLds && dma_wave) {
    const bf16_t* qh = q + (long long)g * R * D;         // the R rows of KV head g are contiguous
    const int nseg = (R + 3) / 4;                           // 1 KiB segments of four rows
    for (int sg = w; sg < nseg; sg += kDmaWaves) {
      const int r = 4 * sg + (lane >> 4);
      const uint32_t off = (uint32_t)(min(r, R - 1) * ROWB + (((lane & 15) ^ swz(r)) << 4));
      lds_dma16_sbase(qh, off, lds_addr(qs) + sg * 1024);
    }
  }
  if (ntiles > 0) issue(0, stage(0));
  if (ntiles > 1) issue(1, stage(1));
#if STD_PHASE_STAMPS
  if (tid == 0) stamp(1);
#endif
  if constexpr (kQLds) {
    if (dma_wave) wait_vm_ahead<kLoads>(min(2, ntiles));      // the tiles issued may still be in flight
    wg_barrier();
  }

  // This wave's query row is the lane's column ln of the S^T tiles; padding
  // rows (and the helper waves) carry zero queries and are never written.
  const int row = KS ? ln : ksw ? 16 * kOwners + ln : w * 16 + ln;
  const bool row_ok = (computes || ksw) && row < R;
  const int lim = row_ok ? causal_off + (row % q_len) : INT_MAX;
  // Q^T operand, 32-wide chunk c: lane (ln, lg) holds q[row][32c + 8lg, +8).
  v8 qf[4];
  if (row_ok) {
    if constexpr (kQLds) {
#pragma unroll
      for (int c = 0; c < 4; ++c) qf[c] = *reinterpret_cast<const v8*>(qs + sw_off(row, 4 * c + lg));
    } else {
      const int hl = row / q_len, i = row - hl * q_len;
      const bf16_t* qrow = q + ((long long)(g * group + hl) * q_len + i) * D;
#pragma unroll
      for (int c = 0; c < 4; ++c) qf[c] = *reinterpret_cast<const v8*>(qrow + 32 * c + 8 * lg);
    }
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) qf[c] = v8{};
  }
  // Collector rows: lanes q_off .. 15 of the key-split waves (the padding rows
  // of the last row tile, R + q_len <= 80) carry position i = ln - q_off's
  // group-mean query, the fp32 mean of the group's 16-bit query rows
  // (modeling_qwen2_5_vl.py hook -> dynamic_selection.py:509-512), split into
  // a 16-bit head qf and a 16-bit remainder qlo (bf16 or fp16, as the cache),
  // so that K.qf + K.qlo carries the mean's precision through the MFMAs.
  // The whole workgroup forms the means, one (position, 16-byte chunk) item
  // per thread, into qm, and the collector lanes read their operands from it:
  // done by the four key-split waves alone, each lane unrolled over its four
  // chunks, this ran about 1.5 KB of code that every CU fetched cold before
  // its first tile step (first tile at 7.7 instead of 3.9 us, 128k keys).
  const int q_off = 16 - q_len;
  v8 qlo[4];
  if constexpr (COLL) {
    for (int t = tid; t < 16 * q_len; t += C::kThreads) {
      const int i = t >> 4, ch = t & 15;
      float m8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int hl = 0; hl < group; ++hl) {
        const uint4 raw = *reinterpret_cast<const uint4*>(qs + sw_off(hl * q_len + i, ch));
        const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          m8[2 * e] += EL::to_f32(w4[e] & 0xffffu);
          m8[2 * e + 1] += EL::to_f32(w4[e] >> 16);
        }
      }
      const float inv = 1.f / (float)group;
      i16x8 hi, lo;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        short h, l;
        EL::split(m8[e] * inv, h, l);
        hi[e] = h;
        lo[e] = l;
      }
      *reinterpret_cast<i16x8*>(qm + sw_off(i, ch)) = hi;
      *reinterpret_cast<i16x8*>(qm + sw_off(16 + i, ch)) = lo;
    }
    // The means are in LDS before any lane reads them; the ring's DMA stays
    // in flight (no vector-memory wait).
    __builtin_amdgcn_s_waitcnt(waitcnt_lgkm0());
    wg_barrier();
#pragma unroll
    for (int c = 0; c < 4; ++c) qlo[c] = v8{};
    if (ksw && ln >= q_off) {
      const int i = ln - q_off;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        qf[c] = *reinterpret_cast<const v8*>(qm + sw_off(i, 4 * c + lg));
        qlo[c] = *reinterpret_cast<const v8*>(qm + sw_off(16 + i, 4 * c + lg));
      }
    }
  }
  float m_c = -1e30f, l_c = 0.f;       // collector row statistics of this lane's keys (log2 domain)
  // With a visual mask, lane t of a key-split wave holds the 16 mask bits of
  // the wave's keys in the split's tile t (t < 64; later tiles load theirs).
  uint32_t vbits = 0;
  if constexpr (COLL) {
    if (ksw && ga.vmask != nullptr && lane < ntiles) {
      const int kb = tile_key0(split, lane, n_split) + 16 * ks_sub;
      if (kb < ga.vis_end && kb + 16 > ga.vis_begin) vbits = (ga.vmask[kb >> 5] >> (kb & 31)) & 0xffffu;
    }
  }
  // Retire the query loads (and with them the two ring tiles issued before
  // them) here: the compiler counts only its own loads, and a wait for them
  // placed inside the loop would drain the ring there. (With kQLds there are
  // none: the rows came through the ring's DMA.)
  if constexpr (!kQLds) __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  // The key split runs QK^T and PV of a tile in the same step, so only one
  // stage is held by compute and three tiles stay in flight; the first of
  // them is issued here.
  if (KS && ntiles > 2) issue(2, stage(2));

  // Running statistics in the log2 domain (scores pre-multiplied by
  // scale*log2(e)): m_run is the row's running max; the row sum is
  // accumulated by an MFMA against a ones operand (every element of lsum
  // equals the row sum of the bf16 probabilities used for PV).
  float m_run = -1e30f;
  f32x4 acc[8], lsum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const v8 ones = __builtin_bit_cast(v8, i16x8{EL::kOne, EL::kOne, EL::kOne, EL::kOne, EL::kOne, EL::kOne, EL::kOne,
                                               EL::kOne});

  // S^T sub-tile j (keys 16j..16j+15 of the tile): lane (ln, lg) element i is
  // key 16j + 4lg + i of query row ln.
  auto qk = [&](const char* st, f32x4* s) {
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      v8 kf[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) kf[j] = *reinterpret_cast<const v8*>(st + sw_off(16 * j + ln, 4 * c + lg));
#pragma unroll
      for (int j = 0; j < 4; ++j) s[j] = EL::mma32(kf[j], qf[c], s[j]);
    }
  };

  // P V over key pairs (sub-tiles 2p, 2p+1) with 16x16x32 MFMA: contraction
  // slots 8lg..8lg+3 are keys 32p + 4lg + {0..3}, slots 8lg+4..8lg+7 keys
  // 32p + 16 + 4lg + {0..3}, for both the V^T operand (two transposed LDS
  // reads) and the P^T operand (the lane's own scores).
  auto softmax_pv = [&](int tt, const char* st, f32x4* s) {
    const char* Vs = st + TILEB;
    const int tile_base = tile_key0(split, tt, n_split);
    v8 vf[2][8];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int rv = 32 * p + 4 * lg + (ln >> 2);
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int chunk = 2 * t + ((ln >> 1) & 1), half = (ln & 1) << 3;
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Vs + sw_off(rv, chunk) + half));
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Vs + sw_off(rv + 16, chunk) + half));
        vf[p][t] = __builtin_bit_cast(v8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) s[j][i] *= scale_log2;
    if (tile_base + TK > kv_len || tile_base + TK - 1 > causal_off) {   // wave-uniform
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = tile_base + 16 * j + 4 * lg + i;
          s[j][i] = (key < kv_len && key <= lim) ? s[j][i] : -INFINITY;
        }
    }
    // Per-lane max against the running max; the running max is raised
    // (cross-lane reduction + rescale, one wave-uniform branch) only when a
    // score exceeds it by more than kRescaleSlack, so probabilities stay
    // <= 2^kRescaleSlack and the common path has no cross-lane traffic.
    float lm = fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3]));
#pragma unroll
    for (int j = 1; j < 4; ++j) lm = fmaxf(lm, fmaxf(fmaxf(s[j][0], s[j][1]), fmaxf(s[j][2], s[j][3])));
    if (__ballot(lm > m_run + kRescaleSlack)) {
      const float mt = xor32_max(xor16_max(lm));
      const float m_new = mt > m_run + kRescaleSlack ? mt : m_run;
      const float alpha = fast_exp2(m_run - m_new);
      lsum *= alpha;
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[t] *= alpha;
      m_run = m_new;
    }
    v8 pb[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      float x[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[i] = fast_exp2(s[2 * p][i] - m_run);
        x[4 + i] = fast_exp2(s[2 * p + 1][i] - m_run);
      }
      const i16x4 lo = EL::pack4(x[0], x[1], x[2], x[3]);
      const i16x4 hi = EL::pack4(x[4], x[5], x[6], x[7]);
      pb[p] = __builtin_bit_cast(v8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) lsum = EL::mma32(ones, pb[p], lsum);
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int p = 0; p < 2; ++p) acc[t] = EL::mma32(vf[p][t], pb[p], acc[t]);
  };

  // Key-split tile (KS waves, and the HYB waves on the last row tile): wave
  // sub-tile ks_sub scores keys 16 ks_sub .. 16 ks_sub + 15 of the tile (one
  // S^T sub-tile, lane (ln, lg) element i = key 16 ks_sub + 4lg + i of row
  // ln) and accumulates P V over them with 16x16x16 MFMAs, whose contraction
  // slots 4lg..4lg+3 are exactly the lane's own four keys (P^T operand) and,
  // through one transposed LDS read per 16 output columns, the same keys of V
  // (V^T operand). Each such wave keeps its own running max, row sum and
  // output rows; ks_merge combines the four.
  const v4 ones4 = __builtin_bit_cast(v4, i16x4{EL::kOne, EL::kOne, EL::kOne, EL::kOne});
  auto ks_tile = [&](int tt, const char* st) {
    f32x4 sc = {0.f, 0.f, 0.f, 0.f}, sl = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const v8 kf = *reinterpret_cast<const v8*>(st + sw_off(16 * ks_sub + ln, 4 * c + lg));
      sc = EL::mma32(kf, qf[c], sc);
      if constexpr (COLL) sl = EL::mma32(kf, qlo[c], sl);
    }
    if constexpr (COLL) {
      // Collector lanes: logits of this wave's four keys of the tile, over
      // the visual keys only; stored, and folded into the lane's (max, sum).
      if (ln >= q_off) {
        const int kb = tile_key0(split, tt, n_split);
        const int key0 = kb + 16 * ks_sub + 4 * lg;
        uint32_t mb = 0xfu;                                   // the lane's four keys: visual-mask bits
        if (ga.vmask != nullptr) {                            // wave-uniform
          uint32_t w16;
          if (tt < 64) {
            w16 = (uint32_t)__builtin_amdgcn_readlane((int)vbits, tt);
          } else {
            const int kw = kb + 16 * ks_sub;
            w16 = (kw < ga.vis_end && kw + 16 > ga.vis_begin) ? (ga.vmask[kw >> 5] >> (kw & 31)) & 0xffffu : 0u;
          }
          mb = (w16 >> (4 * lg)) & 0xfu;
        }
        float z[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool vis = key0 + i >= ga.vis_begin && key0 + i < ga.vis_end && ((mb >> i) & 1u);
          z[i] = vis ? (sc[i] + sl[i]) * scale_log2 : -INFINITY;
        }
        const int vt = kb / TK - ga.vis_begin / TK;           // wave-uniform
        if (vt >= 0 && vt < ga.n_vtiles) {
          float* dst = ga.logits + (((long long)g * ga.n_vtiles + vt) * q_len + (ln - q_off)) * TK + 16 * ks_sub +
                       4 * lg;
          *reinterpret_cast<f32x4*>(dst) = f32x4{z[0], z[1], z[2], z[3]};
        }
        const float mx = fmaxf(fmaxf(z[0], z[1]), fmaxf(z[2], z[3]));
        if (mx > m_c) {
          l_c *= fast_exp2(m_c - mx);
          m_c = mx;
        }
        l_c += (fast_exp2(z[0] - m_c) + fast_exp2(z[1] - m_c)) + (fast_exp2(z[2] - m_c) + fast_exp2(z[3] - m_c));
      }
    }
    const char* Vs = st + TILEB;
    const int rv = 16 * ks_sub + 4 * lg + (ln >> 2);
    v4 vf[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int chunk = 2 * t + ((ln >> 1) & 1), half = (ln & 1) << 3;
      vf[t] = __builtin_bit_cast(v4,
                                 __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Vs + sw_off(rv, chunk) + half)));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) sc[i] *= scale_log2;
    const int tile_base = tile_key0(split, tt, n_split);
    const int key0 = tile_base + 16 * ks_sub + 4 * lg;
    if (tile_base + TK > kv_len || tile_base + TK - 1 > causal_off) {   // wave-uniform
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[i] = (key0 + i < kv_len && key0 + i <= lim) ? sc[i] : -INFINITY;
    }
    const float lm = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
    if (__ballot(lm > m_run + kRescaleSlack)) {
      const float mt = xor32_max(xor16_max(lm));
      const float m_new = mt > m_run + kRescaleSlack ? mt : m_run;
      const float alpha = fast_exp2(m_run - m_new);
      lsum *= alpha;
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[t] *= alpha;
      m_run = m_new;
    }
    const v4 pb = __builtin_bit_cast(v4, EL::pack4(fast_exp2(sc[0] - m_run), fast_exp2(sc[1] - m_run),
                                                           fast_exp2(sc[2] - m_run), fast_exp2(sc[3] - m_run)));
    lsum = EL::mma16(ones4, pb, lsum);
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = EL::mma16(vf[t], pb, acc[t]);
  };
  // Merge of the four key-split waves' (m, l, O) rows r0 + 0..15: each
  // stores its own into LDS (mlw, Ow at ring offset 0 and 1 KiB; the caller
  // guarantees that nobody reads those bytes any more), one barrier, then
  // nthr threads (thread index t) form each output element as the sum over
  // the waves, in wave order, of O rescaled from the wave's max to the common
  // one, and write the normalised row (one split) or the (m, l, O) partial.
  static_assert(1024 + 4 * 16 * OROW * 4 <= 2 * STAGEB, "key-split merge region exceeds two ring stages");
  auto ks_store = [&](char* region) {
    float2* mlw = reinterpret_cast<float2*>(region);
    float* Ow = reinterpret_cast<float*>(region + 1024);
    if (lg == 0) mlw[ks_sub * 16 + ln] = make_float2(m_run, lsum[0]);
#pragma unroll
    for (int t = 0; t < 8; ++t)
      *reinterpret_cast<f32x4*>(Ow + (ks_sub * 16 + ln) * OROW + 16 * t + 4 * lg) = acc[t];
  };
  auto ks_merge_rows = [&](const char* region, int r0, int nthr, int t0) {
    const float2* mlw = reinterpret_cast<const float2*>(region);
    const float* Ow = reinterpret_cast<const float*>(region + 1024);
    // Items are row-major and every thread runs the same number of them (nthr
    // divides 16 * D / 4), so the 32 items of a row sit in 32 consecutive lanes
    // of one wave: the row's max |O| is a five-step butterfly over them.
    for (int item = t0; item < 16 * (D / 4); item += nthr) {
      const int rl = item / (D / 4), d4 = item % (D / 4), r = r0 + rl;
      float2 ml[4];
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) ml[ww] = mlw[ww * 16 + rl];
      const float Mr = fmaxf(fmaxf(ml[0].x, ml[1].x), fmaxf(ml[2].x, ml[3].x));
      float Lr = 0.f;
      f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) {
        const float e = fast_exp2(ml[ww].x - Mr);
        Lr += ml[ww].y * e;
        o += *reinterpret_cast<const f32x4*>(Ow + (ww * 16 + rl) * OROW + 4 * d4) * e;
      }
      const int hl = r / q_len, i = r - hl * q_len;
      if (n_split == 1) {
        if (r < R) {
          bf16_t* dst = out + ((long long)(g * group + hl) * q_len + i) * D + 4 * d4;
          const f32x4 on = o / Lr;
          *reinterpret_cast<i16x4*>(dst) = EL::pack4(on[0], on[1], on[2], on[3]);
        }
      } else if constexpr (std::is_same<PartT<NT, E>, half_t>::value) {
        float amax = fmaxf(fmaxf(fabsf(o[0]), fabsf(o[1])), fmaxf(fabsf(o[2]), fabsf(o[3])));
#pragma unroll
        for (int off = 1; off < 32; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
        if (r < R) {
          const int kx = part_exp(amax);
          const float sx = exp2i(-kx);
          const long long prow = (long long)g * n_split * R + (long long)split * R + r;
          *reinterpret_cast<half4_t*>(ws_o + prow * D + 4 * d4) = __builtin_convertvector(o * sx, half4_t);
          if (d4 == 0) ws_ml[prow] = make_float2(Mr + (float)kx, Lr * sx);
        }
      } else if (r < R) {
        const long long prow = (long long)g * n_split * R + (long long)split * R + r;
        *reinterpret_cast<f32x4*>(ws_o + prow * D + 4 * d4) = o;
        if (d4 == 0) ws_ml[prow] = make_float2(Mr, Lr);
      }
    }
  };
  auto ks_merge = [&](char* region, int r0, int nthr, int t0) {
    ks_store(region);
    __syncthreads();
    ks_merge_rows(region, r0, nthr, t0);
  };

  // Software pipeline, one step per tile u (steps 0..ntiles): after the
  // barrier, tile u+2 is prefetched into the stage tile u-2 used (every wave
  // finished tile u-2's PV before this barrier), the QK^T MFMAs of tile u are
  // issued into one score buffer, then the softmax and PV of tile u-1 run on
  // the other, so matrix and vector work of neighbouring tiles overlap inside
  // a wave and two tiles stay in flight during the step.
  f32x4 sA[4], sB[4];
  auto step = [&](int u, const char* cur, const char* prev, char* ahead2, f32x4* s_new, f32x4* s_old) {
    if (u > ntiles) return;
    if (u < ntiles && dma_wave) wait_vm_ahead<kLoads>(u + 1 < ntiles ? 1 : 0);
    wg_barrier();
#if STD_PHASE_STAMPS
    if (tid == 0 && u < 40) stamp(2 + u);
#endif
    if (u + 2 < ntiles) issue(u + 2, ahead2);
    if (computes) {
      if (u < ntiles) qk(cur, s_new);
      if (u > 0) softmax_pv(u - 1, prev, s_old);
    }
    if (HYB && ksw && u < ntiles) ks_tile(u, cur);
  };
  // Tile u lives in ring stage u % NSTAGE. The loop is unrolled by two only
  // for the score ping-pong; stage addresses are computed at run time, which
  // keeps the loop body small (it is fetched cold by every CU).
  if constexpr (KS) {
    // Key split: QK^T and PV of tile u in step u; tiles u+1 and u+2 may still be in flight when tile u is
    // complete; after the barrier (every wave is done with tile u-1) tile u+3
    // goes into tile u-1's stage, then tile u is scored and accumulated.
    for (int u = 0; u < ntiles; ++u) {
      wait_vm_ahead<kLoads>(min(2, ntiles - 1 - u));
      wg_barrier();
#if STD_PHASE_STAMPS
      if (tid == 0 && u < 40) stamp(2 + u);
#endif
      if (u + 3 < ntiles) issue(u + 3, stage(u + 3));
      ks_tile(u, stage(u));
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __syncthreads();                             // the ring is free: reuse it for the merge
#if STD_PHASE_STAMPS
    if (tid == 0) stamp(43);
#endif
    ks_merge(ring, 0, C::kThreads, tid);
#if STD_PHASE_STAMPS
    if (tid == 0) {
      __builtin_amdgcn_s_waitcnt(0);
      stamp(47);
      stamp(46, (unsigned long long)ntiles);
    }
#endif
    return;
  } else {
    for (int u = 0; u <= ntiles; u += 2) {
      step(u, stage(u), stage(u + 3), stage(u + 2), sA, sB);
      step(u + 1, stage(u + 1), stage(u), stage(u + 3), sB, sA);
    }
  }
  if (dma_wave) __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  if constexpr (HYB) {
    // The row owners may still read the last tile's stage (their final PV);
    // the key-split waves merge through two other stages, then write the last
    // row tile while the owners write theirs.
    const int sl = (ntiles - 1) & (NSTAGE - 1);
    char* region = ring + (sl <= 1 ? (sl + 1) * STAGEB : 0);
    // Collector: each key-split wave's (max, sum) per row over its four lane
    // groups, then (after the barrier) the four waves in wave order.
    float2* cst = reinterpret_cast<float2*>(region + 1024 + 4 * 16 * OROW * 4);
    if constexpr (COLL) {
      static_assert(1024 + 4 * 16 * OROW * 4 + 4 * 16 * 8 <= 2 * STAGEB, "collector statistics exceed the region");
      if (ksw) {
        const float M = xor32_max(xor16_max(m_c));
        const float L = xor32_sum(xor16_sum(l_c * fast_exp2(m_c - M)));
        if (lg == 0) cst[ks_sub * 16 + ln] = make_float2(M, L);
      }
    }
    if (ksw) ks_store(region);
    __syncthreads();
    if (ksw) {
      if constexpr (COLL) {
        const int t = tid - 64 * kOwners;
        if (t < q_len) {
          float2 w[4];
#pragma unroll
          for (int ww = 0; ww < 4; ++ww) w[ww] = cst[ww * 16 + q_off + t];
          const float M = fmaxf(fmaxf(w[0].x, w[1].x), fmaxf(w[2].x, w[3].x));
          float L = 0.f;
#pragma unroll
          for (int ww = 0; ww < 4; ++ww) L += w[ww].y * fast_exp2(w[ww].x - M);
          ga.stats[((long long)g * n_split + split) * q_len + t] = make_float2(M, L);
        }
      }
#if STD_PHASE_STAMPS
      if (tid == 64 * kOwners) stamp(44);
#endif
      ks_merge_rows(region, 16 * kOwners, C::kThreads - 64 * kOwners, tid - 64 * kOwners);
#if STD_PHASE_STAMPS
      if (tid == 64 * kOwners) {
        __builtin_amdgcn_s_waitcnt(0);
        stamp(45);
      }
#endif
      return;
    }
  }
#if STD_PHASE_STAMPS
  if (tid == 0) {
    stamp(43);
    stamp(46, (unsigned long long)ntiles);
  }
#endif
  if (!row_ok) return;

  // Complete rows: normalised output (one split) or the (m, l, O) partial.
  const float l_row = lsum[0];
  const int hl = row / q_len, i = row - hl * q_len;
  if (n_split == 1) {
    bf16_t* dst = out + ((long long)(g * group + hl) * q_len + i) * D + 4 * lg;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const f32x4 o = acc[t] / l_row;
      *reinterpret_cast<i16x4*>(dst + 16 * t) = EL::pack4(o[0], o[1], o[2], o[3]);
    }
  } else if constexpr (!std::is_same<PartT<NT, E>, half_t>::value) {
    const long long prow = (long long)g * n_split * R + (long long)split * R + row;
#pragma unroll
    for (int t = 0; t < 8; ++t) *reinterpret_cast<f32x4*>(ws_o + prow * D + 16 * t + 4 * lg) = acc[t];
    if (lg == 0) ws_ml[prow] = make_float2(m_run, l_row);
  } else {
    // The row's 128 columns are spread over its four lanes (lg).
    float amax = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t)
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(acc[t][0]), fabsf(acc[t][1])), fmaxf(fabsf(acc[t][2]), fabsf(acc[t][3]))));
    amax = xor32_max(xor16_max(amax));
    const int kx = part_exp(amax);
    const float sx = exp2i(-kx);
    const long long prow = (long long)g * n_split * R + (long long)split * R + row;
#pragma unroll
    for (int t = 0; t < 8; ++t)
      *reinterpret_cast<half4_t*>(ws_o + prow * D + 16 * t + 4 * lg) = __builtin_convertvector(acc[t] * sx, half4_t);
    if (lg == 0) ws_ml[prow] = make_float2(m_run + (float)kx, l_row * sx);
  }
#if STD_PHASE_STAMPS
  if (tid == 0) {
    __builtin_amdgcn_s_waitcnt(0);
    stamp(47);
  }
#endif
}

// ===========================================================================
// fp32 kernel: register-staged double buffer, 16x16x4 fp32 MFMA.
struct F32Frag {
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

template <int NT>
struct F32Smem {
  static constexpr int kTileElems = TK * LROW;
  static constexpr int kKVBytes = 2 * 2 * kTileElems * 4;   // K,V x double buffer
  static constexpr int kOBytes = NT * OTILE_BYTES;
  static constexpr int kMLOff = kKVBytes > kOBytes ? kKVBytes : kOBytes;
  static constexpr int kBytes = kMLOff + (WAVES + 1) * NT * 16 * 8;
};

template <int NT>
__global__ void __launch_bounds__(NTHREADS)
attn_f32_kernel(const float* __restrict__ q, float* __restrict__ kc, float* __restrict__ vc,
                float* __restrict__ out, float* __restrict__ ws_o, float2* __restrict__ ws_ml, int q_len,
                int kv_len, int group, long long k_hs, long long v_hs, float scale_log2, int ntiles_total,
                int n_split, int causal_off, const float* __restrict__ new_k, const float* __restrict__ new_v,
                long long n_hs, long long n_rs, int n_new, BatchStrides bs, const int32_t* __restrict__ len_dev,
                int32_t* status) {
  using F = F32Frag;
  using S = F32Smem<NT>;
  constexpr int CPR = D / 4;                    // 16-byte chunks per fp32 row
  constexpr int CPT = TK * CPR / NTHREADS;      // chunks per thread per tile
  __shared__ __align__(16) unsigned char smem[S::kBytes];
  float* Ks = reinterpret_cast<float*>(smem);
  float* Vs = Ks + 2 * S::kTileElems;

  const int g = blockIdx.y, split = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  const int R = group * q_len;
  {
    const long long b = blockIdx.z;
    q += b * bs.q;
    kc += b * bs.k;
    vc += b * bs.v;
    out += b * bs.o;
    if (n_split > 1) {
      ws_o += b * bs.w * D;
      ws_ml += b * bs.w;
    }
  }
  if (len_dev != nullptr) {
    device_length(len_dev, q_len, kv_len, ntiles_total, causal_off);
    if (kv_len == 0 && threadIdx.x == 0 && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0) flag_overflow(status);
  }
  const int ntiles = split_ntiles(split, ntiles_total, n_split);
  float* kh = kc + (long long)g * k_hs;
  float* vh = vc + (long long)g * v_hs;
  if (n_new > 0) {
    append_rows<float>(kh, vh, new_k, new_v, n_hs, n_rs, g, n_new, kv_len, split, n_split, NTHREADS);
    __syncthreads();
  }

  typename F::QFrag qf[NT];
  int lim[NT];
#pragma unroll
  for (int rt = 0; rt < NT; ++rt) {
    const int r = rt * 16 + ln;
    if (r < R) {
      const int hl = r / q_len, i = r - hl * q_len;
      F::load_q(qf[rt], q + ((long long)(g * group + hl) * q_len + i) * D, lg);
      lim[rt] = causal_off + i;
    } else {
      F::zero_q(qf[rt]);
      lim[rt] = INT_MAX;
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
    const int base = tile_key0(split, t, n_split);
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int c = tid + j * NTHREADS;
      const int row = c / CPR, col = c - row * CPR;
      const int key = base + row;
      if (key < kv_len) {
        kreg[j] = *reinterpret_cast<const uint4*>(kh + (long long)key * D + col * 4);
        vreg[j] = *reinterpret_cast<const uint4*>(vh + (long long)key * D + col * 4);
      } else {
        kreg[j] = make_uint4(0, 0, 0, 0);
        vreg[j] = make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto lstore = [&](int buf) {
    float* kd = Ks + buf * S::kTileElems;
    float* vd = Vs + buf * S::kTileElems;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int c = tid + j * NTHREADS;
      const int row = c / CPR, col = c - row * CPR;
      *reinterpret_cast<uint4*>(kd + row * LROW + col * 4) = kreg[j];
      *reinterpret_cast<uint4*>(vd + row * LROW + col * 4) = vreg[j];
    }
  };

  gload(0);
  lstore(0);
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) gload(t + 1);
    const float* Kt = Ks + buf * S::kTileElems;
    const float* Vt = Vs + buf * S::kTileElems;
    const int tile_base = tile_key0(split, t, n_split);
    const bool need_mask = (tile_base + TK > kv_len) || (tile_base + TK - 1 > causal_off);
    typename F::KFrag kf;
    typename F::VFrag vf;
    F::load_k(kf, Kt + (w * 16 + ln) * LROW, lg);
    F::load_v(vf, Vt, w * 16, ln, lg);
    const int key0 = tile_base + w * 16 + 4 * lg;
#pragma unroll
    for (int rt = 0; rt < NT; ++rt) {
      const f32x4 s = F::qk(kf, qf[rt]);
      float sv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[i] = s[i] * scale_log2;
      if (need_mask) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = key0 + i;
          if (key >= kv_len || key > lim[rt]) sv[i] = -INFINITY;
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

#pragma unroll
  for (int rt = 0; rt < NT; ++rt) {
    l_run[rt] += __shfl_xor(l_run[rt], 16);
    l_run[rt] += __shfl_xor(l_run[rt], 32);
  }
  float* So = reinterpret_cast<float*>(smem);
  float2* ml_w = reinterpret_cast<float2*>(smem + S::kMLOff);
  float2* ml_f = ml_w + WAVES * NT * 16;
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
  auto load_o = [&](int r, int d4) -> f32x4 { return *reinterpret_cast<const f32x4*>(So + r * OROW + 4 * d4); };
  finish_split<float>(load_o, ml_f, out, ws_o, ws_ml, g, split, n_split, q_len, group, NTHREADS);
}

// ===========================================================================
// The split launch of the 16-bit kernels with element type E (bf16_t or
// f16_t); the caller launches the merge.
template <int NT, typename E>
void launch_h16(const void* q, void* k, void* v, void* out, int q_len, int kv_len, int group, long long k_hs,
                long long v_hs, float scale_log2, const SplitPlan& p, void* ws_o, float2* ws_ml, const void* nk,
                const void* nv, long long n_hs, long long n_rs, int n_new, dim3 grid, BatchStrides bs,
                const int32_t* len_dev, GatherArgs ga, hipStream_t st) {
  // One row tile and at least two tiles per split on average: key split.
  const bool ks = NT == 1 && p.ntiles >= 2 * p.n_split;
  // Long key ranges stream with non-temporal loads (stream_keys).
  const bool str = stream_keys(p.ntiles);
  // Gathered keys (decode only): a separate instantiation, so the plain
  // kernels carry none of the gather code or arguments.
  auto kern = NT == 1 && ga.idx != nullptr
                  ? (ks ? attn_bf16_kernel<NT, NT == 1, NT == 1, false, E>
                        : attn_bf16_kernel<NT, false, NT == 1, false, E>)
                  : str ? (ks ? attn_bf16_kernel<NT, NT == 1, false, false, E, true>
                              : attn_bf16_kernel<NT, false, false, false, E, true>)
                        : (ks ? attn_bf16_kernel<NT, NT == 1, false, false, E>
                              : attn_bf16_kernel<NT, false, false, false, E>);
  hipLaunchKernelGGL(kern, grid, dim3(Bf16Cfg<NT>::kThreads), 0, st,
                     static_cast<const bf16_t*>(q), static_cast<bf16_t*>(k), static_cast<bf16_t*>(v),
                     static_cast<bf16_t*>(out), static_cast<PartT<NT, E>*>(ws_o), ws_ml, q_len, kv_len, group, k_hs,
                     v_hs, scale_log2, p.ntiles, p.n_split, kv_len - q_len, static_cast<const bf16_t*>(nk),
                     static_cast<const bf16_t*>(nv), n_hs, n_rs, n_new, bs, len_dev,
                     GatherDev{ga.status, ga.idx_hs, ga.n_idx, ga.dense_rows, ga.k, ga.v, ga.k_hs, ga.v_hs}, ga.idx);
}

// The merge launch: the wave form up to kWaveMergeMax splits, the block
// form beyond.
template <typename T, typename PT>
void launch_merge(const void* ws_o, const float2* ws_ml, void* out, int n_split, int q_len, int group, long long out_bs,
                  int n_kv, int R, int n_batch, hipStream_t st) {
  const dim3 grid(R, n_kv, n_batch);
  const PT* o = static_cast<const PT*>(ws_o);
  T* y = static_cast<T*>(out);
  if (n_split > kWaveMergeMax) {
    hipLaunchKernelGGL((attn_merge_kernel<T, PT, 0>), grid, dim3(kMergeThreads), 0, st, o, ws_ml, y, n_split, q_len,
                       group, out_bs, n_kv);
    return;
  }
  const int j = merge_j(n_split);
  auto kern = j == 4 ? attn_merge_kernel<T, PT, 4> : j == 8 ? attn_merge_kernel<T, PT, 8>
            : j == 9 ? attn_merge_kernel<T, PT, 9> : j == 12 ? attn_merge_kernel<T, PT, 12>
                     : attn_merge_kernel<T, PT, 16>;
  hipLaunchKernelGGL(kern, grid, dim3(64), 0, st, o, ws_ml, y, n_split, q_len, group, out_bs, n_kv);
}

template <int NT>
int launch_nt(const void* q, void* k, void* v, void* out, int n_kv, int q_len, int kv_len, int group,
              long long k_hs, long long v_hs, float scale, int dtype, void* ws, const void* nk, const void* nv,
              long long n_hs, long long n_rs, int n_new, int n_batch, BatchStrides bs, const int32_t* len_dev,
              GatherArgs ga, hipStream_t st) {
  const int R = group * q_len;
  const SplitPlan p = plan_splits(n_kv * n_batch, R, kv_len, dtype);
  const WsLayout wl = ws_layout(n_kv * n_batch, R, p, part_bytes_of(dtype, R));
  char* base = static_cast<char*>(ws);
  void* ws_o = p.n_split > 1 ? static_cast<void*>(base + wl.o_off) : nullptr;
  float2* ws_ml = p.n_split > 1 ? reinterpret_cast<float2*>(base + wl.ml_off) : nullptr;
  const float scale_log2 = scale * 1.4426950408889634f;
  const dim3 grid(p.n_split, n_kv, n_batch);
  bs.w = (long long)n_kv * p.n_split * R;
  if (dtype != STD_F32) {
    if (dtype == STD_BF16)
      launch_h16<NT, bf16_t>(q, k, v, out, q_len, kv_len, group, k_hs, v_hs, scale_log2, p, ws_o, ws_ml, nk, nv, n_hs,
                             n_rs, n_new, grid, bs, len_dev, ga, st);
    else
      launch_h16<NT, f16_t>(q, k, v, out, q_len, kv_len, group, k_hs, v_hs, scale_log2, p, ws_o, ws_ml, nk, nv, n_hs,
                            n_rs, n_new, grid, bs, len_dev, ga, st);
  } else {
    hipLaunchKernelGGL((attn_f32_kernel<NT>), grid, dim3(NTHREADS), 0, st, static_cast<const float*>(q),
                       static_cast<float*>(k), static_cast<float*>(v), static_cast<float*>(out),
                       static_cast<float*>(ws_o), ws_ml, q_len,
                       kv_len, group, k_hs, v_hs, scale_log2, p.ntiles, p.n_split, kv_len - q_len,
                       static_cast<const float*>(nk), static_cast<const float*>(nv), n_hs, n_rs, n_new, bs, len_dev,
                       ga.status);
  }
  int s = launch_status();
  if (s != 0 || p.n_split == 1) return s;
  if (dtype == STD_BF16)
    launch_merge<bf16_t, PartT<NT, bf16_t>>(ws_o, ws_ml, out, p.n_split, q_len, group, bs.o, n_kv, R, n_batch, st);
  else if (dtype == STD_F16)
    launch_merge<f16_t, PartT<NT, f16_t>>(ws_o, ws_ml, out, p.n_split, q_len, group, bs.o, n_kv, R, n_batch, st);
  else
    launch_merge<float, float>(ws_o, ws_ml, out, p.n_split, q_len, group, bs.o, n_kv, R, n_batch, st);
  return launch_status();
}

int launch_attn(const void* q, void* k, void* v, void* out, int n_kv, int q_len, int kv_len, int group,
                long long k_hs, long long v_hs, float scale, int dtype, void* ws, const void* nk, const void* nv,
                long long n_hs, long long n_rs, int n_new, int n_batch, BatchStrides bs, const int32_t* len_dev,
                GatherArgs ga, hipStream_t st) {
#define STD_LAUNCH_NT(N)                                                                                       \
  launch_nt<N>(q, k, v, out, n_kv, q_len, kv_len, group, k_hs, v_hs, scale, dtype, ws, nk, nv, n_hs, n_rs, n_new, \
               n_batch, bs, len_dev, ga, st)
  switch ((group * q_len + 15) / 16) {
    case 1: return STD_LAUNCH_NT(1);
    case 2: return STD_LAUNCH_NT(2);
    case 3: return STD_LAUNCH_NT(3);
    case 4: return STD_LAUNCH_NT(4);
    case 5: return STD_LAUNCH_NT(5);
    case 6: return STD_LAUNCH_NT(6);
    default: return STD_E_SHAPE;
  }
#undef STD_LAUNCH_NT
}

size_t attn_workspace_bytes(int n_kv, int rows, int kv_len, int dtype) {
  return ws_layout(n_kv, rows, plan_splits(n_kv, rows, kv_len, dtype), part_bytes_of(dtype, rows)).total;
}

int attn_entry(const void* q, void* k, void* v, void* out, int n_q, int n_kv, int q_len, int kv_len, int d,
               long long k_hs, long long v_hs, float scale, int dtype, void* ws, size_t ws_bytes, const void* nk,
               const void* nv, long long n_hs, long long n_rs, int n_new, void* stream, int n_batch = 1,
               BatchStrides bs = BatchStrides{0, 0, 0, 0}, const int32_t* len_dev = nullptr,
               GatherArgs ga = GatherArgs{nullptr, 0, 0, 0, nullptr, nullptr, 0, 0, nullptr}) {
  if (!q || !k || !v || !out) return STD_E_NULL;
  if (ga.idx != nullptr) {
    // Gathered keys: one bf16 decode problem; indices padded to 16 per row of
    // the index array and 16-byte aligned (they are read four at a time).
    if (!ga.k || !ga.v) return STD_E_NULL;
    if (dtype != STD_BF16 && dtype != STD_F16) return STD_E_DTYPE;
    if (q_len != 1 || n_batch != 1 || n_new > 0) return STD_E_SHAPE;
    if (ga.n_idx < 0 || ga.n_idx > kv_len || ga.dense_rows < 1) return STD_E_SHAPE;
    if (ga.idx_hs < (long long)round_up((size_t)ga.n_idx, 16)) return STD_E_SHAPE;
    if (n_kv > 1 && (ga.k_hs < (long long)ga.dense_rows * D || ga.v_hs < (long long)ga.dense_rows * D))
      return STD_E_SHAPE;
    if (!aligned16(ga.idx) || ga.idx_hs % 4 != 0 || !aligned16(ga.k) || !aligned16(ga.v) ||
        (ga.k_hs * 2) % 16 != 0 || (ga.v_hs * 2) % 16 != 0)
      return STD_E_ALIGN;
  }
  if (n_batch < 1 || n_batch > 65535) return STD_E_SHAPE;
  if (n_batch == 1) {
    bs = BatchStrides{0, 0, 0, 0};
  } else {
    const long long rows = (long long)n_q * q_len * D;
    if (n_new > 0) return STD_E_SHAPE;                       // the fused append serves one problem
    if (bs.q < rows || bs.o < rows || bs.k < 0 || bs.v < 0) return STD_E_SHAPE;
    const int es = dtype_size(dtype);
    if ((bs.q * es) % 16 || (bs.o * es) % 16 || (bs.k * es) % 16 || (bs.v * es) % 16) return STD_E_ALIGN;
  }
  if (n_new > 0 && (!nk || !nv)) return STD_E_NULL;
  if (dtype != STD_F32 && dtype != STD_BF16 && dtype != STD_F16) return STD_E_DTYPE;
  if (d != D || n_q <= 0 || n_kv <= 0 || n_q % n_kv != 0 || q_len < 1 || kv_len < q_len) return STD_E_SHAPE;
  const int group = n_q / n_kv;
  if ((long long)group * q_len > kMaxRows) return STD_E_SHAPE;
  const int es = dtype_size(dtype);
  if (n_kv > 1 && (k_hs < (long long)kv_len * D || v_hs < (long long)kv_len * D)) return STD_E_SHAPE;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out)) return STD_E_ALIGN;
  if ((k_hs * es) % 16 != 0 || (v_hs * es) % 16 != 0) return STD_E_ALIGN;
  if (n_new > 0 && (!aligned16(nk) || !aligned16(nv) || (n_hs * es) % 16 != 0 || (n_rs * es) % 16 != 0))
    return STD_E_ALIGN;
  const size_t need = attn_workspace_bytes(n_kv * n_batch, group * q_len, kv_len, dtype);
  if (need > 0 && (ws == nullptr || ws_bytes < need)) return STD_E_WORKSPACE;
  if (need > 0 && !aligned16(ws)) return STD_E_ALIGN;
  return launch_attn(q, k, v, out, n_kv, q_len, kv_len, group, k_hs, v_hs, scale, dtype, ws, nk, nv, n_hs, n_rs,
                     n_new, n_batch, bs, len_dev, ga, static_cast<hipStream_t>(stream));
}

// Verify + collector. The collector's query rows fill the padding lanes of the
// five-row-tile verify layout's last row tile, so one fused launch serves at
// most coll_chunk(group) verify positions: (group + 1) q <= 80 and q <= 16.
// Longer verifies run chunk by chunk: chunk [a, b) of the positions is the
// verify of rows a..b-1 over the first kv_len - q_len + b keys (row i still
// sees keys [0, kv_len - q_len + i]), with its query rows gathered into the
// workspace and its output rows copied back, and each chunk adds its
// positions' softmax rows to the scores in row order -- the same sums, in the
// same order, as one launch over all rows would form.
int coll_chunk(int group) { return std::min(16, 80 / (group + 1)); }

// Workspace: the verify attention's split partials, then the collector logits
// [n_kv][n_vtiles][q][64] and statistics [n_kv][n_split][q] (q = the chunk
// size), then, for a chunked verify, one chunk's query rows and output rows.
struct CollLayout {
  size_t attn, logits_off, stats_off, q_off, o_off, total;
  int n_vtiles, n_split, q_chunk;
};

// es: element bytes of the rows (2); part_bytes: the split partials' (2 for
// bf16, 4 for fp16; the workspace query sizes for 4, the larger).
CollLayout coll_layout(int n_kv, int group, int q_len, int kv_len, int vis_begin, int vis_end, int es,
                       int part_bytes) {
  CollLayout c{};
  c.q_chunk = std::min(q_len, coll_chunk(group));
  const int R = group * c.q_chunk;
  const SplitPlan p = plan_splits(n_kv, R, kv_len, STD_BF16);     // the largest chunk plan (the longest key range)
  c.n_split = p.n_split;
  c.attn = round_up(ws_layout(n_kv, R, p, part_bytes).total, 256);
  c.n_vtiles = (vis_end - 1) / TK - vis_begin / TK + 1;
  c.logits_off = c.attn;
  c.stats_off = round_up(c.logits_off + (size_t)n_kv * c.n_vtiles * c.q_chunk * TK * sizeof(float), 256);
  c.q_off = round_up(c.stats_off + (size_t)n_kv * p.n_split * c.q_chunk * sizeof(float2), 256);
  c.o_off = c.q_off;
  c.total = c.q_off;
  if (c.q_chunk < q_len) {
    const size_t rows = (size_t)n_kv * group * c.q_chunk * D * es;
    c.o_off = round_up(c.q_off + rows, 256);
    c.total = round_up(c.o_off + rows, 256);
  }
  return c;
}

int verify_collect_entry(const void* q, void* k, void* v, void* out, int n_q, int n_kv, int q_len, int kv_len,
                         const int32_t* len_dev, int d, long long k_hs, long long v_hs, float scale, int dtype,
                         const void* nk, const void* nv, long long n_hs, long long n_rs, int vis_begin, int vis_end,
                         const uint32_t* vmask, const int32_t* vrank, int n_visual, float* scores, long long score_hs,
                         void* ws, size_t ws_bytes, int32_t* status, void* stream) {
  if (!q || !k || !v || !out || !scores) return STD_E_NULL;
  if ((nk == nullptr) != (nv == nullptr)) return STD_E_NULL;
  if ((vmask == nullptr) != (vrank == nullptr)) return STD_E_NULL;
  if (dtype != STD_BF16 && dtype != STD_F16) return STD_E_DTYPE;
  if (d != D || n_q <= 0 || n_kv <= 0 || n_q % n_kv != 0 || q_len < 1 || kv_len < q_len) return STD_E_SHAPE;
  const int group = n_q / n_kv;
  if (coll_chunk(group) < 1 || (long long)group * q_len > 65535) return STD_E_SHAPE;
  if (vis_begin < 0 || vis_end <= vis_begin || vis_end > kv_len - q_len) return STD_E_SHAPE;
  if (vmask == nullptr ? n_visual != vis_end - vis_begin : (n_visual < 1 || n_visual > vis_end - vis_begin))
    return STD_E_SHAPE;
  if (n_kv > 1 && (k_hs < (long long)kv_len * D || v_hs < (long long)kv_len * D)) return STD_E_SHAPE;
  if (n_kv > 1 && score_hs < n_visual) return STD_E_SHAPE;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out)) return STD_E_ALIGN;
  if ((k_hs * 2) % 16 != 0 || (v_hs * 2) % 16 != 0) return STD_E_ALIGN;
  if (nk && (!aligned16(nk) || !aligned16(nv) || (n_hs * 2) % 16 != 0 || (n_rs * 2) % 16 != 0)) return STD_E_ALIGN;
  const int part_bytes = dtype == STD_BF16 ? 2 : 4;
  const CollLayout cl = coll_layout(n_kv, group, q_len, kv_len, vis_begin, vis_end, 2, part_bytes);
  if (ws == nullptr || ws_bytes < cl.total) return STD_E_WORKSPACE;
  if (!aligned16(ws)) return STD_E_ALIGN;
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* base = static_cast<char*>(ws);
  const size_t row_bytes = (size_t)D * 2;
  for (int a = 0; a < q_len; a += cl.q_chunk) {
    const int qc = std::min(cl.q_chunk, q_len - a);
    const bool chunked = qc < q_len;
    const int kv_c = kv_len - q_len + a + qc;                 // keys the chunk's last row sees, plus one
    const int R = group * qc;
    const SplitPlan p = plan_splits(n_kv, R, kv_c, STD_BF16);        // bf16 and fp16 plan alike
    const WsLayout wl = ws_layout(n_kv, R, p, part_bytes);
    void* ws_o = p.n_split > 1 ? static_cast<void*>(base + wl.o_off) : nullptr;
    float2* ws_ml = p.n_split > 1 ? reinterpret_cast<float2*>(base + wl.ml_off) : nullptr;
    const CollArgs ca{reinterpret_cast<float*>(base + cl.logits_off), reinterpret_cast<float2*>(base + cl.stats_off),
                      cl.n_vtiles, vis_begin, vis_end, vmask, a, status};
    const CollOut co{scores, n_kv > 1 ? score_hs : 0LL, vmask, vrank, n_visual, len_dev, a, a > 0 ? 1 : 0};
    const void* qa = q;
    void* oa = out;
    if (chunked) {
      // the chunk's query rows [n_q][qc][D] out of [n_q][q_len][D]
      qa = base + cl.q_off;
      oa = base + cl.o_off;
      const hipError_t e = hipMemcpy2DAsync(base + cl.q_off, qc * row_bytes, static_cast<const char*>(q) + a * row_bytes,
                                            q_len * row_bytes, qc * row_bytes, n_q, hipMemcpyDeviceToDevice, st);
      if (e != hipSuccess) return (int)e;
    }
    const bf16_t* nka = nk ? static_cast<const bf16_t*>(nk) + a * n_rs : nullptr;
    const bf16_t* nva = nv ? static_cast<const bf16_t*>(nv) + a * n_rs : nullptr;
    const int n_new = nk ? qc : 0;
    const int n_rows = p.n_split > 1 ? R : 0;
    auto run = [&](auto elem) -> int {
      using E = decltype(elem);
      using PT = PartT<5, E>;
      auto kern = stream_keys(p.ntiles) ? attn_bf16_kernel<5, false, false, true, E, true>
                                        : attn_bf16_kernel<5, false, false, true, E, false>;
      hipLaunchKernelGGL(kern, dim3(p.n_split, n_kv, 1),
                         dim3(Bf16Cfg<5>::kThreads), 0, st, static_cast<const bf16_t*>(qa), static_cast<bf16_t*>(k),
                         static_cast<bf16_t*>(v), static_cast<bf16_t*>(oa), static_cast<PT*>(ws_o), ws_ml, qc, kv_c,
                         group, k_hs, v_hs,
                         scale * 1.4426950408889634f, p.ntiles, p.n_split, kv_c - qc, nka, nva, n_hs, n_rs, n_new,
                         BatchStrides{0, 0, 0, 0, 0}, len_dev, ca, nullptr);
      const int s = launch_status();
      if (s != 0) return s;
      const bool wave = p.n_split <= kWaveMergeMax;
      const int mj = wave ? merge_j(p.n_split) : 0;
      const dim3 mgrid((wave ? (n_rows + 3) / 4 : n_rows) + (cl.n_vtiles + 15) / 16, n_kv);
      auto mkern = mj == 0 ? merge_coll_kernel<E, PT, 0> : mj == 4 ? merge_coll_kernel<E, PT, 4>
                 : mj == 8 ? merge_coll_kernel<E, PT, 8> : mj == 9 ? merge_coll_kernel<E, PT, 9>
                 : mj == 12 ? merge_coll_kernel<E, PT, 12> : merge_coll_kernel<E, PT, 16>;
      hipLaunchKernelGGL(mkern, mgrid, dim3(kMergeThreads), 0, st, static_cast<const PT*>(ws_o), ws_ml,
                         static_cast<E*>(oa), p.n_split, qc, group, n_rows, ca.logits, ca.stats, co, cl.n_vtiles,
                         vis_begin, vis_end);
      return launch_status();
    };
    const int s = dtype == STD_BF16 ? run(bf16_t{}) : run(f16_t{});
    if (s != 0) return s;
    if (chunked) {
      const hipError_t e = hipMemcpy2DAsync(static_cast<char*>(out) + a * row_bytes, q_len * row_bytes,
                                            base + cl.o_off, qc * row_bytes, qc * row_bytes, n_q,
                                            hipMemcpyDeviceToDevice, st);
      if (e != hipSuccess) return (int)e;
    }
  }
  return 0;
}

}  // namespace

// ---------------------------------------------------------------------------
// Allocation-free decode (std_gqa_decode_noalloc). The split partials live in
// this file-scope device array instead of a caller workspace; every GPU the
// library runs on holds its own copy until the process ends. Host code never
// passes the name `scratch` to a kernel (on the host it is only a stand-in
// symbol): the device address of the current device's copy is looked up once
// per device with hipGetSymbolAddress and kept in scratch_dev. The kernels
// need no initial contents (every partial is written before it is read), so
// nothing is cleared; calls that overlap on one GPU share the array and race.
constexpr size_t kNoAllocScratchBytes = (2u << 20) + (64u << 10);
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_dev[kMaxDevices];

// Device address of the current device's scratch array; the stream (if not
// the null stream) must belong to that device.
int scratch_address(hipStream_t st, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return STD_E_RANGE;
  if (st != nullptr) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(st, &sdev);
    if (e != hipSuccess) return (int)e;
    if (sdev != dev) return STD_E_RANGE;
  }
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_dev[dev] == nullptr) {
    // The lookup enqueues nothing, so a first call made while the caller's
    // stream is being captured into a graph performs it in relaxed capture
    // mode (a global-mode capture may refuse other HIP calls on this thread).
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    e = hipThreadExchangeStreamCaptureMode(&mode);
    if (e != hipSuccess) return (int)e;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    const hipError_t e2 = hipThreadExchangeStreamCaptureMode(&mode);
    if (e != hipSuccess) return (int)e;
    if (e2 != hipSuccess) return (int)e2;
    scratch_dev[dev] = p;
  }
  *out = scratch_dev[dev];
  return 0;
}
}  // namespace
}  // namespace stdhip

using namespace stdhip;

extern "C" int std_attn_split_count(int n_problems, int rows, int kv_len, int dtype) {
  if (dtype != STD_BF16 && dtype != STD_F32 && dtype != STD_F16) return STD_E_DTYPE;
  if (n_problems < 1 || rows < 1 || rows > kMaxRows || kv_len < 1) return STD_E_SHAPE;
  return plan_splits(n_problems, rows, kv_len, dtype).n_split;
}

extern "C" size_t std_gqa_decode_workspace_bytes(int n_q, int n_kv, int kv_len, int d) {
  if (n_q <= 0 || n_kv <= 0 || n_q % n_kv != 0 || kv_len < 1 || d != D) return 0;
  // the larger of the two dtype plans, so one query serves both
  const size_t a = attn_workspace_bytes(n_kv, n_q / n_kv, kv_len, STD_BF16);
  const size_t b = attn_workspace_bytes(n_kv, n_q / n_kv, kv_len, STD_F32);
  return a > b ? a : b;
}

extern "C" int std_gqa_decode(const void* q, const void* k, const void* v, void* out, int n_q, int n_kv,
                              int kv_len, int d, long long k_head_stride, long long v_head_stride, float scale,
                              int dtype, void* workspace, size_t workspace_bytes, void* stream) {
  return attn_entry(q, const_cast<void*>(k), const_cast<void*>(v), out, n_q, n_kv, 1, kv_len, d, k_head_stride,
                    v_head_stride, scale, dtype, workspace, workspace_bytes, nullptr, nullptr, 0, 0, 0, stream);
}

extern "C" size_t std_gqa_decode_batched_workspace_bytes(int n_batch, int n_q, int n_kv, int kv_len, int d) {
  if (n_batch < 1 || n_batch > 65535 || n_q <= 0 || n_kv <= 0 || n_q % n_kv != 0 || kv_len < 1 || d != D) return 0;
  const size_t a = attn_workspace_bytes(n_kv * n_batch, n_q / n_kv, kv_len, STD_BF16);
  const size_t b = attn_workspace_bytes(n_kv * n_batch, n_q / n_kv, kv_len, STD_F32);
  return a > b ? a : b;
}

extern "C" int std_gqa_decode_batched(const void* q, const void* k, const void* v, void* out, int n_batch, int n_q,
                                      int n_kv, int kv_len, int d, long long q_batch_stride, long long k_batch_stride,
                                      long long v_batch_stride, long long out_batch_stride, long long k_head_stride,
                                      long long v_head_stride, float scale, int dtype, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  return attn_entry(q, const_cast<void*>(k), const_cast<void*>(v), out, n_q, n_kv, 1, kv_len, d, k_head_stride,
                    v_head_stride, scale, dtype, workspace, workspace_bytes, nullptr, nullptr, 0, 0, 0, stream, n_batch,
                    BatchStrides{q_batch_stride, k_batch_stride, v_batch_stride, out_batch_stride});
}

extern "C" int std_gqa_decode_append(const void* q, void* k_cache, void* v_cache, const void* new_k, const void* new_v,
                                     void* out, int n_q, int n_kv, int kv_len, int d, long long k_head_stride,
                                     long long v_head_stride, long long new_head_stride, float scale, int dtype,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  return attn_entry(q, k_cache, v_cache, out, n_q, n_kv, 1, kv_len, d, k_head_stride, v_head_stride, scale, dtype,
                    workspace, workspace_bytes, new_k, new_v, new_head_stride, 0, 1, stream);
}

extern "C" size_t std_verify_attn_workspace_bytes(int n_q, int n_kv, int q_len, int kv_len, int d) {
  if (n_q <= 0 || n_kv <= 0 || n_q % n_kv != 0 || q_len < 1 || kv_len < q_len || d != D) return 0;
  const size_t a = attn_workspace_bytes(n_kv, (n_q / n_kv) * q_len, kv_len, STD_BF16);
  const size_t b = attn_workspace_bytes(n_kv, (n_q / n_kv) * q_len, kv_len, STD_F32);
  return a > b ? a : b;
}

extern "C" int std_verify_attn(const void* q, const void* k, const void* v, void* out, int n_q, int n_kv,
                               int q_len, int kv_len, int d, long long k_head_stride, long long v_head_stride,
                               float scale, int dtype, void* workspace, size_t workspace_bytes, void* stream) {
  return attn_entry(q, const_cast<void*>(k), const_cast<void*>(v), out, n_q, n_kv, q_len, kv_len, d, k_head_stride,
                    v_head_stride, scale, dtype, workspace, workspace_bytes, nullptr, nullptr, 0, 0, 0, stream);
}

extern "C" int std_verify_attn_append(const void* q, void* k_cache, void* v_cache, const void* new_k,
                                      const void* new_v, void* out, int n_q, int n_kv, int q_len, int kv_len, int d,
                                      long long k_head_stride, long long v_head_stride, long long new_head_stride,
                                      long long new_row_stride, float scale, int dtype, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  return attn_entry(q, k_cache, v_cache, out, n_q, n_kv, q_len, kv_len, d, k_head_stride, v_head_stride, scale, dtype,
                    workspace, workspace_bytes, new_k, new_v, new_head_stride, new_row_stride, q_len, stream);
}

extern "C" int std_attn_devlen(const void* q, const void* k_cache, const void* v_cache, void* out, int n_q, int n_kv,
                               int q_len, const int32_t* len_dev, int max_kv_len, int d, long long k_head_stride,
                               long long v_head_stride, float scale, int dtype, void* workspace,
                               size_t workspace_bytes, int32_t* status, void* stream) {
  if (!len_dev) return STD_E_NULL;
  return attn_entry(q, const_cast<void*>(k_cache), const_cast<void*>(v_cache), out, n_q, n_kv, q_len, max_kv_len, d,
                    k_head_stride, v_head_stride, scale, dtype, workspace, workspace_bytes, nullptr, nullptr, 0, 0, 0,
                    stream, 1, BatchStrides{0, 0, 0, 0}, len_dev,
                    GatherArgs{nullptr, 0, 0, 0, nullptr, nullptr, 0, 0, status});
}

extern "C" int std_gqa_decode_indexed(const void* q, const void* dense_k, const void* dense_v, int dense_rows,
                                      long long dense_k_head_stride, long long dense_v_head_stride,
                                      const int32_t* index, long long index_head_stride, int n_index,
                                      const void* k_cache, const void* v_cache, long long k_head_stride,
                                      long long v_head_stride, void* out, int n_q, int n_kv, int kv_len,
                                      const int32_t* len_dev, int d, float scale, int dtype, void* workspace,
                                      size_t workspace_bytes, int32_t* status, void* stream) {
  if (!index) return STD_E_NULL;
  const GatherArgs ga{index, index_head_stride, n_index, dense_rows, static_cast<const bf16_t*>(dense_k),
                      static_cast<const bf16_t*>(dense_v), dense_k_head_stride, dense_v_head_stride, status};
  return attn_entry(q, const_cast<void*>(k_cache), const_cast<void*>(v_cache), out, n_q, n_kv, 1, kv_len, d,
                    k_head_stride, v_head_stride, scale, dtype, workspace, workspace_bytes, nullptr, nullptr, 0, 0,
                    0, stream, 1, BatchStrides{0, 0, 0, 0}, len_dev, ga);
}

extern "C" int std_gqa_decode_noalloc(const void* q, const void* k, const void* v, void* out, int n_q, int n_kv,
                                      int kv_len, int d, long long k_head_stride, long long v_head_stride,
                                      float scale, int dtype, void* stream) {
  // The size check comes before any HIP call; attn_entry repeats the full validation.
  if (!q || !k || !v || !out) return STD_E_NULL;
  if (dtype != STD_F32 && dtype != STD_BF16 && dtype != STD_F16) return STD_E_DTYPE;
  if (d != D || n_q <= 0 || n_kv <= 0 || n_q % n_kv != 0 || kv_len < 1 || n_q / n_kv > kMaxRows) return STD_E_SHAPE;
  const size_t need = attn_workspace_bytes(n_kv, n_q / n_kv, kv_len, dtype);
  if (need > kNoAllocScratchBytes) return STD_E_WORKSPACE;
  void* ws = nullptr;
  if (need > 0) {
    const int s = scratch_address(static_cast<hipStream_t>(stream), &ws);
    if (s != 0) return s;
  }
  return attn_entry(q, const_cast<void*>(k), const_cast<void*>(v), out, n_q, n_kv, 1, kv_len, d, k_head_stride,
                    v_head_stride, scale, dtype, ws, need > 0 ? kNoAllocScratchBytes : 0, nullptr, nullptr, 0, 0, 0,
                    stream);
}

extern "C" size_t std_verify_attn_collect_workspace_bytes(int n_q, int n_kv, int q_len, int kv_len, int d,
                                                          int vis_begin, int vis_end) {
  if (n_q <= 0 || n_kv <= 0 || n_q % n_kv != 0 || q_len < 1 || kv_len < q_len || d != D) return 0;
  if (vis_begin < 0 || vis_end <= vis_begin || vis_end > kv_len) return 0;
  if (coll_chunk(n_q / n_kv) < 1) return 0;
  return coll_layout(n_kv, n_q / n_kv, q_len, kv_len, vis_begin, vis_end, 2, 4).total;
}

extern "C" int std_verify_attn_collect(const void* q, void* k_cache, void* v_cache, const void* new_k,
                                       const void* new_v, void* out, int n_q, int n_kv, int q_len, int kv_len,
                                       int d, long long k_head_stride, long long v_head_stride,
                                       long long new_head_stride, long long new_row_stride, float scale, int dtype,
                                       int vis_begin, int vis_end, float* scores, long long scores_head_stride,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  return verify_collect_entry(q, k_cache, v_cache, out, n_q, n_kv, q_len, kv_len, nullptr, d, k_head_stride,
                              v_head_stride, scale, dtype, new_k, new_v, new_head_stride, new_row_stride, vis_begin,
                              vis_end, nullptr, nullptr, vis_end - vis_begin, scores, scores_head_stride, workspace,
                              workspace_bytes, nullptr, stream);
}

extern "C" int std_verify_attn_collect_ex(const void* q, void* k_cache, void* v_cache, const void* new_k,
                                          const void* new_v, void* out, int n_q, int n_kv, int q_len, int kv_len,
                                          const int32_t* len_dev, int d, long long k_head_stride,
                                          long long v_head_stride, long long new_head_stride,
                                          long long new_row_stride, float scale, int dtype, int vis_begin,
                                          int vis_end, const uint32_t* vis_mask, const int32_t* vis_rank,
                                          int n_visual, float* scores, long long scores_head_stride, void* workspace,
                                          size_t workspace_bytes, int32_t* status, void* stream) {
  return verify_collect_entry(q, k_cache, v_cache, out, n_q, n_kv, q_len, kv_len, len_dev, d, k_head_stride,
                              v_head_stride, scale, dtype, new_k, new_v, new_head_stride, new_row_stride, vis_begin,
                              vis_end, vis_mask, vis_rank, n_visual, scores, scores_head_stride, workspace,
                              workspace_bytes, status, stream);
}

#if STD_PHASE_STAMPS
// Timing build only: copies the stamp rows (which = 0, n words) or the merge
// stamps (which = 1) to host memory.
extern "C" int std_phase_stamps(void* host, int which, size_t n) {
  if (which == 0)
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(phase_stamps),
                                    std::min(n, (size_t)kStampWgs * kStampSlots) * 8, 0, hipMemcpyDeviceToHost);
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(merge_stamps), std::min(n, (size_t)kStampMerge * 2) * 8, 0,
                                  hipMemcpyDeviceToHost);
}
#endif
