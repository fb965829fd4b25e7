// Streaming-read ceiling of the HBM: reads a buffer once in the access
// patterns the attention kernels use, so that their achieved bandwidth can be
// set against what a kernel that only reads reaches on the same part.
//
// A tile is 32 KiB. Register modes: 256 threads, each issuing eight 16-byte
// loads per tile (a wave reads 1 KiB contiguous per load). LDS modes: the
// attention kernels' ring of four 32 KiB stages filled by global_load_lds_dwordx4,
// a tile being 16 KiB from the first half of the buffer and 16 KiB from the
// second (as a K tile and a V tile), with the verify kernel's schedule (eight
// waves, two tiles in flight) or the decode key split's (four waves, three
// tiles in flight). Tiles go to workgroups either as one contiguous chunk per
// workgroup (the attention kernels' split of a head's key range) or dealt
// round-robin, with the default or the non-temporal load policy (the
// attention kernels stream long key ranges non-temporally). Nothing is written except one word per workgroup under a
// condition that the data never meets, which keeps the loads live.
#include <climits>

#include "common.h"
#include "lds_dma.h"

namespace stdhip {
namespace {

constexpr int kTileBytes = 32768;
constexpr uint32_t kNever = 0x9e3779b9u;

template <bool RR>
__global__ void __launch_bounds__(256)
stream_regs_kernel(const uint4* __restrict__ src, int ntiles, int per, int n_wg, uint32_t* __restrict__ sink) {
  const int b = blockIdx.x;
  const int t0 = RR ? b : b * per, t_end = RR ? ntiles : t0 + per, step = RR ? n_wg : 1;
  uint32_t acc = 0;
  for (int t = t0; t < t_end; t += step) {
    const uint4* p = src + (long long)t * (kTileBytes / 16) + threadIdx.x;
    uint4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = p[j * 256];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  }
  if (acc == kNever) sink[b] = acc;
}

template <int WAVES, int AHEAD, bool RR, bool NTL = false>
__global__ void __launch_bounds__(64 * WAVES)
stream_lds_kernel(const char* __restrict__ ha, const char* __restrict__ hb, int ntiles, int per, int n_wg,
                  uint32_t* __restrict__ sink) {
  constexpr int kStages = 4;
  constexpr int kHalf = kTileBytes / 2;
  constexpr int kSegs = 16 / WAVES;          // 1 KiB segments of each half per wave per tile
  static_assert(AHEAD >= 2 && AHEAD <= kStages, "one to three tiles in flight beside the one being read");
  __shared__ __align__(16) char ring[kStages * kTileBytes];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int b = blockIdx.x;
  const int t0 = RR ? b : b * per, step = RR ? n_wg : 1;
  const int n = RR ? (ntiles - b + n_wg - 1) / n_wg : per;
  auto stage = [&](int u) { return ring + (u & (kStages - 1)) * kTileBytes; };
  auto issue = [&](int u) {
    const long long t = t0 + (long long)u * step;
    const char* a = ha + t * kHalf;
    const char* c = hb + t * kHalf;
    const uint32_t dst0 = lds_addr(stage(u));
#pragma unroll
    for (int j = 0; j < kSegs; ++j) {
      const int seg = w * kSegs + j;
      const uint32_t off = (uint32_t)(seg * 1024 + lane * 16);
      lds_dma16_sbase<NTL>(a, off, dst0 + seg * 1024);
      lds_dma16_sbase<NTL>(c, off, dst0 + kHalf + seg * 1024);
    }
  };
#pragma unroll
  for (int u = 0; u < AHEAD - 1; ++u)
    if (u < n) issue(u);
  uint32_t acc = 0;
  for (int u = 0; u < n; ++u) {
    // tiles issued so far: 0 .. min(u + AHEAD - 2, n - 1); tile u must have landed
    wait_vm_ahead<2 * kSegs>(min(AHEAD - 2, n - 1 - u));
    wg_barrier();
    // the stage of tile u + AHEAD - 1 last held tile u + AHEAD - 5 (<= u - 1),
    // which every wave finished before this barrier
    if (u + AHEAD - 1 < n) issue(u + AHEAD - 1);
    acc ^= *reinterpret_cast<const uint32_t*>(stage(u) + threadIdx.x * 16);
  }
  if (acc == kNever) sink[b] = acc;
}

}  // namespace
}  // namespace stdhip

using namespace stdhip;

// Measurement helper with no counterpart in the reference: the streaming-read
// ceiling that the attention kernels' bandwidth is compared against.
extern "C" int std_stream_read(const void* src, size_t bytes, int mode, int n_workgroups, uint32_t* sink,
                               void* stream) {
  if (!src || !sink) return STD_E_NULL;
  if (mode < 0 || mode > 7) return STD_E_SHAPE;
  if (bytes == 0 || bytes % kTileBytes != 0 || bytes / kTileBytes > (size_t)INT_MAX) return STD_E_SHAPE;
  if (n_workgroups < 1 || n_workgroups > 65535) return STD_E_SHAPE;
  if (!aligned16(src)) return STD_E_ALIGN;
  const int ntiles = (int)(bytes / kTileBytes);
  const bool rr = (mode & 1) != 0 || mode == 6;
  if (rr ? n_workgroups > ntiles : ntiles % n_workgroups != 0) return STD_E_SHAPE;
  const int per = rr ? 0 : ntiles / n_workgroups;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(n_workgroups);
  const char* a = static_cast<const char*>(src);
  const char* b = a + bytes / 2;
  switch (mode) {
    case 0:
      hipLaunchKernelGGL(stream_regs_kernel<false>, grid, dim3(256), 0, st, static_cast<const uint4*>(src), ntiles,
                         per, n_workgroups, sink);
      break;
    case 1:
      hipLaunchKernelGGL(stream_regs_kernel<true>, grid, dim3(256), 0, st, static_cast<const uint4*>(src), ntiles,
                         per, n_workgroups, sink);
      break;
    case 2:
      hipLaunchKernelGGL((stream_lds_kernel<8, 3, false>), grid, dim3(512), 0, st, a, b, ntiles, per, n_workgroups,
                         sink);
      break;
    case 3:
      hipLaunchKernelGGL((stream_lds_kernel<8, 3, true>), grid, dim3(512), 0, st, a, b, ntiles, per, n_workgroups,
                         sink);
      break;
    case 4:
      hipLaunchKernelGGL((stream_lds_kernel<4, 4, false>), grid, dim3(256), 0, st, a, b, ntiles, per, n_workgroups,
                         sink);
      break;
    case 5:
      hipLaunchKernelGGL((stream_lds_kernel<4, 4, true>), grid, dim3(256), 0, st, a, b, ntiles, per, n_workgroups,
                         sink);
      break;
    case 6:
      hipLaunchKernelGGL((stream_lds_kernel<8, 3, true, true>), grid, dim3(512), 0, st, a, b, ntiles, per,
                         n_workgroups, sink);
      break;
    default:
      hipLaunchKernelGGL((stream_lds_kernel<4, 4, true, true>), grid, dim3(256), 0, st, a, b, ntiles, per,
                         n_workgroups, sink);
      break;
  }
  return launch_status();
}
