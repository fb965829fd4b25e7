// HBM -> LDS direct copies (global_load_lds_dwordx4) and the waits and
// barriers that order them, shared by the attention kernels and the
// streaming-read ceiling kernel.
#pragma once

#include "common.h"

namespace stdhip {

// s_waitcnt immediate (gfx9 encoding) that waits until at most n vector-memory
// operations of this wave are outstanding, leaving the other counters alone.
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
// s_waitcnt immediate that waits for this wave's LDS (and scalar memory)
// operations only, leaving vector-memory loads such as the DMA ring in flight.
constexpr int waitcnt_lgkm0() { return 15 | (3 << 14) | (7 << 4); }

// One wave-wide global_load_lds_dwordx4: lane i copies 16 bytes from
// sbase + voff (a wave-uniform 64-bit base in SGPRs plus a 32-bit per-lane
// byte offset, the global saddr form) to LDS byte lds_base + 16 i. Issued through inline asm on purpose:
// the compiler's own LDS-DMA tracking cannot tell the ring stages apart and
// would put s_waitcnt vmcnt(0) before every LDS read, draining the whole
// prefetch each tile. Completion is instead ordered explicitly by
// wait_vm_ahead (vmcnt) followed by a workgroup barrier before any wave
// reads the stage; the "memory" clobber keeps the compiler from moving LDS
// accesses across the issue. The compiler inserts no hazard wait states for
// inline asm, so the asm carries its own: s_nop 4 (5 wait states) covers both
// the M0 write before an LDS DMA and an SGPR operand written by a VALU
// instruction (v_readfirstlane) shortly before a VMEM instruction reads it.
// NTL: a non-temporal load (the `nt` cache policy): for a stream that is read
// once, the lines are not kept for reuse in the caches, which leaves them to the
// data that is (measured on MI355X: the 128k verify 55.9 -> 51.7 us, the 128k
// dense decode 50.6 -> 46.1 us per layer); a cache that is read again soon
// (the draft's 1024-key compact cache between steps) keeps the default policy.
template <bool NTL = false>
__device__ __forceinline__ void lds_dma16_sbase(const void* sbase, uint32_t voff, uint32_t lds_base) {
  // readfirstlane pins the wave-uniform operands to SGPRs even where the
  // compiler cannot prove them uniform (it folds away when they already are).
  const uint64_t b = reinterpret_cast<uint64_t>(sbase);
  // (readfirstlane returns int: widen through uint32_t, never sign-extend.)
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b)));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b >> 32)));
  const uint64_t base = static_cast<uint64_t>(lo) | (static_cast<uint64_t>(hi) << 32);
  const uint32_t lds = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(lds_base));
  if constexpr (NTL)
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1 nt"
                 :
                 : "v"(voff), "s"(base), "s"(lds)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(base), "s"(lds)
                 : "memory", "m0");
}

// The same copy from a per-lane 64-bit address (gathered rows).
__device__ __forceinline__ void lds_dma16_vaddr(const void* addr, uint32_t lds_base) {
  const uint32_t lds = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(lds_base));
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(addr), "s"(lds) : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  typedef const __attribute__((address_space(3))) char* lds_cptr;
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_cptr)(p)));
}

// Workgroup barrier without the memory fence of __syncthreads (which would
// wait for every outstanding load); the empty asm statements keep the
// compiler from moving LDS accesses across it.
__device__ __forceinline__ void wg_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Wait until the tile `ahead` tiles before the newest issued one has landed
// (each tile is PER_TILE DMA instructions per wave).
template <int PER_TILE>
__device__ __forceinline__ void wait_vm_ahead(int ahead) {
  if (ahead >= 2) __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * PER_TILE));
  else if (ahead == 1) __builtin_amdgcn_s_waitcnt(waitcnt_vm(PER_TILE));
  else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
}

}  // namespace stdhip
