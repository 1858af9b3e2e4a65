// Global -> LDS copies (CDNA3/4 global_load_lds_dwordx4) and the hand-tracked
// waits they need. The compiler does not see these copies in its wait
// counters, so a kernel that uses them keeps its own vector loads out of the
// copies' way (or makes its data arrive through copies as well) and waits with
// wait_vm / wait_copies_and_barrier.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hy3x {

typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const lds_void_t *)p;
}

// 16-byte global -> LDS copy: lane i of the wave writes LDS bytes
// [m0 + 16 i, m0 + 16 i + 16) (m0 = lds, wave-uniform).
__device__ __forceinline__ void dma16(const void *src, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds) : "memory");
}

// The same with a wave-uniform base (scalar registers) and a per-lane 32-bit
// byte offset: the address costs no vector instruction.
__device__ __forceinline__ void dma16_s(const void *sbase, uint32_t voff, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds) : "memory");
}

// Wait until at most N of this wave's vector-memory operations are in flight.
// Copies complete in issue order, so this makes the wave's first copies
// (all but the last N) visible to the wave itself.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt immediate");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// wait_vm<N> plus all LDS operations done, then the workgroup barrier.
template <int N>
__device__ __forceinline__ void wait_copies_and_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt immediate");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

}  // namespace hy3x
