// Shared pieces of the LDS-staged expert GEMMs (gemm_dense.hip, MXFP4
// weights; gemm_dense8.hip, FP8 weights): gfx950 direct-to-LDS loads issued
// as inline assembly, explicit vector-memory waits, fence-free barriers and
// the swizzled activation-tile layout.
#pragma once
#include <cstdint>
#include <hip/hip_runtime.h>

namespace sllm {
namespace dma {

typedef __attribute__((address_space(3))) void* lds_void;

// LDS offset of 16-byte chunk c (K bytes [16 c, +16)) of tile row r: the
// chunk index is XOR-swizzled with the row, so that the 16 rows an MFMA
// fragment read touches spread over the banks.
__device__ __forceinline__ int a_off(int r, int c) {
  return r * 128 + ((c ^ (r & 7)) << 4);
}

__device__ __forceinline__ uint32_t e8m0_of(float pow2) {
  return (__float_as_uint(pow2) >> 23) & 0xFF;
}

// s_waitcnt for the vector-memory counter alone (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima)
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier that orders memory operations in the compiler but
// waits for nothing in the hardware; `lds` also waits for this wave's LDS
// operations first (for data exchanged through LDS).
__device__ __forceinline__ void bar_only() { asm volatile("s_barrier" ::: "memory"); }
__device__ __forceinline__ void bar_lds() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Direct-to-LDS load of 16 (or 4) bytes per lane: lane i's bytes land at
// l + 16 i (4 i); l is wave-uniform. Written as inline assembly so that the
// compiler, which does not see the LDS write, adds no wait of its own
// before the step's LDS reads (it would wait for every load in flight,
// the prefetched stages included); the steps wait for their own stage
// with explicit vmcnt waits instead.
__device__ __forceinline__ void to_lds(const void* g, uint8_t* l, int bytes) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void)l);
  if (bytes == 16)
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(g), "s"(m0) : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off"
                 :: "v"(g), "s"(m0) : "memory", "m0");
}


}  // namespace dma
}  // namespace sllm
