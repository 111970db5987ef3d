// LDS-DMA staging helpers shared by the matrix-core kernels (gfx950).
//
// global_load_lds_dwordx4 copies 16 bytes per lane from global memory straight into LDS at
// M0 + 16 * lane, without VGPRs or ds_write instructions. It is issued through inline asm: the
// compiler's own handling of LDS-DMA makes every later LDS read wait for all outstanding loads
// (it cannot tell a ring of stage buffers apart), and __syncthreads waits for every load at each
// barrier. Kernels using these helpers wait for exactly the loads of the stage they are about to
// read (wait_vmcnt), then meet at stage_barrier.
#pragma once

#include <hip/hip_runtime.h>

namespace mnn {
namespace dev {

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  // gfx9 s_waitcnt encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at [15:14]
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Waits until this wave's LDS reads and writes have completed.
__device__ __forceinline__ void wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt((0xF) | (0x3 << 14) | (0x7 << 4) | (0x0 << 8));
}

// Workgroup barrier without the memory fence of __syncthreads. The empty asm statements keep the
// compiler from moving memory accesses across it: the s_barrier intrinsic alone is not a memory
// operation to the optimiser.
__device__ __forceinline__ void stage_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// 16 bytes per lane from `src` (4-byte aligned is enough) into LDS at byte address
// `lds` + 16 * lane; `lds` must be wave-uniform. M0 is named as clobbered for the reader; the
// compiler treats it as reserved and sets it itself before any instruction of its own that reads it.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(const float* src, unsigned lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds)
               : "memory", "m0");
}
// Same copy with a wave-uniform 64-bit base in SGPRs and a per-lane 32-bit byte offset: the
// address arithmetic of a moving window is then one scalar add per load, no VALU work.
__device__ __forceinline__ void lds_dma16_s(const float* sbase, unsigned voff, unsigned lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase),
               "s"(lds)
               : "memory", "m0");
}
// 4 bytes per lane through a buffer resource at per-lane byte offset `voff` (+ `soff`) into LDS at
// byte address `lds` + 4 * lane (`lds` wave-uniform). An offset past the resource's range reads
// zero, so padding needs no branch.
__device__ __forceinline__ void lds_dma4_buf(__amdgpu_buffer_rsrc_t rsrc, unsigned voff,
                                             unsigned soff, unsigned lds) {
  asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dword %0, %1, %2 offen lds" ::"v"(voff), "s"(rsrc),
               "s"(soff), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// LDS byte address of a __shared__ object.
template <typename T>
__device__ __forceinline__ unsigned lds_address(T* p) {
  return (unsigned)(size_t)(__attribute__((address_space(3))) T*)p;
}

// Slot of 16-byte chunk c (of 8) in row r of a [rows][32 floats] tile: c ^ f(r), f(r) = (r + r/8)
// mod 8. Fragment reads of 32 consecutive rows at one chunk then hit distinct banks.
__device__ __forceinline__ int chunk_swizzle(int r) { return (r + (r >> 3)) & 7; }

// XCD-aware renumbering of a gx x gy grid: workgroups are dealt round robin over the 8 XCDs, so
// consecutive logical tiles are given to workgroups of one XCD (sharing an operand panel in its L2).
__device__ __forceinline__ int xcd_logical_tile(int lin, int total) {
  constexpr int kXcds = 8;
  const int xcd = lin % kXcds, slot = lin / kXcds;
  const int q = total / kXcds, r = total % kXcds;
  return xcd < r ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
}

}  // namespace dev
}  // namespace mnn
