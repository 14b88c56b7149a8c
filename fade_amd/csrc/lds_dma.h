// Direct global -> LDS loads (global_load_lds_*) and s_waitcnt immediates for
// kernels that pipeline tiles through LDS with explicit vmcnt accounting.
//
// The compiler does not see these loads: a kernel that issues them waits for
// them itself (s_waitcnt vmcnt(n) with n = the loads it issued after the ones
// it needs), and must not rely on compiler-inserted waits for them.  LDS
// address = m0 (the wave-uniform base) + lane * size.
//
// Hazards the hardware does not interlock (GFX9-family rules, which the
// compiler's hazard recognizer applies to its own code but cannot apply inside
// inline asm): an LDS DMA reads m0 no sooner than one wait state after an SALU
// write of m0, else it may take the previous base and land in the previous
// load's slot; a VMEM instruction reads an SGPR address no sooner than five
// wait states after a VALU write of it (e.g. v_readfirstlane_b32 producing the
// `sbase` operand).  Hence s_nop 0 after the m0 write, and s_nop 3 (+ the
// s_mov itself = 5) in the forms with a scalar base.
#pragma once

#include <stdint.h>

namespace fade {

// s_waitcnt immediate: at most n vector-memory ops outstanding (expcnt, lgkmcnt untouched).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int kLgkm0 = 15 | (3 << 14) | (7 << 4);  // lgkmcnt(0) only

__device__ __forceinline__ void lds_dma16(const void* g, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_base) : "memory", "m0");
}
__device__ __forceinline__ void lds_dma2(const void* g, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_ushort %0, off" ::"v"(g), "s"(lds_base) : "memory", "m0");
}
__device__ __forceinline__ void lds_dma4(const void* g, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds_base) : "memory", "m0");
}
// Same with a wave-uniform base address and a 32-bit per-lane byte offset.
__device__ __forceinline__ void lds_dma16(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 3\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds_base)
               : "memory", "m0");
}
__device__ __forceinline__ void lds_dma2(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 3\n\tglobal_load_lds_ushort %0, %1" ::"v"(voff), "s"(sbase), "s"(lds_base)
               : "memory", "m0");
}
__device__ __forceinline__ void lds_dma4(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 3\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "s"(lds_base)
               : "memory", "m0");
}

// Non-temporal forms (cache policy nt: the lines are streamed, not kept) for
// data read once per launch, e.g. the decode's K/V tiles.
__device__ __forceinline__ void lds_dma16_nt(const void* g, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(g), "s"(lds_base) : "memory", "m0");
}
__device__ __forceinline__ void lds_dma16_nt(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 3\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sbase), "s"(lds_base)
               : "memory", "m0");
}
__device__ __forceinline__ void lds_dma2_nt(const void* g, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_ushort %0, off nt" ::"v"(g), "s"(lds_base) : "memory", "m0");
}
__device__ __forceinline__ void lds_dma2_nt(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 3\n\tglobal_load_lds_ushort %0, %1 nt" ::"v"(voff), "s"(sbase), "s"(lds_base)
               : "memory", "m0");
}
__device__ __forceinline__ void lds_dma4_nt(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 3\n\tglobal_load_lds_dword %0, %1 nt" ::"v"(voff), "s"(sbase), "s"(lds_base)
               : "memory", "m0");
}

}  // namespace fade
