// vmem.h -- hand-issued vector-memory instructions shared by the MFMA kernels
// (Q8 GEMM, encoder attention): buffer descriptors, loads into VGPRs, LDS DMA
// and the wait-then-barrier that publishes a DMA'd stage to the workgroup.
#pragma once

#include "common.h"

namespace madi {

typedef __attribute__((address_space(3))) uint8_t lds_u8;

// A kernel that issues every vector-memory instruction through these gets no
// vmcnt waits from the compiler (its conservative counts stalled on loads
// issued chunks later); the kernel waits explicitly with the exact counts of
// its fixed issue pattern.  M0 is written only here.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"

// Raw (stride 0) buffer descriptor over [base, base + bytes): SGPR words.
// bytes = 0 gives a descriptor whose every load returns zeros without
// touching memory.  Range checks cover the per-lane offset only, so every
// real load keeps its address in bounds by construction.
typedef u32x4 desc_t;
__device__ inline desc_t make_desc(const void *base, uint32_t bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  return (desc_t){(uint32_t)b, (uint32_t)(b >> 32) & 0xffffu, bytes, 0x00020000u};
}

// The scalar offset operand of a buffer access.  Offsets are uniform, but the
// compiler may compute one on the vector ALU (e.g. a clamp it folds into a
// vector compare); readfirstlane returns it to an SGPR and costs nothing when
// it is already there.
__device__ inline uint32_t sgpr(uint32_t x) { return __builtin_amdgcn_readfirstlane(x); }

// 16 bytes per lane at soff + voff + OFF into VGPRs.
template <int OFF = 0>
__device__ inline void vload16(u32x4 &v, desc_t d, uint32_t voff, uint32_t soff) {
  static_assert(OFF >= 0 && OFF < 4096, "instruction offset range");
  asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen offset:%4"
               : "=v"(v) : "v"(voff), "s"(d), "s"(sgpr(soff)), "n"(OFF));
}
// 2 bytes per lane (zero-extended) at soff + voff into a VGPR.
__device__ inline void vload2(uint32_t &v, desc_t d, uint32_t voff, uint32_t soff) {
  asm volatile("buffer_load_ushort %0, %1, %2, %3 offen"
               : "=v"(v) : "v"(voff), "s"(d), "s"(sgpr(soff)));
}
// One wave-wide DMA of 16 bytes per lane: buffer bytes [soff + voff + OFF,
// +16) -> LDS m0 + OFF + 16*lane (the instruction offset moves both
// addresses), so one M0 value serves all of a chunk's DMAs.  The first DMA
// after M0 changes waits the one state an M0 write needs before an LDS DMA.
template <int OFF, bool FIRST>
__device__ inline void dma16(desc_t d, uint32_t voff, uint32_t soff, uint32_t m0) {
  static_assert(OFF >= 0 && OFF < 4096, "instruction offset range");
  if constexpr (FIRST)
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen offset:%3 lds"
                 ::"v"(voff), "s"(d), "s"(sgpr(soff)), "n"(OFF), "{m0}"(sgpr(m0)) : "memory");
  else
    asm volatile("buffer_load_dwordx4 %0, %1, %2 offen offset:%3 lds"
                 ::"v"(voff), "s"(d), "s"(sgpr(soff)), "n"(OFF), "{m0}"(sgpr(m0)) : "memory");
}
#pragma clang diagnostic pop

__device__ inline uint32_t lds_addr(const uint8_t *p) {
  return (uint32_t)(uintptr_t)(const lds_u8 *)p;
}

// Wait until at most N of this wave's vector-memory ops and none of its LDS
// reads are outstanding, then meet the other waves.  One asm statement, so no
// LDS access can be scheduled between the wait and the barrier.
template <int N>
__device__ inline void wait_then_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

}  // namespace madi
