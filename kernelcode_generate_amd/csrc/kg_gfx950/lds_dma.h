// HBM -> LDS copies with global_load_lds_dwordx4 and the explicit waits they need.
//
// The copies are issued through inline asm so that the compiler neither tracks nor waits
// for them (its own tracking of global_load_lds inserts vmcnt(0) before every LDS read).
// The waits below are therefore the only synchronisation: a wave waits for its own copies
// with s_waitcnt vmcnt, then meets the other waves at s_barrier; the empty asm statement
// after the barrier keeps LDS reads from being moved across it.
// Each copy statement sets M0 itself and lists it as clobbered; clang warns that M0 is a
// reserved register. Nothing else in these kernels reads M0 (gfx9 LDS instructions do not
// use it), so no value the compiler keeps there can be lost.
#pragma once

#include "common.h"

namespace kg_gfx950 {

// Wait until at most N of this wave's vector-memory ops (copies included) are outstanding
// and all of its LDS ops are done, then meet the other waves of the workgroup.
template <int N>
__device__ __forceinline__ void wait_and_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(N) : "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// 16 bytes per lane: lane l's data lands at LDS byte lds_base + 16*l (lds_base must be
// wave-uniform; it goes through M0). gptr is a per-lane 64-bit address.
__device__ __forceinline__ void g2lds16(const void* gptr, const void* lds_base) {
  const uint32_t m0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds_base;
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off"
      :
      : "v"(gptr), "s"(m0)
      : "memory", "m0");
}

// Same with the LDS byte address given directly.
__device__ __forceinline__ void g2lds16_m(const void* gptr, uint32_t m0) {
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off"
      :
      : "v"(gptr), "s"(m0)
      : "memory", "m0");
}

// 16 bytes per lane with a wave-uniform 64-bit base (SGPRs) and a per-lane 32-bit byte
// offset: lane l's data lands at LDS byte m0 + 16*l. (No immediate offset is used: the
// instruction's offset field would also move the LDS address.)
__device__ __forceinline__ void g2lds16_s(uint32_t voff, const void* sbase, uint32_t m0) {
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(voff), "s"(sbase), "s"(m0)
      : "memory", "m0");
}

// Same copy through a raw buffer resource (base = sbase, range kBufRange bytes, stride 0):
// a lane whose voff is kBufOOB lies outside the range, reads nothing and lands zeros in
// LDS. This is how the edges of ragged tiles are zero-filled without a branch. Every valid
// voff must stay below kBufRange. Word 3 is the gfx9-family raw-buffer configuration
// (32-bit data format, no swizzle).
constexpr uint32_t kBufRange = 0x80000000u;
constexpr uint32_t kBufOOB = 0x80000000u;
__device__ __forceinline__ void buf2lds16_s(uint32_t voff, const void* sbase, uint32_t m0) {
  const uint64_t p = (uint64_t)(uintptr_t)sbase;
  u32x4 rsrc;
  rsrc[0] = (uint32_t)p;
  rsrc[1] = (uint32_t)(p >> 32);  // stride field (bits 48-61 of the resource) stays 0
  rsrc[2] = kBufRange;
  rsrc[3] = 0x00020000u;
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %0, %1, 0 offen lds"
      :
      : "v"(voff), "s"(rsrc), "s"(m0)
      : "memory", "m0");
}

// Same copy through a raw buffer resource over [sbase, sbase + range) bytes (range a multiple
// of 16, at most kBufRange): a lane whose voff lies at or past range reads nothing and lands
// zeros in LDS.
__device__ __forceinline__ void buf2lds16_r(uint32_t voff, const void* sbase, uint32_t range, uint32_t m0) {
  const uint64_t p = (uint64_t)(uintptr_t)sbase;
  u32x4 rsrc;
  rsrc[0] = (uint32_t)p;
  rsrc[1] = (uint32_t)(p >> 32);
  rsrc[2] = range;
  rsrc[3] = 0x00020000u;
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %0, %1, 0 offen lds"
      :
      : "v"(voff), "s"(rsrc), "s"(m0)
      : "memory", "m0");
}

// LDS byte address of a shared-memory object (what M0 and ds_* addresses take).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

template <int N>
struct Int {
  static constexpr int value = N;
};

// f(Int<0>{}), f(Int<1>{}), ..., f(Int<N-1>{}), expanded at compile time (`#pragma unroll`
// gives up on large bodies and leaves a runtime index).
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(Int<I>{});
    static_for<N, I + 1>(f);
  }
}
}  // namespace kg_gfx950
