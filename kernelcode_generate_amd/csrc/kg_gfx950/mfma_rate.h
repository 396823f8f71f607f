// Measurement aid: the sustained rate of v_mfma_f32_32x32x16 or v_mfma_f32_16x16x32 (the same
// FLOP per cycle; 32 and 16 cycles per instruction) with no operand movement at all, on given
// operand data. Every wave loads 8 operand registers once and then issues back-to-back MFMAs
// into 8 independent accumulators (each one is reused 8 instructions later, past the
// dependent-issue latency of either shape). With random 16-bit operands the part lowers its clock under
// this load; with all-zero operands it does not: the difference is the power the data's
// switching activity costs, and the random-operand rate is the ceiling any kernel that also
// moves its operands can approach.
#pragma once

#include "common.h"

namespace kg_gfx950 {

constexpr int kMfmaRateThreads = 256;
constexpr int kMfmaRateOperands = 1 << 16;  // 16-byte operand vectors in the source buffer

// times[2*b] = shader-clock ticks (s_memtime) and times[2*b+1] = 100 MHz ticks (s_memrealtime)
// spent by workgroup b's first wave in its MFMA loop.
// kM = 32: v_mfma_f32_32x32x16 (16 accumulator registers); kM = 16: v_mfma_f32_16x16x32 (4).
// For the 16x16x32 form an occupancy bound of 2 workgroups per CU keeps the accumulators in
// VGPRs: with the default bound the compiler places them in AGPRs and copies them between
// AGPRs and VGPRs on every iteration (52 moves per 8 MFMAs). The 32x32x16 form keeps the
// default bound (its loop is move-free either way, and the bound would cap its occupancy).
template <typename Tag, int kM>
__global__ __launch_bounds__(kMfmaRateThreads, kM == 16 ? 2 : 1) void mfma_rate_kernel(const u32x4* __restrict__ operands,
                                                                     unsigned long long* __restrict__ times,
                                                                     float* __restrict__ sink, int iters) {
  using Acc = std::conditional_t<kM == 32, f32x16, f32x4>;
  constexpr int kAccRegs = kM == 32 ? 16 : 4;
  const int t = blockIdx.x * kMfmaRateThreads + threadIdx.x;
  u32x4 a[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) a[j] = operands[(t * 8 + j) & (kMfmaRateOperands - 1)];
  Acc acc[8] = {};
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if constexpr (kM == 32) acc[j] = Half16<Tag>::mfma32(a[j], a[(j + 3) & 7], acc[j]);
      else acc[j] = Half16<Tag>::mfma16(a[j], a[(j + 3) & 7], acc[j]);
    }
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int e = 0; e < kAccRegs; ++e) s += acc[j][e];
  sink[t] = s;
  if (threadIdx.x == 0) {
    times[2 * blockIdx.x] = t1 - t0;
    times[2 * blockIdx.x + 1] = r1 - r0;
  }
}

}  // namespace kg_gfx950
