// fp32 GEMM on gfx950 matrix cores: out[M,N] = lhs[M,K] @ rhs[K,N] (+ bias[N]), all fp32,
// row-major, fp32 products and accumulation (v_mfma_f32_32x32x2_f32).
//
// The fp32 MFMA issues once per 64 cycles (1/16 of the bf16 rate), so this kernel is
// bound by its MFMAs and everything else is arranged to stay out of their way:
//   * 128 x 128 tiles, 4 waves in a 2 x 2 layout of 64 x 64 (2 x 2 blocks of 32 x 32, 64
//     fp32 accumulators per lane), 48 KiB of LDS, so three workgroups share a CU and their
//     waves cover each other's LDS and barrier waits;
//   * K advances in 16-deep slices through a 3-stage LDS ring filled by
//     global_load_lds_dwordx4 (HBM/L2 -> LDS, no registers), two slices ahead;
//   * the MFMA is issued as C^T = B^T A^T (rhs fragment as operand A), so each lane ends
//     with 4 consecutive columns of one output row (one 16-byte store).
// The contraction order inside a slice is permuted so that operand reads are wide: lane
// half h (lane / 32) of k-step kk covers k = 8 ks + 4 h + kk of 16-deep half ks, so one
// ds_read_b128 of an lhs row gives a lane its operands for four k-steps; the rhs operand is
// one fp32 of row k, 32 consecutive columns per lane half (ds_read_b32).
// LDS (64 banks of 4 bytes): lhs slices are [m][16 k] rows of 64 bytes with 16-byte chunk
// c stored at c ^ ((m >> 2) & 3); rhs slices are [k][128 n] rows of 512 bytes with chunk c
// at c ^ 8((k >> 2) & 1): the b128 lhs reads of 16 lanes and the b32 rhs reads of 64 lanes
// each hit distinct banks.
// kRagged: M % 128, N % 128 or K % 16 non-zero; copies go through buffer loads whose
// out-of-range lanes land zeros (rows >= M, chunks past N, k >= K) and stores are masked.
// Host requirements: K % 4 == 0, N % 4 == 0, row strides multiples of 4 and at most 2^22
// elements, 16-byte aligned base pointers.
#pragma once

#include "common.h"
#include "lds_dma.h"

namespace kg_gfx950 {

namespace gemmf {
constexpr int kTile = 128;
constexpr int kBK = 16;
constexpr int kDefaultStages = 3;  // LDS ring depth unless the lowering asks for another
constexpr int kThreads = 256;
constexpr int kStageBytes = 2 * kTile * kBK * 4;  // lhs + rhs slice, 16 KiB
__device__ __forceinline__ int a_mask(int m) { return (m >> 2) & 3; }
__device__ __forceinline__ int b_mask(int k) { return 8 * ((k >> 2) & 1); }
}  // namespace gemmf

// kBias: 0 none, 1 fp32 bias; kStages: the LDS ring depth (slices are copied kStages - 1 ahead)
template <int kBias, bool kRagged, int kStages>
__global__ __launch_bounds__(gemmf::kThreads, 3) void gemm_f32_mfma_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, const float* __restrict__ bias,
    int M, int N, int K, long long lda, long long ldb, long long ldc) {
  using namespace gemmf;
  static_assert(kStages >= 2 && kStages <= 4, "LDS ring depth");
  __shared__ __attribute__((aligned(1024))) char lds[kStages * kStageBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1;  // 64-row half of the tile
  const int wn = wave & 1;   // 64-column half

  const int tiles_n = kRagged ? (N + kTile - 1) / kTile : N / kTile;
  const int tiles_m = kRagged ? (M + kTile - 1) / kTile : M / kTile;
  const int logical = xcd_logical_id(blockIdx.x, gridDim.x);
  constexpr int kGroupM = 8;
  const int group_size = kGroupM * tiles_n;
  const int group = logical / group_size;
  const int first_m = group * kGroupM;
  const int gm = min(tiles_m - first_m, kGroupM);
  const int in_group = logical - group * group_size;
  const int m0 = (first_m + in_group % gm) * kTile;
  const int n0 = (in_group / gm) * kTile;

  // ---- HBM -> LDS copies: 16 per slice (1 KiB each), 4 per wave. Piece p < 2: lhs rows
  // (2 wave + p) * 16 + lane / 4, chunk slot lane & 3. Piece 2 + i: rhs k-rows
  // 2 (2 wave + i) + lane / 32, chunk slot lane & 31. A lane fetches the HBM chunk that the
  // XOR swizzle places at its slot. ----
  uint32_t a_goff[2], b_goff[2];
  int a_klim = K, b_klim[2] = {K, K};
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int r = (2 * wave + p) * 16 + (lane >> 2);
    const int c = (lane & 3) ^ a_mask(r);
    a_goff[p] = (uint32_t)((r * lda + 4 * c) * 4);
    if (kRagged) {
      if (m0 + r >= M) a_goff[p] = kBufOOB;
      a_klim = K - 4 * c;  // the same chunk for both pieces: a_mask(r + 16) == a_mask(r)
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int k = 2 * (2 * wave + i) + (lane >> 5);
    const int c = (lane & 31) ^ b_mask(k);
    b_goff[i] = (uint32_t)((k * ldb + 4 * c) * 4);
    if (kRagged) {
      if (n0 + 4 * c >= N) b_goff[i] = kBufOOB;
      b_klim[i] = K - k;
    }
  }
  const char* a_tile = reinterpret_cast<const char*>(A + (long long)m0 * lda);
  const char* b_tile = reinterpret_cast<const char*>(B + n0);
  const uint32_t lds0 = lds_addr(lds);
  constexpr uint32_t kABytes = kTile * kBK * 4;  // 8 KiB lhs slice, then 8 KiB rhs slice

  auto issue = [&](int kt) {
    const uint32_t st = lds0 + (kt % kStages) * kStageBytes;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const char* src = a_tile + (long long)kt * kBK * 4;  // the piece's rows are in a_goff
      const uint32_t dst = st + (2 * wave + p) * 1024;
      if constexpr (kRagged) buf2lds16_s(kt * kBK < a_klim ? a_goff[p] : kBufOOB, src, dst);
      else g2lds16_s(a_goff[p], src, dst);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const char* src = b_tile + (long long)kt * kBK * ldb * 4;
      const uint32_t dst = st + kABytes + (2 * wave + i) * 1024;
      if constexpr (kRagged) buf2lds16_s(kt * kBK < b_klim[i] ? b_goff[i] : kBufOOB, src, dst);
      else g2lds16_s(b_goff[i], src, dst);
    }
  };

  // ---- fragment reads (byte addresses within a stage) ----
  const int frag = lane & 31;
  const int h = lane >> 5;
  uint32_t a_rd[2][2];  // [row block i][half ks]: row wm*64 + 32 i + frag, chunk 2 ks + h
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int m = wm * 64 + 32 * i + frag;
      a_rd[i][ks] = (uint32_t)(m * 64 + 16 * ((2 * ks + h) ^ a_mask(m)));
    }
  // rhs: column n = wn*64 + 32 j + frag of k-row 8 ks + 4 h + kk; the mask depends on k only
  // through (k >> 2) & 1 = h, so per (j) one base and +512 bytes per k-row.
  uint32_t b_rd[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = wn * 64 + 32 * j + frag;
    b_rd[j] = kABytes + (uint32_t)((4 * h) * 512 + 16 * ((n >> 2) ^ b_mask(4 * h)) + 4 * (n & 3));
  }

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int ktiles = kRagged ? (K + kBK - 1) / kBK : K / kBK;
#pragma unroll
  for (int t = 0; t < kStages - 1; ++t)
    if (t < ktiles) issue(t);
  for (int kt = 0; kt < ktiles; ++kt) {
    // slice kt has landed once at most the copies of the slices after it (4 per slice and
    // wave, up to kStages - 2 slices) are outstanding; the barrier also ends every wave's
    // reads of slice kt-1, whose stage slice kt+kStages-1 refills
    const int later = min(kStages - 2, ktiles - 1 - kt);
    if (later >= 2) wait_and_barrier<8>();
    else if (later == 1) wait_and_barrier<4>();
    else wait_and_barrier<0>();
    if (kt + kStages - 1 < ktiles) issue(kt + kStages - 1);
    const uint32_t st = lds0 + (kt % kStages) * kStageBytes;
    // all fragments of the slice are read before its MFMAs: the reads of half 1 land while
    // the MFMAs of half 0 run
    f32x4 a[2][2];
    float b[2][2][4];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[ks][i] = *(const __attribute__((address_space(3))) f32x4*)(uintptr_t)(st + a_rd[i][ks]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          b[ks][j][kk] = *(const __attribute__((address_space(3))) float*)(uintptr_t)(st + b_rd[j] + (8 * ks + kk) * 512);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(b[ks][j][kk], a[ks][i][kk], acc[i][j], 0, 0, 0);
  }

  // Epilogue: lane l holds C[m][n .. n+3], m = row block + l % 32, n = column block
  // + 8 q + 4 (l / 32), q = 0..3.
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int m = m0 + wm * 64 + 32 * i + frag;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn * 64 + 32 * j + 8 * q + 4 * h;
        if (kRagged && (m >= M || n >= N)) continue;  // N % 4 == 0: n < N covers n .. n+3
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * q + e] + (kBias ? bias[n + e] : 0.f);
        *reinterpret_cast<f32x4*>(C + (long long)m * ldc + n) = v;
      }
  }
}

}  // namespace kg_gfx950

namespace kg_gfx950 {

// Split-K fp32 GEMM for small outputs (C1's 256^3 is 64 blocks of 32 x 32): one 1024-thread
// workgroup per 32 x 32 output block; its 16 waves take interleaved 16-deep K slices (wave
// w: k = 16 (w + 16 i) ..), load their operands straight from HBM/L2 into registers (lhs as
// 16-byte row pieces, rhs as 32 consecutive columns of one k-row per lane half) and run
// v_mfma_f32_32x32x2_f32 with the k order of gemm_f32_mfma_kernel; the 16 partial blocks are
// summed through LDS, wave by wave in order, and the sum is stored once. No workspace: the
// reduction never leaves the workgroup. Host requirements: M % 32 == 0, N % 32 == 0,
// K % 16 == 0, unit inner strides, lhs row stride a multiple of 4, 16-byte aligned lhs.
namespace gemmk {
constexpr int kWaves = 16;
constexpr int kThreads = 64 * kWaves;
static_assert(16 % kWaves == 0, "reduction: 16 accumulator elements per lane over the waves");
}  // namespace gemmk

template <int kBias>
__global__ __launch_bounds__(gemmk::kThreads, 1) void gemm_f32_splitk_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, const float* __restrict__ bias,
    int M, int N, int K, long long lda, long long ldb, long long ldc) {
  using namespace gemmk;
  __shared__ float part[kWaves][16][64];  // [wave][accumulator element][lane], 64 KiB
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int frag = lane & 31, h = lane >> 5;
  const int tiles_n = N / 32;
  const int m0 = (blockIdx.x / tiles_n) * 32;
  const int n0 = (blockIdx.x % tiles_n) * 32;
  const float* a_row = A + (long long)(m0 + frag) * lda + 4 * h;  // + k0 + 8 g
  const float* b_col = B + (long long)(4 * h) * ldb + n0 + frag;  // + (k0 + 8 g + kk) ldb

  f32x16 acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
  for (int k0 = 16 * wave; k0 < K; k0 += 16 * kWaves) {
    f32x4 a[2];
    float b[2][4];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      a[g] = *reinterpret_cast<const f32x4*>(a_row + k0 + 8 * g);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) b[g][kk] = b_col[(long long)(k0 + 8 * g + kk) * ldb];
    }
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(b[g][kk], a[g][kk], acc, 0, 0, 0);
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) part[wave][e][lane] = acc[e];
  __syncthreads();
  // thread t sums elements e = t / 64 + kWaves i of lane l = t % 64 over the waves:
  // C[m0 + l % 32][n0 + 8 (e / 4) + 4 (l / 32) + e % 4]
  const int l = tid & 63;
#pragma unroll
  for (int e = tid >> 6; e < 16; e += kWaves) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) v += part[w][e][l];
    const int n = n0 + 8 * (e >> 2) + 4 * (l >> 5) + (e & 3);
    if constexpr (kBias) v += bias[n];
    C[(long long)(m0 + (l & 31)) * ldc + n] = v;
  }
}

}  // namespace kg_gfx950
