// gemm_quad_kernel: bf16/f16 GEMM for whole kTM x 256 tiles (M % kTM == 0, N % 256 == 0,
// K % 32 == 0), four waves per workgroup, one per SIMD, each computing a (kTM/2) x 128 quarter
// of the tile with v_mfma_f32_16x16x32 and its fp32 accumulators (256 per lane at kTM = 256,
// 128 at kTM = 128) held in the accumulation registers. kTM = 128 is the form for grids whose
// 256 x 256 tiles would leave CUs idle (C2': 8192 x 1024 is 128 such tiles, 256 of 128 x 256).
//
// Against gemm_pipe_kernel (eight waves of 128 x 64) a wave reads 16 KiB of fragments per
// 64 MFMAs instead of 12 KiB per 32: two thirds of the LDS read bytes per MFMA (at kTM = 128,
// 12 KiB per 32 MFMAs against the eight-wave 128-row tile's 8 KiB per 16: three quarters). The LDS
// ring, the copy path (global_load_lds_dwordx4, 1 KiB per wave per copy), the operand
// layouts and the chunk swizzles are gemm_pipe_kernel's (gemmp::a_slot / gemmp::b_slot).
// With one wave per SIMD no second wave covers a stall, so the slice is software-pipelined
// in full: slice kt's 64 MFMAs run from registers while slice kt+1's 24 fragment reads and
// slice kt+kStages's 8 copies are slotted between them; one barrier per slice, at its start,
// publishes slice kt+1's copies and frees slice kt's stage for its refill.
//
// kExact (even ring depths, K / 32 a multiple of the depth and at least twice it): the last
// kStages slices are a compile-time group, so their waits and fragment reads carry no runtime
// conditions (with the runtime conditions those slices took 1.3-1.5x a steady slice's
// cycles). C is written with nontemporal stores: whole 256-byte row segments stream past
// the L2, so less dirty data is left to write back when the kernel ends (measured 1-1.5 %
// shorter launches than write-back stores at C2's shape).
#pragma once

#include "common.h"
#include "gemm.h"
#include "lds_dma.h"

namespace kg_gfx950 {

namespace gemmq {
// acc += a * b on one 16 x 16 block, the accumulator tied to one register tuple of the
// accumulation file for the whole kernel (with the intrinsic, the register allocator
// rotates the 256 live accumulators through the full file with moves at every loop edge).
// Being opaque to the compiler's hazard tracking, the caller waits for the last one to
// finish before reading any accumulator (mfma_drain).
template <typename Tag>
__device__ __forceinline__ void mfma16_tied(f32x4& acc, u32x4 a, u32x4 b) {
  if constexpr (__is_same(Tag, Bf16Tag))
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  else
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// 32 wait states: more than the 16x16x32 MFMA's result latency, before VALU reads of its
// result. The caller then passes every accumulator through mfma_order (an empty asm that
// redefines it), so the compiler cannot move a read of one above the wait.
__device__ __forceinline__ void mfma_drain() { asm volatile("s_nop 15\n\ts_nop 15" ::: "memory"); }
__device__ __forceinline__ void mfma_order(f32x4 (&a)[8]) {
  asm volatile("" : "+a"(a[0]), "+a"(a[1]), "+a"(a[2]), "+a"(a[3]), "+a"(a[4]), "+a"(a[5]), "+a"(a[6]), "+a"(a[7]));
}
constexpr int kT = 256;        // tile columns (and rows of the full-height form)
constexpr int kBK = 32;        // K slice
constexpr int kThreads = 256;  // 4 waves
constexpr int kVecsB = kT * kBK / 8;  // u32x4 per rhs stage (16 KiB)
constexpr int kBPieces = 4;    // rhs copies per wave per slice (2 k-rows each)
constexpr int kDefaultStages = 4;
}  // namespace gemmq

template <typename Tag, int kBias, int kStages, bool kExact, int kTM>
__global__ __launch_bounds__(gemmq::kThreads, 1) void gemm_quad_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, uint16_t* __restrict__ C,
    const void* __restrict__ bias, int M, int N, int K, long long lda, long long ldb, long long ldc) {
  using namespace gemmq;
  using gemmp::a_mask;
  using gemmp::a_slot;
  using gemmp::b_mask;
  using gemmp::b_slot;
  using H = Half16<Tag>;
  static_assert(kStages >= 2 && kStages <= 5, "ring depth");
  static_assert(!kExact || kStages % 2 == 0, "the exact-K form unrolls one ring turn per group");
  static_assert(kTM == 256 || kTM == 128, "tile height");
  constexpr int WM = kTM / 2;                   // rows per wave
  constexpr int NA = WM / 16;                   // lhs blocks per wave (8 or 4)
  constexpr int kVecsA = kTM * kBK / 8;         // u32x4 per lhs stage
  constexpr int kAPieces = kTM * kBK * 2 / 1024 / 4;  // lhs copies per wave per slice (16 rows each)
  constexpr int kPieces = kAPieces + kBPieces;  // copies per wave per slice
  constexpr int kReads = 8 + NA;                // fragment read steps per slice
  constexpr int kMfmas = NA * 8;                // MFMAs per wave per slice
  constexpr int kCopyGap = kMfmas / kPieces;    // MFMAs between a wave's copies
  static_assert(kCopyGap >= 4 && 2 * kReads <= kMfmas, "slots");
  __shared__ u32x4 lds_a[kStages][kVecsA];
  __shared__ u32x4 lds_b[kStages][kVecsB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1;  // WM-row half of the tile
  const int wn = wave & 1;   // 128-column half

  const int tiles_n = N / kT;
  const int tiles_m = M / kTM;
  const int logical = xcd_logical_id(blockIdx.x, gridDim.x);
  constexpr int kGroupM = 4;
  const int group_size = kGroupM * tiles_n;
  const int group = logical / group_size;
  const int first_m = group * kGroupM;
  const int gm = min(tiles_m - first_m, kGroupM);
  const int in_group = logical - group * group_size;
  const int m0 = (first_m + in_group % gm) * kTM;
  const int n0 = (in_group / gm) * kT;

  // ---- HBM -> LDS copies: piece p < kAPieces is lhs rows (wave*kAPieces+p)*16 + lane/4 (the
  // swizzle depends on lane/16 only), piece kAPieces+i is rhs k-rows (wave*4+i)*2 + lane/32 ----
  const int a_row0 = wave * 16 * kAPieces + (lane >> 2);
  const uint32_t a_goff = (uint32_t)((a_row0 * lda + 8 * ((lane & 3) ^ a_mask(a_row0))) * 2);
  uint32_t b_goff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int k = (wave * 4 + i) * 2 + (lane >> 5);
    b_goff[i] = (uint32_t)((k * ldb + 8 * ((lane & 31) ^ b_mask(k))) * 2);
  }
  const char* a_tile = reinterpret_cast<const char*>(A + (long long)m0 * lda);
  const char* b_tile = reinterpret_cast<const char*>(B + n0);
  const long long a_piece = 16 * lda * 2;
  const long long b_step = (long long)kBK * ldb * 2;
  const uint32_t lds_a0 = lds_addr(&lds_a[0][0]);
  const uint32_t lds_b0 = lds_addr(&lds_b[0][0]);
  constexpr uint32_t kStageA = kVecsA * 16;
  constexpr uint32_t kStageB = kVecsB * 16;

  // (the lambdas are forced inline: if one were left a call, the fragment and accumulator
  // arrays it takes by reference would move to scratch memory)
  auto issue_piece = [&](int kt, int s, int piece) __attribute__((always_inline)) {
    if (piece < kAPieces) {
      g2lds16_s(a_goff, a_tile + (long long)kt * kBK * 2 + piece * a_piece,
                lds_a0 + s * kStageA + (wave * kAPieces + piece) * 1024);
    } else {
      const int i = piece - kAPieces;
      g2lds16_s(b_goff[i], b_tile + kt * b_step, lds_b0 + s * kStageB + (wave * 4 + i) * 1024);
    }
  };

  // ---- fragments: lhs block ib = rows wm*WM + 16 ib + lane%16, chunk lane/16 (one
  // ds_read_b128; +1024 bytes per block); rhs block nb = columns wn*128 + 16 nb + lane%16,
  // k-rows 8(lane/16) + 0..7 in two ds_read_b64_tr_b16 (+2048 bytes for k-rows +4) ----
  const int l16 = lane & 15;
  const int lg = lane >> 4;
  const uint32_t a_rd = lds_a0 + a_slot(wm * WM + l16, lg) * 16;
  uint32_t b_rd[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) {
    const int n = wn * 128 + nb * 16 + 4 * (l16 & 3);
    b_rd[nb] = lds_b0 + b_slot(8 * lg + (l16 >> 2), n >> 3) * 16 + (n & 7) * 2;
  }
  struct Frags {
    u32x4 a[NA];
    u32x4 b[8];
  };
  auto read_b = [&](int s, u32x4& f, int nb) __attribute__((always_inline)) {
    const uint32_t ad = b_rd[nb] + s * kStageB;
    const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(uintptr_t)ad);
    const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(uintptr_t)(ad + 2048));
    const u32x2 w0 = __builtin_bit_cast(u32x2, v0), w1 = __builtin_bit_cast(u32x2, v1);
    f = u32x4{w0[0], w0[1], w1[0], w1[1]};
  };
  auto read_a = [&](int s, int ib) __attribute__((always_inline)) -> u32x4 {
    return *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)(a_rd + s * kStageA + ib * 1024);
  };
  // read step r (0..kReads-1): the rhs blocks first (the next slice's first eight MFMAs use
  // lhs block 0 with rhs blocks 0..7), then the lhs blocks
  auto read_step = [&](int s, Frags& f, int r) __attribute__((always_inline)) {
    if (r < 8) read_b(s, f.b[r], r);
    else f.a[r - 8] = read_a(s, r - 8);
  };

  f32x4 acc[NA][8];
#pragma unroll
  for (int i = 0; i < NA; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[i][j][e] = 0.f;
  // opaque from here on: the compiler must not rematerialise the zeros (with accumulator
  // copies) right before the first MFMAs, which would read them without the wait states
  // a VALU write before an MFMA needs
#pragma unroll
  for (int i = 0; i < NA; ++i) mfma_order(acc[i]);

  const int ktiles = K / kBK;
#pragma unroll
  for (int st = 0; st < kStages; ++st)
    if (st < ktiles)
#pragma unroll
      for (int piece = 0; piece < kPieces; ++piece) issue_piece(st, st, piece);
  {
    const int younger = min(kStages - 1, ktiles - 1);
    if (younger >= 4) wait_and_barrier<4 * kPieces>();
    else if (younger == 3) wait_and_barrier<3 * kPieces>();
    else if (younger == 2) wait_and_barrier<2 * kPieces>();
    else if (younger == 1) wait_and_barrier<kPieces>();
    else wait_and_barrier<0>();
  }
  Frags fr[2];  // slice kt's fragments are fr[kt & 1]; the next slice's are read into the other
#pragma unroll
  for (int r = 0; r < kReads; ++r) read_step(0, fr[0], r);

  // One slice in stage S: wait for slice kt+1's copies and meet the other waves (slice kt's
  // stage is then free), then the kMfmas MFMAs with slice kt+1's kReads fragment reads (8 rhs
  // blocks of two LDS instructions, NA lhs blocks of one) on the even steps and slice
  // kt+kStages's kPieces copies kCopyGap steps apart. Mode: 1 steady (more slices follow and a refill is due); 2 one of the last
  // kStages slices of the exact-K form, with kFollow = decltype(follow_tag)::value slices
  // after it, all of them copied already; 0 any slice, with runtime conditions.
  auto slice = [&](int kt, auto stage_tag, auto par_tag, auto mode_tag, auto follow_tag) __attribute__((always_inline)) {
    constexpr int S = decltype(stage_tag)::value;
    constexpr int P = decltype(par_tag)::value;
    constexpr int kMode = decltype(mode_tag)::value;
    constexpr int kFollow = decltype(follow_tag)::value;
    constexpr bool kSteady = kMode == 1;
    Frags& fx = fr[P];
    Frags& fn = fr[P ^ 1];
    const bool more = kSteady || kt + 1 < ktiles;
    const bool refill = kSteady || kt + kStages < ktiles;
    if constexpr (kMode == 2) {
      // the copies of the kFollow later slices are this wave's only outstanding ones
      if constexpr (kFollow >= 1) wait_and_barrier<(kFollow - 1) * kPieces>();
    } else if (kSteady) {
      wait_and_barrier<(kStages - 2) * kPieces>();
    } else if (more) {
      const int younger = min(kStages - 2, ktiles - 2 - kt);
      if (younger >= 3) wait_and_barrier<3 * kPieces>();
      else if (younger == 2) wait_and_barrier<2 * kPieces>();
      else if (younger == 1) wait_and_barrier<kPieces>();
      else wait_and_barrier<0>();
    }
    static_for<kMfmas>([&](auto idx_tag) __attribute__((always_inline)) {
      constexpr int idx = decltype(idx_tag)::value;
      constexpr int i = idx >> 3, j = idx & 7;
      constexpr bool kCopy = idx % kCopyGap == 3 && idx / kCopyGap < kPieces;
      mfma16_tied<Tag>(acc[i][j], fx.b[j], fx.a[i]);  // C^T blocks: lane-contiguous columns
      if constexpr (kMode == 2) {
        if constexpr (kFollow >= 1 && (idx & 1) == 0 && idx < 2 * kReads) read_step((S + 1) % kStages, fn, idx >> 1);
      } else if constexpr (kSteady) {
        if constexpr ((idx & 1) == 0 && idx < 2 * kReads) read_step((S + 1) % kStages, fn, idx >> 1);
        if constexpr (kCopy) issue_piece(kt + kStages, S, idx / kCopyGap);
      } else {
        if ((idx & 1) == 0 && idx < 2 * kReads && more) read_step((S + 1) % kStages, fn, idx >> 1);
        if (kCopy && refill) issue_piece(kt + kStages, S, idx / kCopyGap);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // Slices are unrolled U at a time (a compile-time loop: `#pragma unroll` gives up on the
  // larger bodies) so that each one's stage (kt % kStages) and register set (kt & 1) are
  // constants.
  constexpr int U = kStages % 2 == 0 ? kStages : 2 * kStages;
  auto unrolled = [&](int kt0, auto mode_tag) __attribute__((always_inline)) {
    static_for<U>([&](auto u_tag) __attribute__((always_inline)) {
      constexpr int u = decltype(u_tag)::value;
      if (decltype(mode_tag)::value == 1 || kt0 + u < ktiles)
        slice(kt0 + u, gemmp::StageIdx<u % kStages>{}, gemmp::StageIdx<u & 1>{}, mode_tag, Int<0>{});
    });
  };
  int kt = 0;
  if constexpr (kExact) {
    // ktiles % kStages == 0 and ktiles >= 2 kStages (the launcher checks): steady groups up to
    // the last kStages slices, which run as one compile-time group
    for (; kt + U < ktiles; kt += U) unrolled(kt, Int<1>{});
    static_for<U>([&](auto u_tag) __attribute__((always_inline)) {
      constexpr int u = decltype(u_tag)::value;
      slice(kt + u, gemmp::StageIdx<u % kStages>{}, gemmp::StageIdx<u & 1>{}, Int<2>{}, Int<U - 1 - u>{});
    });
  } else {
    for (; kt + U + kStages <= ktiles; kt += U) unrolled(kt, Int<1>{});
    for (; kt < ktiles; kt += U) unrolled(kt, Int<0>{});
  }

  // Epilogue: lane l holds C[m][n .. n+3] of block (i, j) (m = row block + l % 16, n = column
  // block + 4 (l / 16)). Stored as is, every store instruction would write 32-byte pieces of
  // 16 rows; instead each wave packs P row blocks at a time (bias added, rounded once) into an
  // LDS region of its own, [16P rows][128 columns], and writes them back as whole 256-byte row
  // segments, 16 bytes per lane and 4 rows per instruction (the chip-wide store burst at the
  // end of the kernel drains faster). 16-byte chunk c of region row r sits at slot
  // c ^ (r % 16): the packing writes of 16 rows and the row reads both spread over all banks.
  // A wave reads back only what it wrote itself, so no barrier separates the two; one barrier
  // first retires the ring (every wave is past its last fragment read).
  mfma_drain();
#pragma unroll
  for (int i = 0; i < NA; ++i) mfma_order(acc[i]);
  wait_and_barrier<0>();
  // row blocks per pass: two regions of 4P KiB in each half of the ring (the lhs half is the
  // smaller one at kTM = 128)
  constexpr int P = 2 * 8 * 4096 <= kStages * kStageA ? 8 : 2 * 4 * 4096 <= kStages * kStageA ? 4 : 2;
  static_assert(P <= NA && NA % P == 0 && 2 * P * 4096 <= kStages * kStageA, "two epilogue regions per ring half");
  const uint32_t region = (wave < 2 ? lds_a0 : lds_b0) + (wave & 1) * P * 4096;
#pragma unroll
  for (int i0 = 0; i0 < NA; i0 += P) {
#pragma unroll
    for (int i = i0; i < i0 + P; ++i) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int n = n0 + wn * 128 + j * 16 + 4 * lg;
        float v0 = acc[i][j][0], v1 = acc[i][j][1], v2 = acc[i][j][2], v3 = acc[i][j][3];
        if constexpr (kBias == 1) {
          const float* bp = static_cast<const float*>(bias);
          v0 += bp[n];
          v1 += bp[n + 1];
          v2 += bp[n + 2];
          v3 += bp[n + 3];
        } else if constexpr (kBias == 2) {
          const uint16_t* bp = static_cast<const uint16_t*>(bias);
          v0 += H::to_float(bp[n]);
          v1 += H::to_float(bp[n + 1]);
          v2 += H::to_float(bp[n + 2]);
          v3 += H::to_float(bp[n + 3]);
        }
        u32x2 packed;
        packed[0] = H::pack2(v0, v1);
        packed[1] = H::pack2(v2, v3);
        const int r = 16 * (i - i0) + l16;  // region row; r % 16 == l16
        const uint32_t ad = region + r * 256 + (((2 * j + (lg >> 1)) ^ l16) * 16) + (lg & 1) * 8;
        *(__attribute__((address_space(3))) u32x2*)(uintptr_t)ad = packed;
      }
    }
#pragma unroll
    for (int q = 0; q < 4 * P; ++q) {
      const int r = 4 * q + (lane >> 4);
      const int c = lane & 15;
      const u32x4 v = *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)(region + r * 256 + ((c ^ (r & 15)) * 16));
      const int m = m0 + wm * WM + 16 * i0 + r;
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(C + (long long)m * ldc + n0 + wn * 128 + 8 * c));
    }
  }
}

// One launch of gemm_quad_kernel over (M/kTM) x (N/256) workgroups. bias_kind: 0 none,
// 1 fp32, 2 16-bit.
template <typename Tag, int kStages, int kTM>
hipError_t launch_gemm_quad(const uint16_t* A, const uint16_t* B, uint16_t* C, const void* bias, int bias_kind, int M,
                            int N, int K, long long lda, long long ldb, long long ldc, hipStream_t stream) {
  const int grid = (M / kTM) * (N / gemmq::kT);
  const int ktiles = K / gemmq::kBK;
  const bool exact = kStages % 2 == 0 && ktiles % kStages == 0 && ktiles >= 2 * kStages;
#define KG_GEMM_QUAD(BIAS, EXACT)                                                                                   \
  hipLaunchKernelGGL((gemm_quad_kernel<Tag, BIAS, kStages, EXACT, kTM>), dim3(grid), dim3(gemmq::kThreads), 0, stream, A, \
                     B, C, bias, M, N, K, lda, ldb, ldc)
  if constexpr (kStages % 2 == 0) {
    if (exact) {
      if (bias_kind == 0) KG_GEMM_QUAD(0, true);
      else if (bias_kind == 1) KG_GEMM_QUAD(1, true);
      else KG_GEMM_QUAD(2, true);
      return hipGetLastError();
    }
  }
  if (bias_kind == 0) KG_GEMM_QUAD(0, false);
  else if (bias_kind == 1) KG_GEMM_QUAD(1, false);
  else KG_GEMM_QUAD(2, false);
#undef KG_GEMM_QUAD
  return hipGetLastError();
}

}  // namespace kg_gfx950
