// GEMM kernels for the matmul demos: out[M,N] = lhs[M,K] @ rhs[K,N] (+ bias[N]),
// row-major, fp32 accumulation.
//
// gemm_pipe_kernel: bf16/f16 operands on gfx950 MFMA (v_mfma_f32_16x16x32_{bf16,f16}: the
//   same FLOP per cycle as 32x32x16 at half the cycles per instruction; in this kernel, which
//   runs at the part's power limit, it does the same work for less energy and so holds a
//   higher clock), any M, N % 8 == 0, K % 8 == 0.
//
// gemm_simt_kernel: any dtype (f32/bf16/f16), any shape and stride; 64x64 LDS tiles,
//   4x4 outputs per thread, fp32 FMA accumulation in k order.
#pragma once

#include "common.h"
#include "lds_dma.h"

namespace kg_gfx950 {

// gemm_pipe_kernel: kTM x 256 tiles (kTM = 256, or 128 when 256-row tiles would leave CUs idle) computed by
//   8 waves (2 x 4 waves of kTM/2 x 64, two per SIMD) with 16x16x32 MFMAs. Both operands
//   are copied HBM -> LDS by global_load_lds_dwordx4 (no registers, no VALU work) through a
//   kStages-deep ring of 32-deep K slices (kStages x (kTM/16 + 16) KiB; 4 by default, 2 or
//   3 on request), so loads are issued kStages - 1 slices ahead of their use; every wave issues kTM/128 + 2 of a slice's copies (1 KiB
//   each), slotted between its MFMAs, and while one wave of a SIMD waits on a copy's issue
//   or an LDS read the other keeps the MFMA pipe busy. lhs slices are [m][k] rows of 64 bytes; rhs slices
//   stay [k][n] as in HBM and the MFMA operand (8 consecutive k of one n) is read with two
//   ds_read_b64_tr_b16: within each 16-lane group, lane j addresses 4 consecutive n of
//   k-row j/4 and lane i receives k-rows 0..3 of column i. Chunk swizzles: lhs
//   p = c ^ ((row >> 2) & 3), rhs p = c ^ (4(k & 3) ^ 2((k >> 3) & 1)) -- the fragment
//   reads hit distinct banks of the 64-bank LDS. Each MFMA takes a whole 32-deep slice of a
//   16 x 16 block; a wave's kTM/32 lhs blocks are split in two halves: while the MFMAs of
//   the first half run, the second half's lhs fragments are read; while those of the second
//   run, the next slice's rhs and first-half lhs fragments are read (two register sets,
//   alternating by slice), and the per-slice barrier sits between the two halves.
//   kRagged (M % kTM, N % 256 or K % 32 non-zero): the copies go through buffer loads whose
//   out-of-range lanes land zeros in LDS (edge rows, edge column chunks, k >= K), and the
//   epilogue stores only the rows and columns inside the matrix; the loop is unchanged.
//   Host requirements: K % 8 == 0, N % 8 == 0, row strides multiples of 8 and at most
//   2^22 elements, 16-byte aligned base pointers.
//   Split-K (k_chunk > 0, for outputs of few tiles): workgroup row blockIdx.y runs the K range
//   [y*k_chunk, min(K, (y+1)*k_chunk)) as a GEMM of its own and stores its fp32 sums to
//   partial[y][M][N] (no bias); gemm_splitk_reduce_kernel adds the rows in y order, adds the
//   bias and rounds once.
namespace gemmp {
constexpr int kBM = 256;  // largest tile height (kTM)
constexpr int kBN = 256;
constexpr int kBK = 32;
constexpr int kDefaultStages = 4;  // LDS ring depth unless the caller asks for 2 or 3
constexpr int kThreads = 512;  // 8 waves: 2 x 4 of kTM/2 x 64, two per SIMD
constexpr int kBVecs = kBK * kBN / 8;  // 1024 u32x4 per rhs stage
// LDS has 64 banks of 4 bytes: ds_read_b128 serves 16 lanes per cycle, 64-bit reads 32.
// The swizzles are XOR masks, so the same mask maps an LDS slot back to its HBM chunk.
__device__ __forceinline__ int a_mask(int row) { return (row >> 2) & 3; }
__device__ __forceinline__ int b_mask(int k) { return (4 * (k & 3)) ^ (2 * ((k >> 3) & 1)); }
__device__ __forceinline__ int a_slot(int row, int c) { return row * 4 + (c ^ a_mask(row)); }
__device__ __forceinline__ int b_slot(int k, int c) { return k * 32 + (c ^ b_mask(k)); }
template <int S>
struct StageIdx {
  static constexpr int value = S;
};
}  // namespace gemmp

template <typename Tag, int kBias, int kTM, int kStages, bool kRagged>
__global__ __launch_bounds__(gemmp::kThreads, 1) void gemm_pipe_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, uint16_t* __restrict__ C,
    const void* __restrict__ bias, int M, int N, int K, long long lda, long long ldb, long long ldc,
    float* __restrict__ partial, int k_chunk) {
  using namespace gemmp;
  using H = Half16<Tag>;
  static_assert(kTM == 256 || kTM == 128, "tile height");
  if (k_chunk > 0) {  // split-K: this workgroup row's K range, as a GEMM of its own
    const int k_begin = blockIdx.y * k_chunk;
    A += k_begin;
    B += (long long)k_begin * ldb;
    K = min(k_chunk, K - k_begin);
    partial += (long long)blockIdx.y * M * N;
  }
  static_assert(kStages >= 2 && kStages <= 4, "ring depth");
  constexpr int MB = kTM / 32;              // 16-row lhs blocks per wave
  constexpr int MH = MB / 2;                // of them in each half slice
  constexpr int AP = kTM / 128;             // lhs copies per wave per slice
  constexpr int kPieces = AP + 2;           // copies per wave per slice: AP lhs, 2 rhs
  constexpr int NRX = 4 + MH;               // read steps of a slice's set X: 4 rhs blocks, MH lhs blocks
  constexpr int NM = 4 * MH;                // MFMAs per half slice: MH lhs blocks x 4 rhs blocks
  constexpr int NS0 = NM > MH ? NM : MH;    // interleave steps of half 0 (MH lhs reads)
  constexpr int NS1 = NM > NRX ? NM : NRX;  // interleave steps of half 1 (the next slice's first set)
  constexpr int kAVecs = kTM * kBK / 8;     // u32x4 per lhs stage
  __shared__ u32x4 lds_a[kStages][kAVecs];
  __shared__ u32x4 lds_b[kStages][kBVecs];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2;  // kTM/2-row half of the tile
  const int wn = wave & 3;   // 64-column quarter

  const int tiles_n = kRagged ? (N + kBN - 1) / kBN : N / kBN;
  const int tiles_m = kRagged ? (M + kTM - 1) / kTM : M / kTM;
  const int logical = xcd_logical_id(blockIdx.x, gridDim.x);
  constexpr int kGroupM = 4;
  const int group_size = kGroupM * tiles_n;
  const int group = logical / group_size;
  const int first_m = group * kGroupM;
  const int gm = min(tiles_m - first_m, kGroupM);
  const int in_group = logical - group * group_size;
  const int m0 = (first_m + in_group % gm) * kTM;
  const int n0 = (in_group / gm) * kBN;

  // ---- HBM -> LDS copies ----
  // Piece p < AP: lhs rows (wave*AP+p)*16 + lane/4 (a_mask depends on lane only, so one
  // per-lane offset and 16 rows between pieces). Piece AP+p: rhs k-rows (wave*2+p)*2 +
  // lane/32 (b_mask depends on p and lane).
  const int a_row0 = wave * AP * 16 + (lane >> 2);
  const uint32_t a_goff = (uint32_t)((a_row0 * lda + 8 * ((lane & 3) ^ a_mask(a_row0))) * 2);
  uint32_t b_goff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int k = (wave * 2 + i) * 2 + (lane >> 5);
    b_goff[i] = (uint32_t)((k * ldb + 8 * ((lane & 31) ^ b_mask(k))) * 2);
  }
  const char* a_tile = reinterpret_cast<const char*>(A + (long long)m0 * lda);
  const char* b_tile = reinterpret_cast<const char*>(B + n0);
  const long long a_piece = 16 * lda * 2;
  const long long b_step = (long long)kBK * ldb * 2;
  const uint32_t lds_a0 = lds_addr(&lds_a[0][0]);
  const uint32_t lds_b0 = lds_addr(&lds_b[0][0]);
  constexpr uint32_t kAStage = kAVecs * 16;
  constexpr uint32_t kBStage = kBVecs * 16;
  // Ragged shapes: a copy lane whose lhs row or rhs column chunk lies outside the matrix
  // takes voff kBufOOB for every slice, and one whose k lies at or beyond K (slice kt has
  // k = 32 kt + the lane's k offset) takes it for that slice: both land zeros in LDS, which
  // add nothing to the accumulators, and the epilogue stores only rows < M, columns < N.
  uint32_t a_voff[AP], b_voff[2];
  int a_klim = K, b_klim[2] = {K, K};
  if constexpr (kRagged) {
#pragma unroll
    for (int p = 0; p < AP; ++p) a_voff[p] = m0 + a_row0 + 16 * p < M ? a_goff : kBufOOB;
    a_klim = K - 8 * ((lane & 3) ^ a_mask(a_row0));
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int k = (wave * 2 + i) * 2 + (lane >> 5);
      b_voff[i] = n0 + 8 * ((lane & 31) ^ b_mask(k)) < N ? b_goff[i] : kBufOOB;
      b_klim[i] = K - k;
    }
  }

  auto issue_piece = [&](int kt, int s, int piece) {  // piece 0..kPieces-1: AP lhs then 2 rhs
    if (piece < AP) {
      const char* src = a_tile + (long long)kt * kBK * 2 + piece * a_piece;
      const uint32_t dst = lds_a0 + s * kAStage + (wave * AP + piece) * 1024;
      if constexpr (kRagged) buf2lds16_s(kt * kBK < a_klim ? a_voff[piece] : kBufOOB, src, dst);
      else g2lds16_s(a_goff, src, dst);
    } else {
      const int i = piece - AP;
      const char* src = b_tile + kt * b_step;
      const uint32_t dst = lds_b0 + s * kBStage + (wave * 2 + i) * 1024;
      if constexpr (kRagged) buf2lds16_s(kt * kBK < b_klim[i] ? b_voff[i] : kBufOOB, src, dst);
      else g2lds16_s(b_goff[i], src, dst);
    }
  };

  // ---- fragment reads (v_mfma_f32_16x16x32: 16-row lhs blocks x 16-column rhs blocks, the
  // whole 32-deep slice in one step) ----
  // lhs block ib: rows wm*kTM/2 + 16 ib + lane%16, 16-byte chunk lane/16 (8 k): one
  // ds_read_b128; block ib+1 is 16 rows on (same mask): +1024 bytes. rhs block nb: columns
  // wn*64 + 16 nb + lane%16, k-rows 8*(lane/16) + 0..7 in two ds_read_b64_tr_b16 (k-rows +4:
  // +2048 bytes, same mask). Per-lane byte addresses, LDS base included.
  const int l16 = lane & 15;
  const int lg = lane >> 4;
  const uint32_t a_rd = lds_a0 + a_slot(wm * (kTM / 2) + l16, lg) * 16;
  uint32_t b_rd[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    const int n = wn * 64 + nb * 16 + 4 * (l16 & 3);
    b_rd[nb] = lds_b0 + b_slot(8 * lg + (l16 >> 2), n >> 3) * 16 + (n & 7) * 2;
  }

  // A slice's fragments come in two sets: X (the 4 rhs blocks and lhs blocks 0..MH-1, read
  // before the slice) and Y (lhs blocks MH..MB-1, read during its first half).
  struct FragX {
    u32x4 b[4];
    u32x4 a[MH];
  };
  auto read_b = [&](int s, u32x4& f, int nb) {
    const uint32_t ad = b_rd[nb] + s * kBStage;
    const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(uintptr_t)ad);
    const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(uintptr_t)(ad + 2048));
    const u32x2 w0 = __builtin_bit_cast(u32x2, v0), w1 = __builtin_bit_cast(u32x2, v1);
    f = u32x4{w0[0], w0[1], w1[0], w1[1]};
  };
  auto read_a = [&](int s, int ib) -> u32x4 {
    return *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)(a_rd + s * kAStage + ib * 1024);
  };
  // read step r (0..NRX-1) of set X: the rhs blocks first (two transposed reads each), then lhs
  auto read_x = [&](int s, FragX& f, int r) {
    if (r < 4) read_b(s, f.b[r], r);
    else f.a[r - 4] = read_a(s, r - 4);
  };

  f32x4 acc[MB][4];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[i][j][e] = 0.f;

  const int ktiles = kRagged ? (K + kBK - 1) / kBK : K / kBK;
#pragma unroll
  for (int st = 0; st < kStages; ++st)
    if (st < ktiles)
#pragma unroll
      for (int piece = 0; piece < kPieces; ++piece) issue_piece(st, st, piece);
  {
    const int younger = min(kStages - 1, ktiles - 1);
    if (younger >= 3) wait_and_barrier<3 * kPieces>();
    else if (younger == 2) wait_and_barrier<2 * kPieces>();
    else if (younger == 1) wait_and_barrier<kPieces>();
    else wait_and_barrier<0>();
  }
  FragX fr[2];   // set X of slice kt is fr[kt & 1]; the next slice's is read into the other
  u32x4 fy[MH];  // this slice's set Y
#pragma unroll
  for (int r = 0; r < NRX; ++r) read_x(0, fr[0], r);

  // One 32-deep slice in stage S: the MFMAs of lhs blocks 0..MH-1 with the reads of set Y
  // slotted in between, barrier, the MFMAs of blocks MH..MB-1 with the next slice's set X
  // and this stage's refill copies slotted in between. kSteady: more slices follow and a
  // refill is due.
  auto slice = [&](int kt, auto stage_tag, auto par_tag, auto steady_tag) {
    constexpr int S = decltype(stage_tag)::value;
    constexpr int P = decltype(par_tag)::value;
    constexpr bool kSteady = decltype(steady_tag)::value != 0;
    FragX& fx = fr[P];
    FragX& fn = fr[P ^ 1];
#pragma unroll
    for (int idx = 0; idx < NS0; ++idx) {
      const int i = idx >> 2, j = idx & 3;
      if (idx < NM) acc[i][j] = H::mfma16(fx.b[j], fx.a[i], acc[i][j]);
      if (idx < MH) fy[idx] = read_a(S, MH + idx);
      __builtin_amdgcn_sched_barrier(0);
    }
    const bool more = kSteady || kt + 1 < ktiles;
    const bool refill = kSteady || kt + kStages < ktiles;
    if (kSteady) {
      wait_and_barrier<(kStages - 2) * kPieces>();  // slices kt+2 .. kt+kStages-1 may be in flight
    } else if (more) {
      const int younger = min(kStages - 2, ktiles - 2 - kt);
      if (younger >= 2) wait_and_barrier<2 * kPieces>();
      else if (younger == 1) wait_and_barrier<kPieces>();
      else wait_and_barrier<0>();
    }
    if (kSteady) {
#pragma unroll
      for (int idx = 0; idx < NS1; ++idx) {
        const int i = idx >> 2, j = idx & 3;
        if (idx < NM) acc[MH + i][j] = H::mfma16(fx.b[j], fy[i], acc[MH + i][j]);
        if (idx < NRX) read_x((S + 1) % kStages, fn, idx);
        if ((idx & 1) && (idx >> 1) < kPieces) issue_piece(kt + kStages, S, idx >> 1);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      if (refill)
#pragma unroll
        for (int piece = 0; piece < kPieces; ++piece) issue_piece(kt + kStages, S, piece);
      if (more)
#pragma unroll
        for (int r = 0; r < NRX; ++r) read_x((S + 1) % kStages, fn, r);
#pragma unroll
      for (int idx = 0; idx < NM; ++idx) {
        const int i = idx >> 2, j = idx & 3;
        acc[MH + i][j] = H::mfma16(fx.b[j], fy[i], acc[MH + i][j]);
      }
    }
  };

  // Slices are unrolled U at a time so that each one's stage (kt % kStages) and register set
  // (kt & 1) are compile-time constants.
  constexpr int U = kStages % 2 == 0 ? kStages : 2 * kStages;
  auto unrolled = [&](int kt0, auto steady_tag) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // u as a constant: one slice per case
      if (kt0 + u < ktiles || decltype(steady_tag)::value) {
        if (u == 0) slice(kt0 + 0, StageIdx<0 % kStages>{}, StageIdx<0>{}, steady_tag);
        if (u == 1) slice(kt0 + 1, StageIdx<1 % kStages>{}, StageIdx<1>{}, steady_tag);
        if constexpr (U > 2) {
          if (u == 2) slice(kt0 + 2, StageIdx<2 % kStages>{}, StageIdx<0>{}, steady_tag);
          if (u == 3) slice(kt0 + 3, StageIdx<3 % kStages>{}, StageIdx<1>{}, steady_tag);
        }
        if constexpr (U > 4) {
          if (u == 4) slice(kt0 + 4, StageIdx<4 % kStages>{}, StageIdx<0>{}, steady_tag);
          if (u == 5) slice(kt0 + 5, StageIdx<5 % kStages>{}, StageIdx<1>{}, steady_tag);
        }
      }
    }
  };
  int kt = 0;
  for (; kt + U + kStages <= ktiles; kt += U) unrolled(kt, StageIdx<1>{});  // every slice refills its stage
  for (; kt < ktiles; kt += U) unrolled(kt, StageIdx<0>{});

  // Epilogue: lane l holds C[m][n .. n+3] of block (ib, nb): m = row block + l % 16, n = column
  // block + 4 (l / 16).
  auto out_value = [&](int i, int j, int n) -> u32x2 {  // bias added, rounded once
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
    return packed;
  };
  if (!kRagged && k_chunk == 0) {
    // Whole tiles: each wave packs P row blocks at a time into an LDS region of its own,
    // [16P rows][64 columns], and writes them back as whole 128-byte row segments (16 bytes
    // per lane, 8 rows per instruction) instead of 32-byte pieces of 16 rows. 16-byte chunk c
    // of region row r sits at slot c ^ (r % 8): two lanes per bank for the packing writes,
    // none shared for the row reads. One barrier retires the ring first; a wave reads back
    // only what it wrote itself.
    constexpr int kRingHalf = kStages * (kAVecs * 16 < kBVecs * 16 ? kAVecs * 16 : kBVecs * 16);
    constexpr int P = MB * 8192 <= kRingHalf ? MB : (MB / 2) * 8192 <= kRingHalf ? MB / 2 : MB / 4;
    static_assert(P >= 1 && MB % P == 0 && P * 8192 <= kRingHalf, "four epilogue regions fit in each half of the ring");
    wait_and_barrier<0>();
    const uint32_t region = (wave < 4 ? lds_a0 : lds_b0) + (wave & 3) * P * 2048;
#pragma unroll
    for (int i0 = 0; i0 < MB; i0 += P) {
#pragma unroll
      for (int i = i0; i < i0 + P; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const u32x2 packed = out_value(i, j, n0 + wn * 64 + j * 16 + 4 * lg);
          const int r = 16 * (i - i0) + l16;
          const uint32_t ad = region + r * 128 + (((2 * j + (lg >> 1)) ^ (r & 7)) * 16) + (lg & 1) * 8;
          *(__attribute__((address_space(3))) u32x2*)(uintptr_t)ad = packed;
        }
#pragma unroll
      for (int q = 0; q < 2 * P; ++q) {
        const int r = 8 * q + (lane >> 3);
        const int c = lane & 7;
        const u32x4 v = *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)(region + r * 128 + ((c ^ (r & 7)) * 16));
        const int m = m0 + wm * (kTM / 2) + 16 * i0 + r;
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(C + (long long)m * ldc + n0 + wn * 64 + 8 * c));
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    const int m = m0 + wm * (kTM / 2) + i * 16 + l16;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      {
        const int n = n0 + wn * 64 + j * 16 + 4 * lg;
        if (kRagged && (m >= M || n >= N)) continue;  // N % 8 == 0: n < N covers n .. n+3
        if (k_chunk > 0) {
          *reinterpret_cast<f32x4*>(partial + (long long)m * N + n) = acc[i][j];
          continue;
        }
        st8(C + (long long)m * ldc + n, out_value(i, j, n));
      }
    }
  }
}

// Sum of the split-K partial products: out[m][n] = round(sum_y partial[y][m][n] + bias[n]),
// y in order; one thread per 4 consecutive columns of a row (N % 8 == 0), one wave per
// workgroup so that small outputs still spread over every CU.
constexpr int kSplitReduceThreads = 64;
template <typename Tag, int kBias>
__global__ __launch_bounds__(kSplitReduceThreads) void gemm_splitk_reduce_kernel(
    const float* __restrict__ partial, int splits, uint16_t* __restrict__ C, const void* __restrict__ bias, int M, int N,
    long long ldc) {
  using H = Half16<Tag>;
  const long long idx = (long long)blockIdx.x * kSplitReduceThreads + threadIdx.x;
  const int nq = N >> 2;
  if (idx >= (long long)M * nq) return;
  const int m = (int)(idx / nq);
  const int n = (int)(idx - (long long)m * nq) * 4;
  const long long plane = (long long)M * N;
  const float* p = partial + (long long)m * N + n;
  f32x4 s = *reinterpret_cast<const f32x4*>(p);
  for (int y = 1; y < splits; ++y) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(p + y * plane);
#pragma unroll
    for (int e = 0; e < 4; ++e) s[e] += v[e];
  }
  if constexpr (kBias == 1) {
    const float* bp = static_cast<const float*>(bias);
#pragma unroll
    for (int e = 0; e < 4; ++e) s[e] += bp[n + e];
  } else if constexpr (kBias == 2) {
    const uint16_t* bp = static_cast<const uint16_t*>(bias);
#pragma unroll
    for (int e = 0; e < 4; ++e) s[e] += H::to_float(bp[n + e]);
  }
  u32x2 packed;
  packed[0] = H::pack2(s[0], s[1]);
  packed[1] = H::pack2(s[2], s[3]);
  st8(C + (long long)m * ldc + n, packed);
}

// Generic path: any element type, any shape/strides (element strides), optional bias.
// Each 256-thread block computes a T x T tile (T = 64, 32 or 16: the host picks the largest
// that still gives every CU a block); each thread a T/16 x T/16 micro tile. K advances in
// 32-deep slices; the next slice is loaded into registers while the FMAs of the current
// one run, so the loop pays one global-load latency in total rather than one per slice.
template <typename TA, typename TB, typename TC, typename TBias, int T>
__global__ __launch_bounds__(256) void gemm_simt_kernel(const TA* __restrict__ A, const TB* __restrict__ B,
                                                        TC* __restrict__ C, const TBias* __restrict__ bias,
                                                        int M, int N, int K, long long sam, long long sak,
                                                        long long sbk, long long sbn, long long scm,
                                                        long long scn, long long sbias) {
  static_assert(T == 64 || T == 32 || T == 16, "tile");
  constexpr int MT = T / 16;  // micro tile
  constexpr int TK = 32;
  constexpr int kPer = T * TK / 256;  // elements of each operand per thread and slice
  __shared__ float As[TK][T + 1];
  __shared__ float Bs[TK][T + 1];
  const int tid = threadIdx.x;
  const int tx = tid & 15;
  const int ty = tid >> 4;
  // one-dimensional grid: block b covers tile column b % ceil(N/T), tile row b / ceil(N/T)
  const int n_tiles = (N + T - 1) / T;
  const int m0 = (int)(blockIdx.x / n_tiles) * T;
  const int n0 = (int)(blockIdx.x % n_tiles) * T;
  float acc[MT][MT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[i][j] = 0.f;

  // element q of this thread: A row (tid + 256q) / TK, k (tid + 256q) % TK (consecutive
  // threads walk k); B k-row (tid + 256q) / T, column (tid + 256q) % T (they walk n)
  float ra[kPer], rb[kPer];
  auto load_slice = [&](int k0) {
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int e = tid + 256 * q;
      const int m = m0 + e / TK, ka = k0 + e % TK;
      ra[q] = (m < M && ka < K) ? Elem<TA>::load(A + m * sam + ka * sak) : 0.f;
      const int kb = k0 + e / T, n = n0 + e % T;
      rb[q] = (kb < K && n < N) ? Elem<TB>::load(B + kb * sbk + n * sbn) : 0.f;
    }
  };
  load_slice(0);
  for (int k0 = 0; k0 < K; k0 += TK) {
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int e = tid + 256 * q;
      As[e % TK][e / TK] = ra[q];
      Bs[e / T][e % T] = rb[q];
    }
    __syncthreads();
    if (k0 + TK < K) load_slice(k0 + TK);
#pragma unroll
    for (int kk = 0; kk < TK; ++kk) {
      float a[MT], b[MT];
#pragma unroll
      for (int i = 0; i < MT; ++i) a[i] = As[kk][ty * MT + i];
#pragma unroll
      for (int j = 0; j < MT; ++j) b[j] = Bs[kk][tx * MT + j];
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < MT; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int m = m0 + ty * MT + i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      const int n = n0 + tx * MT + j;
      if (n >= N) continue;
      float v = acc[i][j];
      if (bias != nullptr) v += Elem<TBias>::load(bias + n * sbias);
      Elem<TC>::store(C + m * scm + n * scn, v);
    }
  }
}

// One launch of gemm_pipe_kernel (grid x splits workgroups; splits > 1: fp32 partials of
// k_chunk-deep K chunks into `partial`, reduced by gemm_splitk_reduce_kernel afterwards).
// bias_kind: 0 none, 1 fp32, 2 16-bit.
template <typename Tag, int kTM, int kStages, bool kRagged>
hipError_t launch_gemm_pipe(const uint16_t* A, const uint16_t* B, uint16_t* C, const void* bias, int bias_kind, int M,
                            int N, int K, long long lda, long long ldb, long long ldc, float* partial, int k_chunk,
                            int grid, int splits, hipStream_t stream) {
#define KG_GEMM_PIPE(BIAS)                                                                                             \
  hipLaunchKernelGGL((gemm_pipe_kernel<Tag, BIAS, kTM, kStages, kRagged>), dim3(grid, splits), dim3(gemmp::kThreads), 0, \
                     stream, A, B, C, bias, M, N, K, lda, ldb, ldc, partial, k_chunk)
  if (bias_kind == 0) KG_GEMM_PIPE(0);
  else if (bias_kind == 1) KG_GEMM_PIPE(1);
  else KG_GEMM_PIPE(2);
#undef KG_GEMM_PIPE
  return hipGetLastError();
}

}  // namespace kg_gfx950
