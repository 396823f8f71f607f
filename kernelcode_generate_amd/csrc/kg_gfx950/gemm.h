// GEMM kernels for the matmul demos: out[M,N] = lhs[M,K] @ rhs[K,N] (+ bias[N]),
// row-major, fp32 accumulation.
//
// gemm_pipe_kernel: bf16/f16 operands on gfx950 MFMA (v_mfma_f32_32x32x16_{bf16,f16}; the
//   32x32x16 form is the one that reaches full matrix-core rate on gfx950, the 16x16x32
//   form issues at half of it), any M, N % 8 == 0, K % 8 == 0.
//
// gemm_simt_kernel: any dtype (f32/bf16/f16), any shape and stride; 64x64 LDS tiles,
//   4x4 outputs per thread, fp32 FMA accumulation in k order.
#pragma once

#include "common.h"
#include "lds_dma.h"

namespace kg_gfx950 {

// gemm_pipe_kernel: kTM x 256 tiles (kTM = 256, or 128 when 256-row tiles would leave CUs idle) computed by
//   8 waves (2 x 4 waves of kTM/2 x 64, two per SIMD) with 32x32x16 MFMAs. Both operands
//   are copied HBM -> LDS by global_load_lds_dwordx4 (no registers, no VALU work) through a
//   kStages-deep ring of 32-deep K slices (kStages x (kTM/16 + 16) KiB; 4 by default, 2 or
//   3 on request), so loads are issued kStages - 1 slices ahead of their use; every wave issues kTM/128 + 2 of a slice's copies (1 KiB
//   each), slotted between its MFMAs, and while one wave of a SIMD waits on a copy's issue
//   or an LDS read the other keeps the MFMA pipe busy. lhs slices are [m][k] rows of 64 bytes; rhs slices
//   stay [k][n] as in HBM and the MFMA operand (8 consecutive k of one n) is read with two
//   ds_read_b64_tr_b16: within each 16-lane group, lane j addresses 4 consecutive n of
//   k-row j/4 and lane i receives k-rows 0..3 of column i. Chunk swizzles: lhs
//   p = c ^ ((row >> 2) & 3), rhs p = c ^ 4(k & 3) -- the fragment reads hit distinct
//   banks of the 64-bank LDS. Fragments are double-buffered in registers: while the MFMAs
//   of one 16-deep half of a slice run, the other half (or the next slice's first half) is
//   being read, and the per-slice barrier sits between the two halves.
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
__device__ __forceinline__ int b_mask(int k) { return 4 * (k & 3); }
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
  constexpr int MI = kTM / 64;              // 32-row fragments per wave
  constexpr int AP = kTM / 128;             // lhs copies per wave per slice
  constexpr int kPieces = AP + 2;           // copies per wave per slice: AP lhs, 2 rhs
  constexpr int NR = MI + 4;                // fragment reads per half slice: MI lhs, 4 rhs
  constexpr int NM = 2 * MI;                // MFMAs per half slice
  constexpr int NSTEP = NM > NR ? NM : NR;  // interleave steps per half slice
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

  // ---- fragment reads ----
  // lhs block i is 32 rows below block 0 (same mask): +2048 bytes; rhs k-rows +4 (t) and
  // +16 (ks) keep the mask: +2048 / +8192 bytes. Per-lane byte addresses, LDS base included.
  const int frag_row = lane & 31;
  const int frag_half = lane >> 5;
  const int g = lane >> 4;
  const int j16 = lane & 15;
  const int b_nofs = 16 * (g & 1) + 4 * (j16 & 3);
  const int b_kofs = 8 * (g >> 1) + (j16 >> 2);
  uint32_t a_rd[2], b_rd[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) a_rd[ks] = lds_a0 + a_slot(wm * (kTM / 2) + frag_row, 2 * ks + frag_half) * 16;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = wn * 64 + j * 32 + b_nofs;
    b_rd[j] = lds_b0 + b_slot(b_kofs, n >> 3) * 16 + (n & 7) * 2;
  }

  struct Frag {
    u32x4 a[MI];
    u32x4 b[2];
  };
  // read #r (0..NR-1) of a fragment set: MI lhs b128 reads, then 4 rhs transposed reads
  auto read_piece = [&](int s, int ks, Frag& f, int r) {
    if (r < MI) {
      f.a[r] = *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)(a_rd[ks] + s * kAStage + r * 2048);
    } else {
      const int j = (r - MI) >> 1, t = (r - MI) & 1;
      const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)(uintptr_t)(b_rd[j] + s * kBStage + t * 2048 + ks * 8192));
      const u32x2 w = __builtin_bit_cast(u32x2, v);
      f.b[j][2 * t] = w[0];
      f.b[j][2 * t + 1] = w[1];
    }
  };

  f32x16 acc[MI][2];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

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
  Frag f0, f1;
#pragma unroll
  for (int r = 0; r < NR; ++r) read_piece(0, 0, f0, r);

  // One 32-deep slice in stage S: MFMAs of half 0 with the reads of half 1 slotted in
  // between, barrier, MFMAs of half 1 with the next slice's first reads and this stage's
  // refill copies slotted in between. kSteady: more slices follow and a refill is due.
  auto slice = [&](int kt, auto stage_tag, auto steady_tag) {
    constexpr int S = decltype(stage_tag)::value;
    constexpr bool kSteady = decltype(steady_tag)::value != 0;
#pragma unroll
    for (int idx = 0; idx < NSTEP; ++idx) {
      const int i = idx >> 1, j = idx & 1;
      if (idx < NM) acc[i][j] = H::mfma32(f0.b[j], f0.a[i], acc[i][j]);
      if (idx < NR) read_piece(S, 1, f1, idx);
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
      for (int idx = 0; idx < NSTEP; ++idx) {
        const int i = idx >> 1, j = idx & 1;
        if (idx < NM) acc[i][j] = H::mfma32(f1.b[j], f1.a[i], acc[i][j]);
        if (idx < NR) read_piece((S + 1) % kStages, 0, f0, idx);
        if ((idx & 1) && (idx >> 1) < kPieces) issue_piece(kt + kStages, S, idx >> 1);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      if (refill)
#pragma unroll
        for (int piece = 0; piece < kPieces; ++piece) issue_piece(kt + kStages, S, piece);
      if (more)
#pragma unroll
        for (int r = 0; r < NR; ++r) read_piece((S + 1) % kStages, 0, f0, r);
#pragma unroll
      for (int idx = 0; idx < NM; ++idx) {
        const int i = idx >> 1, j = idx & 1;
        acc[i][j] = H::mfma32(f1.b[j], f1.a[i], acc[i][j]);
      }
    }
  };

  int kt = 0;
  for (; kt + 2 * kStages <= ktiles; kt += kStages) {  // every slice refills its stage
    slice(kt, StageIdx<0>{}, StageIdx<1>{});
    slice(kt + 1, StageIdx<1>{}, StageIdx<1>{});
    if constexpr (kStages > 2) slice(kt + 2, StageIdx<2 % kStages>{}, StageIdx<1>{});
    if constexpr (kStages > 3) slice(kt + 3, StageIdx<3 % kStages>{}, StageIdx<1>{});
  }
  for (; kt < ktiles; kt += kStages) {
    slice(kt, StageIdx<0>{}, StageIdx<0>{});
    if (kt + 1 < ktiles) slice(kt + 1, StageIdx<1>{}, StageIdx<0>{});
    if constexpr (kStages > 2)
      if (kt + 2 < ktiles) slice(kt + 2, StageIdx<2 % kStages>{}, StageIdx<0>{});
    if constexpr (kStages > 3)
      if (kt + 3 < ktiles) slice(kt + 3, StageIdx<3 % kStages>{}, StageIdx<0>{});
  }

#pragma unroll
  for (int i = 0; i < MI; ++i) {
    const int m = m0 + wm * (kTM / 2) + i * 32 + frag_row;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn * 64 + j * 32 + 8 * q + 4 * frag_half;
        if (kRagged && (m >= M || n >= N)) continue;  // N % 8 == 0: n < N covers n .. n+3
        float v0 = acc[i][j][4 * q], v1 = acc[i][j][4 * q + 1], v2 = acc[i][j][4 * q + 2], v3 = acc[i][j][4 * q + 3];
        if (k_chunk > 0) {
          *reinterpret_cast<f32x4*>(partial + (long long)m * N + n) = f32x4{v0, v1, v2, v3};
          continue;
        }
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
        st8(C + (long long)m * ldc + n, packed);
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

}  // namespace kg_gfx950
