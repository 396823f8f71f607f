// GEMM kernels for the matmul demos: out[M,N] = lhs[M,K] @ rhs[K,N] (+ bias[N]),
// row-major, fp32 accumulation.
//
// gemm_mfma_kernel: bf16/f16 operands on gfx950 MFMA (v_mfma_f32_16x16x32_{bf16,f16}).
//   Macro tile 256x256x64, 256 threads = 4 waves in a 2x2 layout, 128x128 per wave
//   (8x8 MFMA blocks, 256 fp32 accumulators per lane). LDS double buffer, 2 x 64 KiB.
//   lhs tiles are K-contiguous in HBM and land in LDS as [m][k]; rhs tiles are
//   N-contiguous, so each thread loads an 8(k) x 8(n) block with 16-byte loads and
//   transposes it in registers (v_perm_b32) before writing [n][k] rows to LDS. Both LDS
//   arrays use 128-byte rows whose 16-byte chunks are XOR-swizzled so that the MFMA
//   fragment reads (ds_read_b128) and the tile writes are bank-conflict free.
//   The MFMA is issued with the rhs fragment as operand A and the lhs fragment as
//   operand B, which yields C^T blocks: every lane then owns 4 consecutive columns of
//   one output row, stored as one 8-byte write.
//
// gemm_simt_kernel: any dtype (f32/bf16/f16), any shape and stride; 64x64 LDS tiles,
//   4x4 outputs per thread, fp32 FMA accumulation in k order.
#pragma once

#include "common.h"

namespace kg_gfx950 {

namespace gemm {

constexpr int kBM = 256;
constexpr int kBN = 256;
constexpr int kBK = 64;
constexpr int kThreads = 256;
constexpr int kChunks = kBK / 8;          // 16-byte chunks per LDS row
constexpr int kTileVecs = kBM * kChunks;  // u32x4 per operand tile (2048)

__device__ __forceinline__ int swz_a(int row, int chunk) { return row * kChunks + (chunk ^ (row & 7)); }
__device__ __forceinline__ int swz_b(int n, int chunk) {
  return n * kChunks + (chunk ^ (n & 7) ^ ((n >> 3) & 7));
}

}  // namespace gemm

// Requirements checked by the host: K % 8 == 0, N % 8 == 0, lda/ldb/ldc multiples of 8,
// 16-byte aligned base pointers. kMasked handles M, N, K that are not tile multiples.
template <typename Tag, bool kMasked, int kBias>  // kBias: 0 none, 1 fp32 bias, 2 16-bit bias
__global__ __launch_bounds__(gemm::kThreads, 1) void gemm_mfma_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, uint16_t* __restrict__ C,
    const void* __restrict__ bias, int M, int N, int K, long long lda, long long ldb, long long ldc) {
  using namespace gemm;
  using H = Half16<Tag>;
  __shared__ u32x4 lds[2][2][kTileVecs];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;

  // Workgroup -> output tile: XCD-local logical id, then groups of 4 tile-rows.
  const int tiles_m = (M + kBM - 1) / kBM;
  const int tiles_n = (N + kBN - 1) / kBN;
  const int logical = xcd_logical_id(blockIdx.x, gridDim.x);
  constexpr int kGroupM = 4;
  const int group_size = kGroupM * tiles_n;
  const int group = logical / group_size;
  const int first_m = group * kGroupM;
  const int gm = min(tiles_m - first_m, kGroupM);
  const int in_group = logical - group * group_size;
  const int tm = first_m + in_group % gm;
  const int tn = in_group / gm;
  const int m0 = tm * kBM;
  const int n0 = tn * kBN;

  // Global load assignment.
  // lhs: 8 loads per thread, row = i*32 + tid/8, chunk = tid%8.
  const int a_row = tid >> 3;
  const int a_chunk = tid & 7;
  // rhs: one 8x8 block per thread: n-block nb = tid%32, k-block kb = tid/32.
  const int b_nb = tid & 31;
  const int b_kb = tid >> 5;

  const uint16_t* a_ptr = A + (long long)(m0 + a_row) * lda + a_chunk * 8;
  const uint16_t* b_ptr = B + (long long)(b_kb * 8) * ldb + n0 + b_nb * 8;

  u32x4 a_pref[8];
  u32x4 b_pref[8];

  auto load_tile = [&](int kt) {
    const int k0 = kt * kBK;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if constexpr (kMasked) {
        const int m = m0 + i * 32 + a_row;
        const int k = k0 + a_chunk * 8;
        a_pref[i] = (m < M && k < K) ? ld16(a_ptr + (long long)i * 32 * lda + k0) : u32x4{0, 0, 0, 0};
      } else {
        a_pref[i] = ld16(a_ptr + (long long)i * 32 * lda + k0);
      }
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      if constexpr (kMasked) {
        const int k = k0 + b_kb * 8 + r;
        const int n = n0 + b_nb * 8;
        b_pref[r] = (k < K && n < N) ? ld16(b_ptr + (long long)(k0 + r) * ldb) : u32x4{0, 0, 0, 0};
      } else {
        b_pref[r] = ld16(b_ptr + (long long)(k0 + r) * ldb);
      }
    }
  };

  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = i * 32 + a_row;
      lds[buf][0][swz_a(row, a_chunk)] = a_pref[i];
    }
    u32x4 bt[8];
    transpose8x8_b16(b_pref, bt);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int n = b_nb * 8 + j;
      lds[buf][1][swz_b(n, b_kb)] = bt[j];
    }
  };

  f32x4 acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int ktiles = (K + kBK - 1) / kBK;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  const int frag_row = lane & 15;
  const int frag_chunk = lane >> 4;

  for (int kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < ktiles) load_tile(kt + 1);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int c = kk * 4 + frag_chunk;
      u32x4 af[8];
      u32x4 bf[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) af[i] = lds[cur][0][swz_a(wm * 128 + i * 16 + frag_row, c)];
#pragma unroll
      for (int j = 0; j < 8; ++j) bf[j] = lds[cur][1][swz_b(wn * 128 + j * 16 + frag_row, c)];
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = H::mfma16(bf[j], af[i], acc[i][j]);
    }
    if (kt + 1 < ktiles) store_tile(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: lane owns C[m][n..n+3] of every 16x16 block.
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int m = m0 + wm * 128 + i * 16 + frag_row;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int n = n0 + wn * 128 + j * 16 + frag_chunk * 4;
      f32x4 v = acc[i][j];
      if constexpr (kBias == 1) {
        const float* bp = static_cast<const float*>(bias);
        if (!kMasked || n < N) {
          v[0] += bp[n];
          v[1] += bp[n + 1];
          v[2] += bp[n + 2];
          v[3] += bp[n + 3];
        }
      } else if constexpr (kBias == 2) {
        const uint16_t* bp = static_cast<const uint16_t*>(bias);
        if (!kMasked || n < N) {
          v[0] += H::to_float(bp[n]);
          v[1] += H::to_float(bp[n + 1]);
          v[2] += H::to_float(bp[n + 2]);
          v[3] += H::to_float(bp[n + 3]);
        }
      }
      u32x2 packed;
      packed[0] = pack16(H::from_float(v[0]), H::from_float(v[1]));
      packed[1] = pack16(H::from_float(v[2]), H::from_float(v[3]));
      if (!kMasked || (m < M && n < N)) st8(C + (long long)m * ldc + n, packed);
    }
  }
}

// Generic path: any element type, any shape/strides (element strides), optional bias.
// Each 256-thread block computes a 64x64 tile; each thread a 4x4 micro tile.
template <typename TA, typename TB, typename TC, typename TBias>
__global__ __launch_bounds__(256) void gemm_simt_kernel(const TA* __restrict__ A, const TB* __restrict__ B,
                                                        TC* __restrict__ C, const TBias* __restrict__ bias,
                                                        int M, int N, int K, long long sam, long long sak,
                                                        long long sbk, long long sbn, long long scm,
                                                        long long scn, long long sbias) {
  constexpr int T = 64;
  constexpr int TK = 16;
  __shared__ float As[TK][T + 1];
  __shared__ float Bs[TK][T + 1];
  const int tid = threadIdx.x;
  const int tx = tid & 15;
  const int ty = tid >> 4;
  const int m0 = blockIdx.y * T;
  const int n0 = blockIdx.x * T;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;

  for (int k0 = 0; k0 < K; k0 += TK) {
    for (int e = tid; e < T * TK; e += 256) {
      const int r = e / TK;
      const int kk = e % TK;
      const int m = m0 + r;
      const int k = k0 + kk;
      As[kk][r] = (m < M && k < K) ? Elem<TA>::load(A + m * sam + k * sak) : 0.f;
    }
    for (int e = tid; e < T * TK; e += 256) {
      const int kk = e / T;
      const int c = e % T;
      const int k = k0 + kk;
      const int n = n0 + c;
      Bs[kk][c] = (k < K && n < N) ? Elem<TB>::load(B + k * sbk + n * sbn) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < TK; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + ty * 4 + i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + tx * 4 + j;
      if (n >= N) continue;
      float v = acc[i][j];
      if (bias != nullptr) v += Elem<TBias>::load(bias + n * sbias);
      Elem<TC>::store(C + m * scm + n * scn, v);
    }
  }
}

}  // namespace kg_gfx950
