// Implicit-GEMM conv2d on gfx950 MFMA for 16-bit NCHW tensors with C = F = 64,
// a 3x3 window, stride 1, dilation 1 and padding 1 on every side (so Ho = H, Wo = W),
// W a multiple of 8 and at most 56; fp32 accumulation.
//
// GEMM view per output row: Y^T[w][f] = sum_k X[w][k] W^T[k][f] with the contraction index k
// ordered (tap = 3*kh + kw, channel): 36 steps of 16 = 9 taps x 4 channel groups. In that
// order 8 consecutive k of one pixel are 8 consecutive channels, so with the input tile
// stored channel-last in LDS an MFMA operand-A fragment (v_mfma_f32_32x32x16: 8 k of one
// pixel per lane) is one 16-byte read.
//
// One workgroup per 7 output rows of one image (the C3 shape, N=32 and H=56, is 256
// workgroups: one per CU), and the row blocks of one image on one XCD, so the two halo rows
// two blocks share are fetched from HBM once and served to the second block by that XCD's
// L2. 8 waves in two roles, one of each per SIMD:
//  - compute waves 0-3: wave = (filter block fb, pixel block pb), 32 filters x 32 pixels.
//    Each holds its filters' weights for all 576 k in registers (36 operand-B fragments),
//    so the inner loop reads only input fragments from LDS. Output rows are computed in
//    phases of 2, 3 and 2 rows (one accumulator per row), and each phase's results go to
//    one of two LDS output buffers.
//  - staging waves 4-7: load the 9 input rows of the block in two parts, tile rows 0-3
//    and 4-8 (rows outside the image are zeros), the second once the first is stored, so
//    that at the start of the kernel HBM serves only what the first phase needs. Each wave
//    takes two channel octets: one load instruction per channel reads the part's W*2-byte
//    row pieces, which are contiguous in NCHW, and lane (tile row, 8-column block) ends up
//    with an 8-channel x 8-column block, which it transposes in registers and writes
//    channel-last into LDS. Afterwards they write each finished phase's output buffer to
//    HBM as coalesced 16-byte stores while the compute waves run the next phase.
// The weights reach LDS with whole-wave 1 KiB loads (L2-resident after the first
// workgroups) and are moved into registers while the input rows are still arriving.
//
// LDS layout (64 banks of 4 bytes; ds_read_b128 serves 16 lanes per cycle): a pixel of the
// input tile is 128 bytes (8 chunks of 8 channels); chunk c of column col sits at slot
// c ^ ((col >> 1) & 7), so 16 consecutive pixels at one chunk hit 16 distinct 16-byte bank
// groups. Tile rows are 16 bytes longer than their 58 columns: a staging write (lanes =
// (tile row, 8-column block) at one column offset and chunk) then meets each bank group from
// at most 4 addresses where a whole-256-byte pitch put up to 9 on one. Weights are [f][576 values] with rows padded to 1168 bytes, so 16 consecutive
// filters at one offset fall in distinct bank groups. Output buffers (in the weight area,
// once the weights are in registers) are laid out [f][row][w] like Y with filter planes
// padded so the 8-byte writes of 32 consecutive filters spread over all bank groups.
#pragma once

#include "conv2d.h"
#include "lds_dma.h"

namespace kg_gfx950 {

namespace convk {

constexpr int kThreads = 512;       // waves 0-3 compute, waves 4-7 stage
constexpr int kStageThreads = 256;
constexpr int kRows = 7;            // output rows per workgroup
constexpr int kInRows = kRows + 2;  // input rows per workgroup
constexpr int kCols = 58;           // LDS tile columns: W <= 56 plus two zero columns
constexpr int kC = 64;
constexpr int kF = 64;
constexpr int kKSteps = 36;                      // 9 taps x 4 groups of 16 channels
constexpr int kRowPitch = kCols * 128 + 16;      // bytes per tile row (see the LDS layout)
constexpr int kXBytes = kInRows * kRowPitch;     // channel-last input tile
constexpr int kWPitch = kC * 9 * 2 + 16;         // one filter's weights in LDS, padded
constexpr int kWBytes = kF * kWPitch;
constexpr int kMaxPhaseRows = 3;
constexpr int kOutBytes = kF * (kMaxPhaseRows * (kCols - 2) * 2 + 16);  // one output buffer
static_assert(2 * kOutBytes <= kWBytes, "the output buffers reuse the weight area");

__host__ __device__ constexpr int x_slot(int col, int c8) { return c8 ^ ((col >> 1) & 7); }
// Filter-plane stride of an output buffer holding R rows: R*W*2 bytes, rounded so that
// stride/16 is odd.
__host__ __device__ constexpr int out_stride(int R, int W) { return R * W * 2 + (((R * W / 8) & 1) ? 0 : 16); }

}  // namespace convk

// Barrier schedule (both roles meet at the same five barriers):
//   step  staging waves                          compute waves
//   0     load tile rows 0-3, zero columns       weights HBM/L2 -> LDS
//   1     tile rows 0-3 -> LDS, load rows 4-8    weights -> registers
//   2     tile rows 4-8 -> LDS                   rows 0-1 -> output buffer 0
//   3     write buffer 0                         rows 2-4 -> output buffer 1
//   4     write buffer 1                         rows 5-6 -> output buffer 0
//   5     write buffer 0                         -
template <typename Tag, int kBias>  // kBias: 0 none, 1 fp32, 2 16-bit
__global__ __launch_bounds__(convk::kThreads, 1) void conv2d_3x3s1p1_mfma_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, uint16_t* __restrict__ y,
    const void* __restrict__ bias, int N, int H, int W) {
  using namespace convk;
  using Hf = Half16<Tag>;
  __shared__ __attribute__((aligned(1024))) u32x4 lds[(kXBytes + kWBytes) / 16];
  u32x4* x_lds = lds;                                            // [row][col][8 chunks]
  char* w_lds = reinterpret_cast<char*>(lds + kXBytes / 16);     // [f][576 values + pad]
  char* out_lds = w_lds;  // two output buffers, once the weights are in registers

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  const int row_blocks = (H + kRows - 1) / kRows;
  const int unit = xcd_logical_id(blockIdx.x, gridDim.x);
  const int n = unit / row_blocks;
  const int r0 = (unit - n * row_blocks) * kRows;  // first output row
  const long long hw = (long long)H * W;

  if (wave >= 4) {
    // ================= staging waves =================
    const int wblocks = W >> 3;
    // Two parts of the tile: rows 0-3 (what output rows 0-1 need) and rows 4-8. In part q,
    // lane = (tile row kHalfRow0[q] + lane / wblocks, 8-column block lane % wblocks); wave v
    // holds channel octets 2(v-4) and 2(v-4)+1. Tile row t is input row r0 - 1 + t.
    constexpr int kHalfRow0[2] = {0, 4};
    constexpr int kHalfRows[2] = {4, 5};
    const int oct0 = 2 * (wave - 4);
    const int lrow = lane / wblocks;
    const int col = lane - lrow * wblocks;
    u32x4 set[2][2][8];  // [half][octet][channel]
    auto load_half = [&](int q) {
      const int h = r0 - 1 + kHalfRow0[q] + lrow;
      if (lrow < kHalfRows[q] && h >= 0 && h < H) {
        const uint16_t* src = x + ((long long)n * kC + 8 * oct0) * hw + (long long)h * W + 8 * col;
#pragma unroll
        for (int o = 0; o < 2; ++o)
#pragma unroll
          for (int e = 0; e < 8; ++e) set[q][o][e] = ld16(src + (8 * o + e) * hw);
      } else {
#pragma unroll
        for (int o = 0; o < 2; ++o)
#pragma unroll
          for (int e = 0; e < 8; ++e) set[q][o][e] = u32x4{0, 0, 0, 0};
      }
    };
    load_half(0);
    auto store_half = [&](int q) {
      if (lrow >= kHalfRows[q]) return;
      const int base = (kHalfRow0[q] + lrow) * (kRowPitch / 16) + (1 + 8 * col) * 8;
#pragma unroll
      for (int o = 0; o < 2; ++o) {
        u32x4 cols[8];
        transpose8x8_b16(set[q][o], cols);
#pragma unroll
        for (int j = 0; j < 8; ++j) x_lds[base + 8 * j + x_slot(1 + 8 * col + j, oct0 + o)] = cols[j];
      }
    };
    // Output rows row0 .. row0+R-1 of buffer `buf` to HBM. Staging wave v (4..7) writes
    // filters 16(v-4) .. +15, two per pass (lane / 32), 16 bytes per lane: a filter's rv rows
    // are rv*W/8 <= 21 consecutive chunks of Y. Rows past H are not written.
    auto flush = [&](int row0, int R, int buf) {
      const int ho0 = r0 + row0;
      const int rv = min(R, H - ho0);
      const int per_f = rv * W / 8;
      const int k = lane & 31;
      if (rv <= 0 || k >= per_f) return;
      const int stride = out_stride(R, W);
      const char* ob = out_lds + buf * kOutBytes;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int f2 = (wave - 4) * 16 + 2 * i + (lane >> 5);
        const u32x4 v = *reinterpret_cast<const u32x4*>(ob + f2 * stride + 16 * k);
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(y + ((long long)n * kF + f2) * hw + (long long)ho0 * W + 8 * k));
      }
    };

    // zero columns (0 and W+1 .. kCols-1) of every tile row
    const int zcols = kCols - W;
    for (int i = tid - kStageThreads; i < kInRows * zcols * 8; i += kStageThreads) {
      const int c8 = i & 7;
      const int zc = (i >> 3) % zcols;
      const int r = (i >> 3) / zcols;
      const int zcol = zc == 0 ? 0 : W + zc;
      x_lds[r * (kRowPitch / 16) + zcol * 8 + x_slot(zcol, c8)] = u32x4{0, 0, 0, 0};
    }
    __syncthreads();  // 1
    store_half(0);
    load_half(1);
    __syncthreads();  // 2
    store_half(1);
    __syncthreads();  // 3
    flush(0, 2, 0);
    __syncthreads();  // 4
    flush(2, 3, 1);
    __syncthreads();  // 5
    flush(5, 2, 0);
    return;
  }

  // ================= compute waves: (filter block fb, pixel block pb) =================
  const int fb = wave >> 1;
  const int pb = wave & 1;
  const int f = 32 * fb + (lane & 31);
  const int hsel = lane >> 5;
  const bool live = 32 * pb < W;  // wave-uniform

  // The weights (64 filters x 576 values in (channel, kh, kw) order, 73,728 contiguous
  // bytes) go to LDS first, each wave copying a quarter with whole-wave 1 KiB loads.
#pragma unroll
  for (int i = 0; i < 18; ++i) {
    const int g = wave * 18432 + i * 1024 + 16 * lane;
    const int fr = g / 1152;
    *reinterpret_cast<u32x4*>(w_lds + fr * kWPitch + (g - fr * 1152)) = ld16(reinterpret_cast<const char*>(w) + g);
  }
  // Operand-B fragments: wreg[4*tap + cg] = channels 16cg + 8hsel .. +7 of filter f at tap.
  // The 8 channels 16cg + 8hsel .. +7 at all 9 taps are 72 contiguous values (nine 16-byte
  // reads); element e of them is channel e / 9 at tap e % 9.
  u32x4 wreg[kKSteps];
  auto read_w = [&](int cg) {
    u32x4 raw[9];
    const char* wsrc = w_lds + f * kWPitch + hsel * 144 + cg * 288;
#pragma unroll
    for (int i = 0; i < 9; ++i) raw[i] = *reinterpret_cast<const u32x4*>(wsrc + 16 * i);
#pragma unroll
    for (int u = 0; u < 9; ++u) {
      u32x4 frag;
#pragma unroll
      for (int q = 0; q < 4; ++q) {  // channels 2q, 2q+1 at tap u: elements 9*(2q)+u, 9*(2q+1)+u
        const int e0 = (2 * q) * 9 + u;
        const int e1 = (2 * q + 1) * 9 + u;
        const uint32_t a = raw[e0 >> 3][(e0 >> 1) & 3];
        const uint32_t b = raw[e1 >> 3][(e1 >> 1) & 3];
        const uint32_t lo = (e0 & 1) ? (a >> 16) : (a & 0xffffu);
        const uint32_t hi = (e1 & 1) ? (b >> 16) : (b & 0xffffu);
        frag[q] = lo | (hi << 16);
      }
      wreg[4 * u + cg] = frag;
    }
  };

  const uint32_t lds0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)&lds[0];
  // A operand: pixel w = 32pb + lane%32 (dead lanes past W read column W-1), channels
  // 16cg + 8hsel .. +7 at tap (kh, kw): LDS byte (r + kh)*pitch + (w + kw)*128 + 16*slot.
  const int wpix = min(32 * pb + (lane & 31), W - 1);
  uint32_t a_off[3][4];
#pragma unroll
  for (int kw = 0; kw < 3; ++kw)
#pragma unroll
    for (int cg = 0; cg < 4; ++cg) {
      const int col = wpix + kw;
      a_off[kw][cg] = lds0 + col * 128 + 16 * x_slot(col, 2 * cg + hsel);
    }
  auto read_a = [&](int kw, int cg, int trow) -> u32x4 {  // tile row trow, column offset kw
    return *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)(a_off[kw][cg] + trow * kRowPitch);
  };
  float bv = 0.f;
  if constexpr (kBias == 1) bv = static_cast<const float*>(bias)[f];
  if constexpr (kBias == 2) bv = Hf::to_float(static_cast<const uint16_t*>(bias)[f]);

  // Groups [g0, g1) of a phase over output rows row0 .. row0+R-1. Output row r at tap
  // (kh, kw) reads tile row r + kh, so group g = 3*cg + kw (channel group cg, column offset
  // kw) reads the R+2 fragments of tile rows row0 .. row0+R+1 once and runs its 3R MFMAs
  // (kh = 0..2, r = 0..R-1) on them: R+2 LDS reads per 3R MFMAs. The next group's fragments
  // are read while the current group's MFMAs run.
  auto groups = [&](auto rows_tag, int row0, f32x16* acc, int g0, int g1, bool first) {
    constexpr int R = decltype(rows_tag)::value;
    constexpr int T = R + 2;
    u32x4 af[13][T];
#pragma unroll
    for (int t = 0; t < T; ++t) af[g0][t] = read_a(g0 - 3 * (g0 / 3), g0 / 3, row0 + t);
#pragma unroll
    for (int g = g0; g < g1; ++g) {
      const int cg = g / 3, kw = g - 3 * (g / 3);
      const int ncg = (g + 1) / 3, nkw = (g + 1) - 3 * ((g + 1) / 3);
      int i = 0;
#pragma unroll
      for (int kh = 0; kh < 3; ++kh)
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (first && g == g0 && kh == 0)
            acc[r] = Hf::mfma32(af[g][r], wreg[4 * kw + cg], f32x16{});
          else
            acc[r] = Hf::mfma32(af[g][r + kh], wreg[4 * (3 * kh + kw) + cg], acc[r]);
          if (g + 1 < g1 && i < T) af[g + 1][i] = read_a(nkw, ncg, row0 + i);
          ++i;
          __builtin_amdgcn_sched_barrier(0);
        }
    }
  };
  // Output rows row0 .. row0+R-1 into output buffer `buf` ([f][row][w]; lane holds filter f,
  // pixels 32pb + 8j + 4*hsel + 0..3 of each row).
  auto stage_out = [&](auto rows_tag, const f32x16* acc, int buf) {
    constexpr int R = decltype(rows_tag)::value;
    const int stride = out_stride(R, W);
    char* ob = out_lds + buf * kOutBytes;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int wo = 32 * pb + 8 * j + 4 * hsel;
        if (wo < W) {
          u32x2 packed;
          if constexpr (kBias == 0) {
            packed[0] = Hf::pack2(acc[r][4 * j], acc[r][4 * j + 1]);
            packed[1] = Hf::pack2(acc[r][4 * j + 2], acc[r][4 * j + 3]);
          } else {
            packed[0] = Hf::pack2(acc[r][4 * j] + bv, acc[r][4 * j + 1] + bv);
            packed[1] = Hf::pack2(acc[r][4 * j + 2] + bv, acc[r][4 * j + 3] + bv);
          }
          *reinterpret_cast<u32x2*>(ob + f * stride + (r * W + wo) * 2) = packed;
        }
      }
  };

  __syncthreads();  // 1: weights in LDS
  if (live) {
#pragma unroll
    for (int cg = 0; cg < 4; ++cg) read_w(cg);
  }
  __syncthreads();  // 2: tile rows 0-3 in LDS; every wave's weights are in registers
  if (live) {
    f32x16 acc[2];
    groups(Int<2>{}, 0, acc, 0, 12, true);
    stage_out(Int<2>{}, acc, 0);
  }
  __syncthreads();  // 3: tile rows 4-8 in LDS; rows 0-1 in buffer 0
  if (live) {
    f32x16 acc[3];
    groups(Int<3>{}, 2, acc, 0, 12, true);
    stage_out(Int<3>{}, acc, 1);
  }
  __syncthreads();  // 4: rows 2-4 in buffer 1
  if (live) {
    f32x16 acc[2];
    groups(Int<2>{}, 5, acc, 0, 12, true);
    stage_out(Int<2>{}, acc, 0);
  }
  __syncthreads();  // 5: rows 5-6 in buffer 0
}

inline bool conv_mfma_supported(const ConvShape& s) {
  return s.c == convk::kC && s.f == convk::kF && s.kh == 3 && s.kw == 3 && s.sh == 1 && s.sw == 1 && s.dh == 1 &&
         s.dw == 1 && s.pt == 1 && s.pl == 1 && s.ho == s.h && s.wo == s.w && s.w % 8 == 0 && s.w >= 8 &&
         s.w <= convk::kCols - 2 && s.h >= 1 && s.n >= 1 &&
         (long long)s.n * ((s.h + convk::kRows - 1) / convk::kRows) < (1ll << 31);
}

template <typename Tag>
hipError_t launch_conv2d_mfma(const uint16_t* x, const uint16_t* w, uint16_t* y, const void* bias, int bias_kind,
                              const ConvShape& s, hipStream_t stream) {
  const int grid = s.n * ((s.h + convk::kRows - 1) / convk::kRows);
  if (bias_kind == 1)
    hipLaunchKernelGGL((conv2d_3x3s1p1_mfma_kernel<Tag, 1>), dim3(grid), dim3(convk::kThreads), 0, stream, x, w, y, bias,
                       s.n, s.h, s.w);
  else if (bias_kind == 2)
    hipLaunchKernelGGL((conv2d_3x3s1p1_mfma_kernel<Tag, 2>), dim3(grid), dim3(convk::kThreads), 0, stream, x, w, y, bias,
                       s.n, s.h, s.w);
  else
    hipLaunchKernelGGL((conv2d_3x3s1p1_mfma_kernel<Tag, 0>), dim3(grid), dim3(convk::kThreads), 0, stream, x, w, y, bias,
                       s.n, s.h, s.w);
  return hipGetLastError();
}

}  // namespace kg_gfx950
