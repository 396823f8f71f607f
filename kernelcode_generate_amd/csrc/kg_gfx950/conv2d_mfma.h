// Implicit-GEMM conv2d on gfx950 MFMA for 16-bit NCHW tensors with C = F = 64,
// a 3x3 window, stride 1, dilation 1 and padding 1 on every side (so Ho = H, Wo = W),
// W a multiple of 8 and at most 56; fp32 accumulation.
//
// GEMM view per output row: Y^T[w][f] = sum_k X[w][k] W^T[k][f] with the contraction index k
// ordered (tap = 3*kh + kw, channel): 36 steps of 16 = 9 taps x 4 channel groups. In that
// order 8 consecutive k of one pixel are 8 consecutive channels, so with the input tile
// stored channel-last in LDS an MFMA operand-A fragment (v_mfma_f32_32x32x16: 8 k of one
// pixel per lane) is one 16-byte read, and so is an operand-B fragment from the reordered
// weights.
//
// One workgroup per 7 output rows of one image: the C3 shape (N=32, H=56) is 256
// workgroups, one per CU, of 8 waves in two roles, one of each per SIMD. Compute waves 0-3:
// wave w owns filter block w >> 1 and pixel block w & 1 (32 each) of all 7 rows: 7
// accumulators, and per k step one weight fragment shared by 7 input fragments (252 MFMAs
// per wave). Staging waves 4-7 put the weights (rewritten per tap into k order) and the 9
// input rows (8-channel x 8-column blocks loaded along W, transposed in registers and
// written channel-last, with a zero column on each side and zero rows outside the image)
// into LDS one channel group of 16 at a time while the compute waves run the previous
// group, and write finished output rows to HBM while the compute waves run the next rows,
// so staging and MFMA work overlap instead of alternating.
//
// LDS layout (64 banks of 4 bytes; ds_read_b128 serves 16 lanes per cycle): a pixel of the
// input tile is 128 bytes (8 chunks of 8 channels); chunk c of column col sits at slot
// c ^ ((col >> 1) & 7), so 16 consecutive pixels at one chunk hit 16 distinct 16-byte bank
// groups. A weight fragment (filter f, 8 channels) is 16 bytes at slot h ^ ((f >> 3) & 1)
// of the filter's 32-byte pair.
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
constexpr int kXBytes = kInRows * kCols * 128;   // channel-last input tile
constexpr int kWBytes = kKSteps * kF * 32;       // weights: 16 channels x 2 bytes per (step, f)

__host__ __device__ constexpr int x_slot(int col, int c8) { return c8 ^ ((col >> 1) & 7); }
__host__ __device__ constexpr int w_slot(int f, int h) { return h ^ ((f >> 3) & 1); }

}  // namespace convk

template <typename Tag, int kBias>  // kBias: 0 none, 1 fp32, 2 16-bit
__global__ __launch_bounds__(convk::kThreads, 1) void conv2d_3x3s1p1_mfma_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, uint16_t* __restrict__ y,
    const void* __restrict__ bias, int N, int H, int W) {
  using namespace convk;
  using Hf = Half16<Tag>;
  __shared__ __attribute__((aligned(1024))) u32x4 lds[(kXBytes + kWBytes) / 16];
  u32x4* x_lds = lds;                  // [row][col][8 chunks]
  u32x4* w_lds = lds + kXBytes / 16;   // [step][f][2 chunks]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  const int row_blocks = (H + kRows - 1) / kRows;
  const int n = blockIdx.x / row_blocks;
  const int r0 = (blockIdx.x - n * row_blocks) * kRows;  // first output row

  // ---- roles: waves 0-3 run the MFMAs, waves 4-7 (staging thread st = t - 256) load,
  // reorder and store the next channel group and write finished outputs to HBM, so a step
  // costs max(compute, staging) instead of their sum. Each SIMD holds one wave of each. ----
  const bool stager = wave >= 4;  // wave-uniform
  const int st = tid - kStageThreads;
  // Staging, fixed per thread (every channel group cg uses the same roles): st 0..127:
  // weights of filter st/2, channel octet 2cg + (st&1) (144 contiguous bytes: 8 channels x
  // 9 taps), rewritten per tap into k order. st 128..255: input block b = st - 128 = (tile
  // row, octet 2cg + parity, 8-column block) of tile rows 0..8 (tile row r holds input row
  // r0 - 1 + r): 8 rows of 16 bytes along W, transposed to channel-last. Sources and LDS
  // destinations are computed once here.
  const bool w_role = stager && st < 128;  // wave-uniform
  const int wf = (st >> 1) & 63, wh = st & 1;
  const uint16_t* w_src = w + (long long)wf * (kC * 9) + wh * 72;
  const int w_dst = wf * 2 + w_slot(wf, wh);
  const int wblocks = W >> 3;
  const int in_blocks = kInRows * 2 * wblocks;  // <= 126 for W <= 56
  const int xb = (stager && !w_role) ? st - 128 : 0;
  const int xb_col = xb % wblocks;
  const int xb_par = (xb / wblocks) & 1;
  const int xb_row = xb / (2 * wblocks);
  const int x_h = r0 - 1 + xb_row;
  const bool x_store = stager && !w_role && xb < in_blocks;
  const bool x_load = x_store && x_h >= 0 && x_h < H;
  const long long hw = (long long)H * W;
  const uint16_t* x_src = x + ((long long)n * kC + 8 * xb_par) * hw + (long long)(x_load ? x_h : 0) * W + 8 * xb_col;
  const int x_dst = (xb_row * kCols + 1 + 8 * xb_col) * 8;  // column 1 + 8*xb_col, chunk 0

  // Loads of channel group cg into the register set. Every path writes all nine entries:
  // with paths that write different entries the compiler merges the stores through a
  // selected pointer and moves the set to scratch memory.
  auto stage_load = [&](u32x4 (&stage)[9], int cg) {
    if (w_role) {
#pragma unroll
      for (int i = 0; i < 9; ++i) stage[i] = ld16(w_src + cg * 144 + 8 * i);
    } else {
      if (x_load) {
#pragma unroll
        for (int e = 0; e < 8; ++e) stage[e] = ld16(x_src + cg * 16 * hw + e * hw);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) stage[e] = u32x4{0, 0, 0, 0};
      }
      stage[8] = u32x4{0, 0, 0, 0};
    }
  };
  // w_lds[(step*64 + f)*2 + w_slot(f, h)] holds channels 16*(step&3) + 8h .. +7 of filter f at
  // tap step>>2: tap u of the weight role's octet.
  auto store_w = [&](const u32x4 (&stage)[9], int cg, int u) {
    u32x4 frag;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // channels 2q and 2q+1 of the octet at tap u: elements (2q)*9+u and (2q+1)*9+u
      const int e0 = (2 * q) * 9 + u;
      const int e1 = (2 * q + 1) * 9 + u;
      const uint32_t a = stage[e0 >> 3][(e0 >> 1) & 3];
      const uint32_t b = stage[e1 >> 3][(e1 >> 1) & 3];
      const uint32_t lo = (e0 & 1) ? (a >> 16) : (a & 0xffffu);
      const uint32_t hi = (e1 & 1) ? (b >> 16) : (b & 0xffffu);
      frag[q] = lo | (hi << 16);
    }
    w_lds[(4 * u + cg) * kF * 2 + w_dst] = frag;
  };
  // The input tile is channel-last: chunk c of column col at x_slot(col, c). Column
  // 1 + 8*xb_col + j has mask ((1 + 8*xb_col + j) >> 1) & 7 = (4*xb_col + ((j + 1) >> 1)) & 7.
  auto store_x = [&](const u32x4 (&cols)[8], int cg, int j) {
    const int mask = (4 * xb_col + ((j + 1) >> 1)) & 7;
    x_lds[x_dst + 8 * j + ((2 * cg + xb_par) ^ mask)] = cols[j];
  };
  auto stage_store = [&](const u32x4 (&stage)[9], int cg) {
    if (w_role) {
#pragma unroll
      for (int u = 0; u < 9; ++u) store_w(stage, cg, u);
    } else if (x_store) {
      u32x4 xcols[8];
      transpose8x8_b16(stage, xcols);
#pragma unroll
      for (int j = 0; j < 8; ++j) store_x(xcols, cg, j);
    }
  };
  u32x4 set0[9];
  if (stager) {
    stage_load(set0, 0);
    // zero columns (0 and W+1 .. kCols-1) of every tile row
    const int zcols = kCols - W;
    for (int i = st; i < kInRows * zcols * 8; i += kStageThreads) {
      const int c8 = i & 7;
      const int zc = (i >> 3) % zcols;
      const int r = (i >> 3) / zcols;
      const int col = zc == 0 ? 0 : W + zc;
      x_lds[(r * kCols + col) * 8 + x_slot(col, c8)] = u32x4{0, 0, 0, 0};
    }
    stage_store(set0, 0);
    stage_load(set0, 1);
  }
  __syncthreads();

  // ---- compute: wave = (filter block fb, pixel block pb) over all 7 rows (staging waves
  // get the indices of wave - 4, unused) ----
  const int fb = (wave >> 1) & 1;
  const int pb = wave & 1;
  const int f = 32 * fb + (lane & 31);
  const int hsel = lane >> 5;
  const bool live = !stager && 32 * pb < W;  // wave-uniform
  const uint32_t lds0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)&lds[0];
  // A operand: pixel w = 32pb + lane%32 (dead lanes past W read column W-1), channels
  // 16cg + 8hsel .. +7 at tap (kh, kw): LDS byte ((r + kh)*58 + w + kw)*128 + 16*slot.
  const int wpix = min(32 * pb + (lane & 31), W - 1);
  uint32_t a_off[3][4];
#pragma unroll
  for (int kw = 0; kw < 3; ++kw)
#pragma unroll
    for (int cg = 0; cg < 4; ++cg) {
      const int col = wpix + kw;
      a_off[kw][cg] = lds0 + col * 128 + 16 * x_slot(col, 2 * cg + hsel);
    }
  const uint32_t b_off = lds0 + kXBytes + (f * 2 + w_slot(f, hsel)) * 16;
  auto read_a = [&](int tap, int cg, int r) -> u32x4 {
    const int kh = tap / 3, kw = tap - 3 * (tap / 3);
    return *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)(a_off[kw][cg] + (r + kh) * kCols * 128);
  };
  auto read_b = [&](int tap, int cg) -> u32x4 {
    return *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)(b_off + (4 * tap + cg) * kF * 32);
  };
  // R accumulators (output rows row0 .. row0+R-1), channel group cg: 9 taps x R MFMAs, one
  // weight fragment shared by the R input fragments of a tap, fragments read a tap ahead.
  auto compute_cg = [&](auto rows_tag, int row0, int cg, f32x16 (&acc)[decltype(rows_tag)::value]) {
    constexpr int R = decltype(rows_tag)::value;
    if (!live) return;
    u32x4 a_cur[R], a_nxt[R], b_cur, b_nxt;
#pragma unroll
    for (int r = 0; r < R; ++r) a_cur[r] = read_a(0, cg, row0 + r);
    b_cur = read_b(0, cg);
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        acc[r] = Hf::mfma32(a_cur[r], b_cur, acc[r]);
        if (tap + 1 < 9) a_nxt[r] = read_a(tap + 1, cg, row0 + r);
        if (r == 0 && tap + 1 < 9) b_nxt = read_b(tap + 1, cg);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int r = 0; r < R; ++r) a_cur[r] = a_nxt[r];
      b_cur = b_nxt;
    }
  };
  // Output rows row0 .. row0+R-1 go out through LDS (laid out [f][row][w] like Y, filter
  // planes `stride` bytes apart) so that the HBM writes are whole 16-byte chunks of each
  // filter plane, consecutive per lane; scattered 8-byte stores from the MFMA layout write
  // far below HBM speed. Lane holds filter f, pixels 32pb + 8j + 4*hsel + 0..3 of each row.
  // stride = R*W*2 rounded so that stride/16 is odd: the 8-byte writes of 32 consecutive
  // filters then spread over all 16-byte bank groups (two lanes per group).
  float bv = 0.f;
  if constexpr (kBias == 1) bv = static_cast<const float*>(bias)[f];
  if constexpr (kBias == 2) bv = Hf::to_float(static_cast<const uint16_t*>(bias)[f]);
  char* out_lds = reinterpret_cast<char*>(x_lds);
  auto out_stride = [&](int R) { return R * W * 2 + (((R * W / 8) & 1) ? 0 : 16); };
  auto stage_out = [&](auto rows_tag, const f32x16 (&acc)[decltype(rows_tag)::value]) {
    constexpr int R = decltype(rows_tag)::value;
    if (!live) return;
    const int stride = out_stride(R);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int wo = 32 * pb + 8 * j + 4 * hsel;
        if (wo < W) {
          u32x2 packed;
          packed[0] = Hf::pack2(acc[r][4 * j] + bv, acc[r][4 * j + 1] + bv);
          packed[1] = Hf::pack2(acc[r][4 * j + 2] + bv, acc[r][4 * j + 3] + bv);
          *reinterpret_cast<u32x2*>(out_lds + f * stride + (r * W + wo) * 2) = packed;
        }
      }
  };
  // Staging wave v (4..7) writes filters 16(v-4) .. +15, two per pass (lane / 32), 16 bytes
  // per lane: a filter's rv rows are rv*W/8 <= 28 consecutive chunks of Y. Rows past H are
  // not written.
  auto flush_out = [&](int R, int row0) {
    const int ho0 = r0 + row0;
    const int rv = min(R, H - ho0);
    const int per_f = rv * W / 8;
    const int k = lane & 31;
    if (rv <= 0 || k >= per_f) return;
    const int stride = out_stride(R);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int f2 = (wave - 4) * 16 + 2 * i + (lane >> 5);
      const u32x4 v = *reinterpret_cast<const u32x4*>(out_lds + f2 * stride + 16 * k);
      st16(y + ((long long)n * kF + f2) * hw + (long long)ho0 * W + 8 * k, v);
    }
  };

  constexpr int kRowsA = 4;  // output rows 0..3: tile rows 0..5
  constexpr int kRowsB = kRows - kRowsA;
  // ---- group A, one channel group per step: the compute waves run group cg while the
  // staging waves store group cg+1 (loaded during the previous step) into LDS regions
  // group cg does not read and issue the loads of group cg+2 ----
  f32x16 acc_a[kRowsA];
#pragma unroll
  for (int r = 0; r < kRowsA; ++r)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc_a[r][i] = 0.f;
#pragma unroll
  for (int cg = 0; cg < 4; ++cg) {
    if (!stager) {
      compute_cg(Int<kRowsA>{}, 0, cg, acc_a);
    } else if (cg + 1 < 4) {
      stage_store(set0, cg + 1);
      if (cg + 2 < 4) stage_load(set0, cg + 2);
    }
    __syncthreads();
  }
  // ---- A's outputs into tile rows 0..3 (only group A read them; 64 planes of
  // out_stride(4) <= 29696 bytes = 4 tile rows for W <= 56); the staging waves write them
  // to HBM while the compute waves run group B (output rows 4..6, tile rows 4..8) ----
  stage_out(Int<kRowsA>{}, acc_a);
  __syncthreads();
  f32x16 acc_b[kRowsB];
  if (!stager) {
#pragma unroll
    for (int r = 0; r < kRowsB; ++r)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc_b[r][i] = 0.f;
#pragma unroll
    for (int cg = 0; cg < 4; ++cg) compute_cg(Int<kRowsB>{}, kRowsA, cg, acc_b);
  } else {
    flush_out(kRowsA, 0);
  }
  __syncthreads();  // A's outputs are read back and group B is done
  stage_out(Int<kRowsB>{}, acc_b);
  __syncthreads();
  if (stager) flush_out(kRowsB, kRowsA);
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
