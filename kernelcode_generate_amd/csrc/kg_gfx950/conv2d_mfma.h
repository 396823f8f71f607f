// Implicit-GEMM conv2d on gfx950 MFMA for 16-bit NCHW tensors with C = F = 64,
// a 3x3 window, stride 1, dilation 1 and padding 1 on every side (so Ho = H, Wo = W),
// W a multiple of 8 and at most 56; fp32 accumulation.
//
// GEMM view per image: Y^T[p][f] = sum_k X[p][k] W^T[k][f] with p = ho*W + wo and the
// contraction index k ordered (tap = 3*kh + kw, channel): 18 chunks of 32 = 9 taps x
// 2 channel halves. In that order 8 consecutive k of one pixel are 8 consecutive channels,
// so with the input tile stored channel-last in LDS every MFMA operand-A fragment is a
// single 16-byte read.
//
// Persistent workgroups (one per CU, 4 waves). Each workgroup first rewrites the weights
// into LDS in that k order: a thread loads the 8 channels x 9 taps of one filter (144
// contiguous bytes) with 16-byte loads and regroups them per tap with v_perm_b32. It
// then walks work items (image n, 4 output rows): the 6 input rows an item needs are
// loaded as 8-channel x 8-column blocks (16-byte loads along W), transposed in registers
// and written channel-last into a double-buffered LDS tile with one zero column on each
// side and zero rows outside the image; the next item's rows are fetched while the
// current one is computed. Wave w computes output row 4i+w for all 64 filters:
// 4 pixel blocks x 4 filter blocks of v_mfma_f32_16x16x32 per k chunk, operands read
// from LDS (XOR-swizzled 16-byte chunks). The result layout puts 4 consecutive output
// columns of one filter in each lane: one 8-byte store.
#pragma once

#include "conv2d.h"

namespace kg_gfx950 {

namespace convk {

constexpr int kThreads = 256;
constexpr int kRows = 4;               // output rows per work item (one per wave)
constexpr int kInRows = kRows + 2;     // input rows per item
constexpr int kCols = 58;              // LDS tile columns: W <= 56 plus two zero columns
constexpr int kC = 64;
constexpr int kF = 64;
constexpr int kKChunks = 18;           // 9 taps x 2 channel halves of 32
constexpr int kXVecs = kInRows * kCols * 8;   // u32x4 per input tile (8 chunks of 8 channels)
constexpr int kWVecs = kKChunks * kF * 4;     // u32x4 of reordered weights

__device__ __forceinline__ int x_swz(int ww) { return (ww & 7) ^ ((ww >> 3) & 7); }
__device__ __forceinline__ int w_swz(int f) { return (f >> 1) & 3; }

}  // namespace convk

template <typename Tag, int kBias>  // kBias: 0 none, 1 fp32, 2 16-bit
__global__ __launch_bounds__(convk::kThreads, 1) void conv2d_3x3s1p1_mfma_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, uint16_t* __restrict__ y,
    const void* __restrict__ bias, int N, int H, int W) {
  using namespace convk;
  using Hf = Half16<Tag>;
  __shared__ u32x4 w_lds[kWVecs];
  __shared__ u32x4 x_lds[2][kXVecs];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4;
  const int r16 = lane & 15;

  // Zero both input tiles once: the border columns and any columns past W stay zero.
  for (int i = tid; i < 2 * kXVecs; i += kThreads) (&x_lds[0][0])[i] = u32x4{0, 0, 0, 0};

  // Reordered weights: w_lds[(kc*64 + f)*4 + (grp ^ w_swz(f))] holds channels
  // 32*(kc&1) + 8*grp .. +7 of filter f at tap kc>>1.
#pragma unroll
  for (int rep = 0; rep < 2; ++rep) {
    const int combo = tid + kThreads * rep;  // (filter, channel octet)
    const int f = combo >> 3;
    const int co = combo & 7;
    const uint16_t* src = w + (long long)f * (kC * 9) + co * 72;
    uint32_t v[36];
#pragma unroll
    for (int i = 0; i < 9; ++i) {
      const u32x4 t = ld16(src + 8 * i);
      v[4 * i] = t[0];
      v[4 * i + 1] = t[1];
      v[4 * i + 2] = t[2];
      v[4 * i + 3] = t[3];
    }
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
      u32x4 frag;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        // channels 2q and 2q+1 of the octet at this tap: elements (2q)*9+tap, (2q+1)*9+tap
        const int e0 = (2 * q) * 9 + tap;
        const int e1 = (2 * q + 1) * 9 + tap;
        const uint32_t a = v[e0 >> 1];
        const uint32_t b = v[e1 >> 1];
        const uint32_t lo = (e0 & 1) ? (a >> 16) : (a & 0xffffu);
        const uint32_t hi = (e1 & 1) ? (b >> 16) : (b & 0xffffu);
        frag[q] = lo | (hi << 16);
      }
      const int kc = 2 * tap + (co >> 2);
      const int grp = co & 3;
      w_lds[(kc * kF + f) * 4 + (grp ^ w_swz(f))] = frag;
    }
  }

  const int row_blocks = (H + kRows - 1) / kRows;
  const int items = N * row_blocks;
  const int wblocks = W >> 3;                  // 8-column blocks per row
  const int blocks = kInRows * 8 * wblocks;    // 8x8 staging blocks per item
  constexpr int kMaxRounds = (kInRows * 8 * 7 + kThreads - 1) / kThreads;  // W <= 56

  u32x4 pre[kMaxRounds][8];

  auto load_item = [&](int item) {
    const int n = item / row_blocks;
    const int ho0 = (item % row_blocks) * kRows;
#pragma unroll
    for (int rd = 0; rd < kMaxRounds; ++rd) {
      const int b = tid + kThreads * rd;
      const int wb = b % wblocks;
      const int co = (b / wblocks) & 7;
      const int r = b / (wblocks * 8);
      const int h = ho0 - 1 + r;
      const bool live = b < blocks && h >= 0 && h < H;
      const uint16_t* src = x + (((long long)n * kC + 8 * co) * H + h) * W + 8 * wb;
#pragma unroll
      for (int e = 0; e < 8; ++e) pre[rd][e] = live ? ld16(src + (long long)e * H * W) : u32x4{0, 0, 0, 0};
    }
  };
  auto store_item = [&](int buf) {
#pragma unroll
    for (int rd = 0; rd < kMaxRounds; ++rd) {
      const int b = tid + kThreads * rd;
      if (b < blocks) {
        const int wb = b % wblocks;
        const int co = (b / wblocks) & 7;
        const int r = b / (wblocks * 8);
        u32x4 t[8];
        transpose8x8_b16(pre[rd], t);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int ww = 1 + 8 * wb + j;
          x_lds[buf][(r * kCols + ww) * 8 + (co ^ x_swz(ww))] = t[j];
        }
      }
    }
  };

  int item = blockIdx.x;
  if (item < items) load_item(item);
  __syncthreads();  // zero fill and weights complete before the first tile lands
  if (item < items) store_item(0);
  __syncthreads();

  int cur = 0;
  for (; item < items; item += gridDim.x) {
    const int next = item + gridDim.x;
    if (next < items) load_item(next);

    f32x4 acc[4][4];
#pragma unroll
    for (int pb = 0; pb < 4; ++pb)
#pragma unroll
      for (int fb = 0; fb < 4; ++fb) acc[pb][fb] = f32x4{0.f, 0.f, 0.f, 0.f};

    int wo_lane[4];
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) wo_lane[pb] = min(16 * pb + r16, W - 1);  // dead lanes read a live column

#pragma unroll 2
    for (int kc = 0; kc < kKChunks; ++kc) {
      const int tap = kc >> 1;
      const int kh = tap / 3;
      const int kw = tap - 3 * kh;
      const int chunk = 4 * (kc & 1) + g;
      u32x4 a[4], b[4];
#pragma unroll
      for (int pb = 0; pb < 4; ++pb) {
        const int ww = wo_lane[pb] + kw;
        a[pb] = x_lds[cur][((wave + kh) * kCols + ww) * 8 + (chunk ^ x_swz(ww))];
      }
#pragma unroll
      for (int fb = 0; fb < 4; ++fb) {
        const int f = 16 * fb + r16;
        b[fb] = w_lds[(kc * kF + f) * 4 + (g ^ w_swz(f))];
      }
#pragma unroll
      for (int pb = 0; pb < 4; ++pb)
#pragma unroll
        for (int fb = 0; fb < 4; ++fb) acc[pb][fb] = Hf::mfma16(a[pb], b[fb], acc[pb][fb]);
    }

    const int n = item / row_blocks;
    const int ho = (item % row_blocks) * kRows + wave;
    if (ho < H) {
#pragma unroll
      for (int fb = 0; fb < 4; ++fb) {
        const int f = 16 * fb + r16;
        float bv = 0.f;
        if constexpr (kBias == 1) bv = static_cast<const float*>(bias)[f];
        if constexpr (kBias == 2) bv = Hf::to_float(static_cast<const uint16_t*>(bias)[f]);
        uint16_t* yrow = y + (((long long)n * kF + f) * H + ho) * W;
#pragma unroll
        for (int pb = 0; pb < 4; ++pb) {
          const int wo = 16 * pb + 4 * g;
          if (wo < W) {
            const f32x4 v = acc[pb][fb];
            u32x2 packed;
            packed[0] = Hf::pack2(v[0] + bv, v[1] + bv);
            packed[1] = Hf::pack2(v[2] + bv, v[3] + bv);
            st8(yrow + wo, packed);
          }
        }
      }
    }
    if (next < items) store_item(cur ^ 1);
    __syncthreads();
    cur ^= 1;
  }
}

inline bool conv_mfma_supported(const ConvShape& s) {
  return s.c == convk::kC && s.f == convk::kF && s.kh == 3 && s.kw == 3 && s.sh == 1 && s.sw == 1 && s.dh == 1 &&
         s.dw == 1 && s.pt == 1 && s.pl == 1 && s.ho == s.h && s.wo == s.w && s.w % 8 == 0 && s.w >= 8 &&
         s.w <= convk::kCols - 2 && s.h >= 1 && s.n >= 1;
}

template <typename Tag>
hipError_t launch_conv2d_mfma(const uint16_t* x, const uint16_t* w, uint16_t* y, const void* bias, int bias_kind,
                              const ConvShape& s, hipStream_t stream) {
  int cus = 256;
  int dev = 0;
  if (hipGetDevice(&dev) == hipSuccess) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) cus = v;
  }
  const long long items = (long long)s.n * ((s.h + convk::kRows - 1) / convk::kRows);
  const int grid = (int)(items < cus ? items : cus);
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
