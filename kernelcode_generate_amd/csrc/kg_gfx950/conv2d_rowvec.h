// Implicit-GEMM conv2d on gfx950 MFMA for NCHW convs of stride S = 1 or 2 (both directions)
// and dilation 1 whose input and output rows split into whole pieces of G pixels (W % G == 0
// and Wo % G == 0; 16-bit: G = 8 or 4, fp32: G = 4), with a KW = 3 window and left pad 1 or
// a KW = 1 window and left pad 0 (any C, F, KH, top/bottom pads; C KH KW a multiple of 8,
// fp32: of 4). fp32 accumulation. The 16-bit kernel is described first; the fp32 one
// (conv2d_rowvec_f32_kernel) differs in its MFMA and operand reads.
//
// GEMM view as in conv2d_igemm.h: Y[n][f][p] = sum_k W[f][k] Xcol[k][(n, p)] with k =
// (c, kh, kw) in the weight's own order. What differs is how Xcol reaches LDS. The k-row
// (c, kh, kw) of G consecutive output pixels wo0 .. of one row is the input pixels
// S wo0 - pl + kw + S u (u < G) of input row S ho - pt + kh: so a thread that owns a (c, kh)
// run and a G-pixel output piece loads the aligned G-pixel input pieces of that row that
// cover all KW windows (three for 3x3, two or one for 1x1), builds the KW windows in
// registers (stride 1: v_alignbyte; stride 2: v_perm of every other 16-bit element; all
// offsets compile-time) and writes them as KW k-rows. Pieces outside the
// row (the left/right padding) and rows outside the image load nothing and hold zeros; W %
// G == 0 keeps every piece wholly inside or wholly outside. One load serves KW k-rows, so a
// 32-deep K step takes one vector load per thread where the per-element gather took 16.
//
// Xcol sits in LDS k-major, [k-row][128 pixels] (256 bytes a row, 16-byte chunk c of row r
// at c ^ 4(r & 3)), and the MFMA operand (8 consecutive k of one pixel) is read with two
// ds_read_b64_tr_b16: within each 16-lane group, lane j addresses 4 consecutive pixels of
// k-row j/4 and lane i receives k-rows 0..3 of pixel i; under the chunk swizzle the 32 lanes
// served together hit 16 distinct chunks of one 256-byte bank cycle. Weights stay [f][k] rows
// of one slice (16 KW values, 16-byte chunk loads), padded to an odd number of 16-byte
// chunks per row so 16 consecutive rows at one chunk hit distinct banks.
//
// A workgroup (4 waves, 2 x 2) computes BM (64 or 128) filters x 128 output pixels and walks
// K in slices of 16 KW k-rows (16 runs (c, kh) x KW taps): KW MFMA steps of 16 per slice,
// two LDS stages (or the 3 or 4 of a deeper ring the lowering asks for) and two register
// sets, so a slice's loads are issued two slices before its
// MFMAs; register use is bounded for two waves per SIMD (unbounded, the 128-filter
// instantiations took one wave per SIMD and ran 7-12 % slower on 3x3 shapes). Each lane ends with 4 consecutive output pixels of one filter (Wo % 4 == 0 keeps
// them in one row of one image) and stores them as one 8-byte piece.
#pragma once

#include <type_traits>

#include "common.h"
#include "conv2d.h"
#include "conv2d_igemm.h"
#include "lds_dma.h"

namespace kg_gfx950 {

namespace convr {
constexpr int kBN = 128;      // output pixels per tile
constexpr int kThreads = 256;  // 4 waves, 2 x 2
constexpr int kRuns = 16;      // (c, kh) runs per K slice

struct Params {
  int n, c, h, w, f, kh, ho, wo, pt;
  int K;     // C KH KW
  int runs;  // C KH
  int P;     // Ho Wo
  int NP;    // N Ho Wo
  int bias_kind;  // 0 none, 1 fp32, 2 same 16-bit type
  int kcs;        // split-K: slices per workgroup row (blockIdx.y); 0 = the whole K range
  FastDiv div_kh, div_p, div_wo;
};

// byte offset of 16-byte chunk c of k-row r in an Xcol stage
__host__ __device__ constexpr int xoff(int r, int c) { return r * 256 + ((c ^ (4 * (r & 3))) * 16); }

template <int KW, int PL, int G, int S>
struct Geometry {
  static_assert(G == 8 || G == 4, "pieces of 8 or 4 pixels");
  static_assert(PL >= 0 && PL < G, "left pad within one piece");
  static_assert(S == 1 || S == 2, "stride 1 or 2");
  static constexpr int kKR = 16 * KW;                    // k-rows per slice
  static constexpr int kWPitch = 32 * KW + 16;           // weight row bytes in LDS: an odd number of chunks
  static constexpr int kM0 = (G - PL) % G;               // first needed element within the first piece
  static constexpr int kLast = kM0 + KW - 1 + S * (G - 1);  // last needed element
  static constexpr int kPieces = kLast / G + 1;          // aligned pieces covering all KW windows
  static constexpr int kDw = G / 2;                      // dwords per piece
  static constexpr int kGroups = kBN / G;                // pieces per k-row of a tile
  static constexpr int kItems = kRuns * kGroups / kThreads;  // (run, piece) items per thread and slice
};

template <int BM, int KW, int PL, int G, int S>
constexpr int rowvec_stage_bytes() {
  return Geometry<KW, PL, G, S>::kKR * 256 + BM * Geometry<KW, PL, G, S>::kWPitch;
}
}  // namespace convr

template <typename Tag, int kMI, int KW, int PL, int G, int S, int kRing>
__global__ __launch_bounds__(convr::kThreads, 2) void conv2d_rowvec_kernel(const uint16_t* __restrict__ x,
                                                                        const uint16_t* __restrict__ wt,
                                                                        uint16_t* __restrict__ y,
                                                                        const void* __restrict__ bias,
                                                                        convr::Params s,
                                                                        float* __restrict__ partial) {
  using namespace convr;
  using Geo = Geometry<KW, PL, G, S>;
  using Hf = Half16<Tag>;
  constexpr int BM = 64 * kMI;
  constexpr int KR = Geo::kKR;
  constexpr int kXBytes = KR * 256;
  constexpr int kStage = rowvec_stage_bytes<BM, KW, PL, G, S>();
  constexpr int kWChunks = BM * 2 * KW;  // 16-byte weight chunks per slice
  constexpr int kWPerThread = (kWChunks + kThreads - 1) / kThreads;
  using Piece = typename std::conditional<G == 8, u32x4, u32x2>::type;
  static_assert(kRing >= 2 && kRing <= 4 && kRing * kStage <= 160 * 1024, "LDS ring");
  __shared__ __attribute__((aligned(1024))) char lds[kRing * kStage];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_m = (s.f + BM - 1) / BM;
  const int logical = xcd_logical_id(blockIdx.x, gridDim.x);
  const int m0 = (logical % tiles_m) * BM;  // the filter tiles of one pixel tile are adjacent
  const int n0 = (logical / tiles_m) * kBN;

  // ---- this thread's output piece: pixels j0 .. j0+G-1 of one output row ----
  const int g = tid % Geo::kGroups;
  const int q0 = tid / Geo::kGroups;  // first run; item i takes run q0 + i * (16 / kItems)
  const int j0 = n0 + G * g;
  const bool piece_ok = j0 < s.NP;
  const uint32_t jn = fdiv(piece_ok ? j0 : 0, s.div_p);
  const uint32_t jp = (piece_ok ? j0 : 0) - jn * s.P;
  const uint32_t jho = fdiv(jp, s.div_wo);
  const int wo0 = (int)(jp - jho * s.wo);
  const int hbase = S * (int)jho - s.pt;               // input row of kh = 0
  const int pc0 = (S * wo0 - PL + G) / G - 1;          // first aligned input piece (may be -1)
  const int wpieces = s.w / G;
  const long long hw = (long long)s.h * s.w;
  const uint16_t* xn = x + (long long)jn * s.c * hw;

  // two register sets: slice s is loaded into set s & 1 two slices before its MFMAs
  Piece raw[2][Geo::kItems][Geo::kPieces];
  u32x4 rw[2][kWPerThread];
  auto load_regs = [&](int kt, auto set_tag) {
    constexpr int SET = decltype(set_tag)::value;
#pragma unroll
    for (int it = 0; it < Geo::kItems; ++it) {
      const int run = kt * kRuns + q0 + it * (kRuns / Geo::kItems);
      const uint32_t c = fdiv((uint32_t)run, s.div_kh);
      const int hi = hbase + (run - (int)c * s.kh);
      const bool row_ok = piece_ok && run < s.runs && (unsigned)hi < (unsigned)s.h;
      const uint16_t* src = xn + (long long)c * hw + (long long)hi * s.w + G * pc0;
#pragma unroll
      for (int p = 0; p < Geo::kPieces; ++p) {
        const bool ok = row_ok && (unsigned)(pc0 + p) < (unsigned)wpieces;
        raw[SET][it][p] = ok ? *reinterpret_cast<const Piece*>(src + G * p) : Piece{};
      }
    }
    const int k0 = kt * KR;
#pragma unroll
    for (int i = 0; i < kWPerThread; ++i) {
      const int ci = tid + kThreads * i;
      const int row = ci / (2 * KW), kc = ci - row * (2 * KW);
      const int f = m0 + row, k = k0 + 8 * kc;
      rw[SET][i] = (ci < kWChunks && f < s.f && k < s.K) ? ld16(wt + (long long)f * s.K + k) : u32x4{0, 0, 0, 0};
    }
  };
  // window kw of item `it`: elements kM0 + kw + S u (u < G) of its concatenated pieces
  auto window = [&](int it, auto set_tag, auto kw_tag) -> Piece {
    constexpr int SET = decltype(set_tag)::value;
    constexpr int st = Geo::kM0 + decltype(kw_tag)::value;
    constexpr int kDw = Geo::kDw;
    auto dw = [&](int i) -> uint32_t { return raw[SET][it][i / kDw][i % kDw]; };
    Piece out;
#pragma unroll
    for (int d = 0; d < kDw; ++d) {
      const int e = st + 2 * S * d;  // element of output pixel 2d; pixel 2d+1 is element e + S
      if constexpr (S == 1) {
        if ((st & 1) == 0) out[d] = dw(e >> 1);
        else out[d] = __builtin_amdgcn_alignbyte(dw((e >> 1) + 1), dw(e >> 1), 2);
      } else {
        if ((st & 1) == 0) out[d] = lo_halves(dw(e >> 1), dw((e >> 1) + 1));
        else out[d] = hi_halves(dw(e >> 1), dw((e >> 1) + 1));
      }
    }
    return out;
  };
  auto store_lds = [&](int buf, auto set_tag) {
    char* st = lds + buf * kStage;
#pragma unroll
    for (int it = 0; it < Geo::kItems; ++it) {
      const int q = q0 + it * (kRuns / Geo::kItems);
      auto put = [&](auto kw_tag) {
        constexpr int kw = decltype(kw_tag)::value;
        const int r = KW * q + kw;
        const Piece v = window(it, set_tag, kw_tag);
        if constexpr (G == 8) {
          *reinterpret_cast<u32x4*>(st + xoff(r, g)) = v;
        } else {
          *reinterpret_cast<u32x2*>(st + xoff(r, g >> 1) + 8 * (g & 1)) = v;
        }
      };
      put(Int<0>{});
      if constexpr (KW > 1) put(Int<1>{});
      if constexpr (KW > 2) put(Int<2>{});
    }
#pragma unroll
    for (int i = 0; i < kWPerThread; ++i) {
      const int ci = tid + kThreads * i;
      if (ci < kWChunks) {
        const int row = ci / (2 * KW), kc = ci - row * (2 * KW);
        *reinterpret_cast<u32x4*>(st + kXBytes + row * Geo::kWPitch + 16 * kc) = rw[decltype(set_tag)::value][i];
      }
    }
  };

  // ---- fragment addresses (bytes within a stage) ----
  const int frag = lane & 31, h = lane >> 5;
  const int lg = lane >> 4, j16 = lane & 15;
  const int b_kofs = 8 * (lg >> 1) + (j16 >> 2);  // k-row of the first transposed read
  int x_rd[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int px = wn * 64 + 32 * b + 16 * (lg & 1) + 4 * (j16 & 3);
    x_rd[b] = xoff(b_kofs, px >> 3) + 2 * (px & 7);  // +1024: k-rows +4; +4096: next K step
  }
  int w_rd[kMI];
#pragma unroll
  for (int i = 0; i < kMI; ++i) w_rd[i] = kXBytes + (wm * (BM / 2) + 32 * i + frag) * Geo::kWPitch + 16 * h;

  f32x16 acc[kMI][2];
#pragma unroll
  for (int i = 0; i < kMI; ++i)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][b][e] = 0.f;

  int nk = (s.runs + kRuns - 1) / kRuns;
  auto compute = [&](int buf) {
    const char* st = lds + buf * kStage;
    const uint32_t sbase = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)st;
#pragma unroll
    for (int ks = 0; ks < KW; ++ks) {
      u32x4 af[kMI], bf[2];
#pragma unroll
      for (int i = 0; i < kMI; ++i)
        af[i] = *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)(sbase + w_rd[i] + 32 * ks);
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s16x4*)(uintptr_t)(sbase + x_rd[b] + 1024 * t + 4096 * ks));
          const u32x2 w2 = __builtin_bit_cast(u32x2, v);
          bf[b][2 * t] = w2[0];
          bf[b][2 * t + 1] = w2[1];
        }
#pragma unroll
      for (int i = 0; i < kMI; ++i)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[i][b] = Hf::mfma32(bf[b], af[i], acc[i][b]);
    }
  };
  // slice kt: its MFMAs read LDS stage kt % kRing; slice kt + 1 goes from register set
  // (kt + 1) & 1 to stage (kt + 1) % kRing; slice kt + 2 is loaded into set kt & 1 meanwhile.
  // The stage a slice is stored to was last read kRing - 1 steps earlier, before that
  // step's barrier.
  // split-K: this workgroup row's slices kt0 .. kt0 + nk - 1 (kt below counts from kt0)
  int kt0 = 0;
  if (s.kcs > 0) {
    kt0 = blockIdx.y * s.kcs;
    nk = min(nk - kt0, s.kcs);
    partial += (long long)blockIdx.y * s.NP * s.f;
  }
  auto step = [&](int kt, auto par_tag) {
    constexpr int par = decltype(par_tag)::value;
    if (kt + 2 < nk) load_regs(kt0 + kt + 2, Int<par>{});
    compute(kRing == 2 ? par : (int)((unsigned)kt % kRing));
    if (kt + 1 < nk) store_lds(kRing == 2 ? (par ^ 1) : (int)((unsigned)(kt + 1) % kRing), Int<par ^ 1>{});
    __syncthreads();
  };
  load_regs(kt0, Int<0>{});
  store_lds(0, Int<0>{});
  if (nk > 1) load_regs(kt0 + 1, Int<1>{});
  __syncthreads();
  for (int kt = 0; kt < nk; kt += 2) {
    step(kt, Int<0>{});
    if (kt + 1 < nk) step(kt + 1, Int<1>{});
  }

  // ---- epilogue: lane holds Y[f][j .. j+3], f = tile row wm*BM/2 + 32 i + lane % 32,
  // j = tile pixel wn*64 + 32 b + 8 q + 4 (lane / 32); P % 4 == 0 keeps j .. j+3 in one image ----
#pragma unroll
  for (int i = 0; i < kMI; ++i) {
    const int f = m0 + wm * (BM / 2) + 32 * i + frag;
    if (f >= s.f) continue;
    float bv = 0.f;
    if (s.bias_kind == 1) bv = static_cast<const float*>(bias)[f];
    if (s.bias_kind == 2) bv = Hf::to_float(static_cast<const uint16_t*>(bias)[f]);
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int j = n0 + wn * 64 + 32 * b + 8 * q + 4 * h;
        if (j >= s.NP) continue;
        const uint32_t n = fdiv(j, s.div_p);
        const uint32_t p = j - n * s.P;
        if (s.kcs > 0) {  // fp32 partial sums in Y's layout, no bias
          *reinterpret_cast<f32x4*>(partial + ((long long)n * s.f + f) * s.P + p) =
              f32x4{acc[i][b][4 * q], acc[i][b][4 * q + 1], acc[i][b][4 * q + 2], acc[i][b][4 * q + 3]};
          continue;
        }
        u32x2 packed;
        packed[0] = Hf::pack2(acc[i][b][4 * q] + bv, acc[i][b][4 * q + 1] + bv);
        packed[1] = Hf::pack2(acc[i][b][4 * q + 2] + bv, acc[i][b][4 * q + 3] + bv);
        st8(y + ((long long)n * s.f + f) * s.P + p, packed);
      }
  }
}

// fp32 form of the same scheme, on v_mfma_f32_32x32x2_f32 (one k per lane and operand):
// 4-pixel (16-byte) pieces, K slices of 8 (c, kh) runs x KW taps (8 KW k-rows). Xcol rows
// are 128 fp32 pixels padded to 544 bytes, so the two k-rows one operand read covers (4
// apart, see below) fall 32 banks apart, and the MFMA operand is one ds_read_b32 per lane.
// Weights are [f][8 KW k] rows read as 16-byte chunks of 4 k: lane half h of MFMA kk of
// 8-k group g takes k = 8g + 4h + kk from its weight chunk, and the Xcol read takes the
// same k-row, so both operands follow one (permuted) contraction order.
namespace convr {
constexpr int kRunsF32 = 8;        // (c, kh) runs per fp32 K slice
constexpr int kXPitchF32 = 544;    // bytes per fp32 Xcol row: 512 + 32
template <int KW, int PL, int S>
struct GeometryF32 {
  static constexpr int G = 4;
  static_assert(PL >= 0 && PL < G, "left pad within one piece");
  static_assert(S == 1 || S == 2, "stride 1 or 2");
  static constexpr int kKR = kRunsF32 * KW;                 // k-rows per slice
  static constexpr int kWPitch = 4 * kKR + 16;              // an odd number of 16-byte chunks
  static constexpr int kM0 = (G - PL) % G;
  static constexpr int kLast = kM0 + KW - 1 + S * (G - 1);
  static constexpr int kPieces = kLast / G + 1;
  static constexpr int kGroups = kBN / G;                   // 32 pieces per k-row of a tile
  static_assert(kRunsF32 * kGroups == kThreads, "one (run, piece) item per thread and slice");
};
template <int BM, int KW, int PL, int S>
constexpr int rowvec_f32_stage_bytes() {
  return GeometryF32<KW, PL, S>::kKR * kXPitchF32 + BM * GeometryF32<KW, PL, S>::kWPitch;
}
}  // namespace convr

template <int kMI, int KW, int PL, int S, int kRing>
__global__ __launch_bounds__(convr::kThreads, 2) void conv2d_rowvec_f32_kernel(const float* __restrict__ x,
                                                                              const float* __restrict__ wt,
                                                                              float* __restrict__ y,
                                                                              const float* __restrict__ bias,
                                                                              convr::Params s,
                                                                              float* __restrict__ partial) {
  using namespace convr;
  using Geo = GeometryF32<KW, PL, S>;
  constexpr int G = Geo::G;
  constexpr int BM = 64 * kMI;
  constexpr int KR = Geo::kKR;
  constexpr int kXBytes = KR * kXPitchF32;
  constexpr int kStage = rowvec_f32_stage_bytes<BM, KW, PL, S>();
  constexpr int kWChunks = BM * (KR / 4);  // 16-byte weight chunks per slice
  constexpr int kWPerThread = (kWChunks + kThreads - 1) / kThreads;
  static_assert(kRing >= 2 && kRing <= 4 && kRing * kStage <= 160 * 1024, "LDS ring");
  __shared__ __attribute__((aligned(1024))) char lds[kRing * kStage];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_m = (s.f + BM - 1) / BM;
  const int logical = xcd_logical_id(blockIdx.x, gridDim.x);
  const int m0 = (logical % tiles_m) * BM;
  const int n0 = (logical / tiles_m) * kBN;

  const int g = tid % Geo::kGroups;
  const int q = tid / Geo::kGroups;  // this thread's run within a slice
  const int j0 = n0 + G * g;
  const bool piece_ok = j0 < s.NP;
  const uint32_t jn = fdiv(piece_ok ? j0 : 0, s.div_p);
  const uint32_t jp = (piece_ok ? j0 : 0) - jn * s.P;
  const uint32_t jho = fdiv(jp, s.div_wo);
  const int wo0 = (int)(jp - jho * s.wo);
  const int hbase = S * (int)jho - s.pt;
  const int pc0 = (S * wo0 - PL + G) / G - 1;
  const int wpieces = s.w / G;
  const long long hw = (long long)s.h * s.w;
  const float* xn = x + (long long)jn * s.c * hw;

  u32x4 raw[2][Geo::kPieces];
  u32x4 rw[2][kWPerThread];
  auto load_regs = [&](int kt, auto set_tag) {
    constexpr int SET = decltype(set_tag)::value;
    const int run = kt * kRunsF32 + q;
    const uint32_t c = fdiv((uint32_t)run, s.div_kh);
    const int hi = hbase + (run - (int)c * s.kh);
    const bool row_ok = piece_ok && run < s.runs && (unsigned)hi < (unsigned)s.h;
    const float* src = xn + (long long)c * hw + (long long)hi * s.w + G * pc0;
#pragma unroll
    for (int p = 0; p < Geo::kPieces; ++p) {
      const bool ok = row_ok && (unsigned)(pc0 + p) < (unsigned)wpieces;
      raw[SET][p] = ok ? ld16(src + G * p) : u32x4{0, 0, 0, 0};
    }
    const int k0 = kt * KR;
#pragma unroll
    for (int i = 0; i < kWPerThread; ++i) {
      const int ci = tid + kThreads * i;
      const int row = ci / (KR / 4), kc = ci - row * (KR / 4);
      const int f = m0 + row, k = k0 + 4 * kc;
      rw[SET][i] = (ci < kWChunks && f < s.f && k < s.K) ? ld16(wt + (long long)f * s.K + k) : u32x4{0, 0, 0, 0};
    }
  };
  auto store_lds = [&](int buf, auto set_tag) {
    constexpr int SET = decltype(set_tag)::value;
    char* st = lds + buf * kStage;
    auto put = [&](auto kw_tag) {
      constexpr int kw = decltype(kw_tag)::value;
      constexpr int e0 = Geo::kM0 + kw;  // element of output pixel u: e0 + S u
      u32x4 v;
#pragma unroll
      for (int u = 0; u < G; ++u) v[u] = raw[SET][(e0 + S * u) / G][(e0 + S * u) % G];
      *reinterpret_cast<u32x4*>(st + (KW * q + kw) * kXPitchF32 + 16 * g) = v;
    };
    put(Int<0>{});
    if constexpr (KW > 1) put(Int<1>{});
    if constexpr (KW > 2) put(Int<2>{});
#pragma unroll
    for (int i = 0; i < kWPerThread; ++i) {
      const int ci = tid + kThreads * i;
      if (ci < kWChunks) {
        const int row = ci / (KR / 4), kc = ci - row * (KR / 4);
        *reinterpret_cast<u32x4*>(st + kXBytes + row * Geo::kWPitch + 16 * kc) = rw[SET][i];
      }
    }
  };

  const int frag = lane & 31, h = lane >> 5;
  int x_rd[2];  // Xcol k-row 4h (+ 8 g + kk) at pixel wn*64 + 32 b + lane % 32
#pragma unroll
  for (int b = 0; b < 2; ++b) x_rd[b] = 4 * h * kXPitchF32 + 4 * (wn * 64 + 32 * b + frag);
  int w_rd[kMI];  // weight chunk 2g + h of filter row wm*BM/2 + 32 i + lane % 32
#pragma unroll
  for (int i = 0; i < kMI; ++i) w_rd[i] = kXBytes + (wm * (BM / 2) + 32 * i + frag) * Geo::kWPitch + 16 * h;

  f32x16 acc[kMI][2];
#pragma unroll
  for (int i = 0; i < kMI; ++i)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][b][e] = 0.f;

  int nk = (s.runs + kRunsF32 - 1) / kRunsF32;
  auto compute = [&](int buf) {
    const uint32_t sbase = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)(lds + buf * kStage);
#pragma unroll
    for (int g8 = 0; g8 < KR / 8; ++g8) {
      f32x4 af[kMI];
#pragma unroll
      for (int i = 0; i < kMI; ++i)
        af[i] = *(const __attribute__((address_space(3))) f32x4*)(uintptr_t)(sbase + w_rd[i] + 32 * g8);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        float bf[2];
#pragma unroll
        for (int b = 0; b < 2; ++b)
          bf[b] = *(const __attribute__((address_space(3))) float*)(uintptr_t)(sbase + x_rd[b] +
                                                                               (8 * g8 + kk) * kXPitchF32);
#pragma unroll
        for (int i = 0; i < kMI; ++i)
#pragma unroll
          for (int b = 0; b < 2; ++b)
            acc[i][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(bf[b], af[i][kk], acc[i][b], 0, 0, 0);
      }
    }
  };
  // split-K: this workgroup row's slices kt0 .. kt0 + nk - 1 (kt below counts from kt0)
  int kt0 = 0;
  if (s.kcs > 0) {
    kt0 = blockIdx.y * s.kcs;
    nk = min(nk - kt0, s.kcs);
    partial += (long long)blockIdx.y * s.NP * s.f;
  }
  auto step = [&](int kt, auto par_tag) {  // LDS stages as in the 16-bit kernel
    constexpr int par = decltype(par_tag)::value;
    if (kt + 2 < nk) load_regs(kt0 + kt + 2, Int<par>{});
    compute(kRing == 2 ? par : (int)((unsigned)kt % kRing));
    if (kt + 1 < nk) store_lds(kRing == 2 ? (par ^ 1) : (int)((unsigned)(kt + 1) % kRing), Int<par ^ 1>{});
    __syncthreads();
  };
  load_regs(kt0, Int<0>{});
  store_lds(0, Int<0>{});
  if (nk > 1) load_regs(kt0 + 1, Int<1>{});
  __syncthreads();
  for (int kt = 0; kt < nk; kt += 2) {
    step(kt, Int<0>{});
    if (kt + 1 < nk) step(kt + 1, Int<1>{});
  }

  // ---- epilogue: lane holds Y[f][j .. j+3] as in the 16-bit kernel; one 16-byte store ----
#pragma unroll
  for (int i = 0; i < kMI; ++i) {
    const int f = m0 + wm * (BM / 2) + 32 * i + frag;
    if (f >= s.f) continue;
    const float bv = s.bias_kind != 0 ? bias[f] : 0.f;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int j = n0 + wn * 64 + 32 * b + 8 * qq + 4 * h;
        if (j >= s.NP) continue;
        const uint32_t n = fdiv(j, s.div_p);
        const uint32_t p = j - n * s.P;
        // split-K: fp32 partial sums in Y's layout, no bias
        const float bj = s.kcs > 0 ? 0.f : bv;
        float* dst = s.kcs > 0 ? partial : y;
        *reinterpret_cast<f32x4*>(dst + ((long long)n * s.f + f) * s.P + p) =
            f32x4{acc[i][b][4 * qq] + bj, acc[i][b][4 * qq + 1] + bj, acc[i][b][4 * qq + 2] + bj,
                  acc[i][b][4 * qq + 3] + bj};
      }
  }
}

// Pieces of G pixels: 8 when W and Wo are multiples of 8, else 4 when they are multiples of
// 4, else 0 (the row-vector path does not apply).
inline int conv_rowvec_piece(const ConvShape& s) {
  if (s.w % 8 == 0 && s.wo % 8 == 0) return 8;
  if (s.w % 4 == 0 && s.wo % 4 == 0) return 4;
  return 0;
}

// f32: fp32 operands (4-pixel pieces only, K % 4 == 0); else 16-bit (K % 8 == 0).
inline bool conv_rowvec_supported(const ConvShape& s, bool f32 = false) {
  const long long K = (long long)s.c * s.kh * s.kw;
  const bool window = (s.kw == 3 && s.pl == 1) || (s.kw == 1 && s.pl == 0);
  const bool pieces = f32 ? (s.w % 4 == 0 && s.wo % 4 == 0 && K % 4 == 0) : (conv_rowvec_piece(s) != 0 && K % 8 == 0);
  return window && pieces && (s.sh == 1 || s.sh == 2) && s.sw == s.sh && s.dh == 1 && s.dw == 1 && s.kh >= 1 &&
         s.ho >= 1 && s.wo >= 1 && K < (1ll << 30) && (long long)s.n * s.ho * s.wo < (1ll << 31) &&
         (long long)s.c * s.kh < (1ll << 30) && (long long)s.n * s.c * s.h * s.w < (1ll << 40);
}

// BM = 128 filters per tile when F > 64 and such tiles still give every CU of the MI355X
// (256) two workgroups; else 64.
inline int conv_rowvec_mi(const ConvShape& s) {
  const long long cols = ((long long)s.n * s.ho * s.wo + convr::kBN - 1) / convr::kBN;
  return s.f > 64 && ((s.f + 127) / 128) * cols >= 512 ? 2 : 1;
}

// MFMA instructions of one launch: per tile and slice, 4 waves x MI x 2 blocks x (16-bit:
// KW steps of 32x32x16; fp32: 4 KW MFMAs of 32x32x2).
inline long long conv_rowvec_mfma(const ConvShape& s, bool f32 = false) {
  const long long mi = conv_rowvec_mi(s);
  const long long tiles = ((s.f + 64 * mi - 1) / (64 * mi)) * (((long long)s.n * s.ho * s.wo + convr::kBN - 1) / convr::kBN);
  const long long runs = f32 ? convr::kRunsF32 : convr::kRuns;
  const long long slices = ((long long)s.c * s.kh + runs - 1) / runs;
  return tiles * slices * 4 * mi * 2 * s.kw * (f32 ? 4 : 1);
}

// Split-K for grids of fewer than two workgroups per CU: slices (16 or, fp32, 8 (c, kh) runs)
// cut into chunks of at least 2, the split count chosen by a time model fitted to measured
// row-piece convs of grids under 512 workgroups: a slice takes 280 + 135 KW ns (fp32
// 515 + 250 KW) on a CU of its own and twice that per workgroup on a CU shared by two (the
// grid runs in ceil(workgroups / 256) rounds), the fp32 partials' write and read move 8
// bytes per output element and split at about 4 bytes/ns, and the reduction launch adds
// 4 us. Small outputs gain most (N=1 28x28 C=F=128 3x3: 8 splits, 20 -> 10 us); large ones
// keep one pass (N=32 of that: the partials would cost 19 us to save 8).
// Returns the split count (1: none) and the slices per chunk; the fp32 partials stay
// under max_partial_bytes.
inline int conv_rowvec_splits(const ConvShape& s, bool f32, long long max_partial_bytes, int* kcs) {
  const long long runs = f32 ? convr::kRunsF32 : convr::kRuns;
  const long long nk = ((long long)s.c * s.kh + runs - 1) / runs;
  const long long np = (long long)s.n * s.ho * s.wo;
  const long long nfp = np * s.f;
  const int mi = conv_rowvec_mi(s);
  const long long grid = ((s.f + 64 * mi - 1) / (64 * mi)) * ((np + convr::kBN - 1) / convr::kBN);
  *kcs = 0;
  if (grid >= 512 || nk < 4 || nfp >= (1ll << 31)) return 1;
  const long long smax =
      std::min(std::min((512 + grid - 1) / grid, nk / 2), max_partial_bytes / (nfp * 4));
  const long long slice_ns = f32 ? 515 + 250 * s.kw : 280 + 135 * s.kw;
  long long best = 1, best_ns = (grid + 255) / 256 * nk * slice_ns;
  for (long long sp = 2; sp <= smax; ++sp) {
    const long long t = (grid * sp + 255) / 256 * ((nk + sp - 1) / sp) * slice_ns + sp * nfp * 8 / 4000 + 4000;
    if (t < best_ns) { best = sp; best_ns = t; }
  }
  if (best < 2) return 1;
  const long long c = (nk + best - 1) / best;
  *kcs = (int)c;
  return (int)((nk + c - 1) / c);
}

inline convr::Params conv_rowvec_params(const ConvShape& s, int bias_kind) {
  convr::Params p;
  p.n = s.n; p.c = s.c; p.h = s.h; p.w = s.w; p.f = s.f; p.kh = s.kh; p.ho = s.ho; p.wo = s.wo; p.pt = s.pt;
  p.K = s.c * s.kh * s.kw;
  p.runs = s.c * s.kh;
  p.P = s.ho * s.wo;
  p.NP = s.n * p.P;
  p.bias_kind = bias_kind;
  p.kcs = 0;
  p.div_kh = make_fast_div((uint32_t)s.kh);
  p.div_p = make_fast_div((uint32_t)p.P);
  p.div_wo = make_fast_div((uint32_t)s.wo);
  return p;
}

// fp32 operands; a bias (kind 1 or 2) is fp32 either way.
// splits > 1: split-K into the fp32 workspace `partial` (splits x N F Ho Wo floats) with kcs
// slices per chunk, then the reduction into y (conv_splitk_reduce_kernel).
template <int kRing>
hipError_t launch_conv2d_rowvec_f32_ring(const float* x, const float* w, float* y, const float* bias, int bias_kind,
                                         const ConvShape& s, hipStream_t stream, float* partial, int splits, int kcs) {
  convr::Params p = conv_rowvec_params(s, bias_kind);
  if (splits > 1) p.kcs = kcs;
  else splits = 1;
  const int mi = conv_rowvec_mi(s);
  const int grid = ((s.f + 64 * mi - 1) / (64 * mi)) * ((p.NP + convr::kBN - 1) / convr::kBN);
#define KG_CONV_RVF(MI, KW_, PL_, S_) \
  hipLaunchKernelGGL((conv2d_rowvec_f32_kernel<MI, KW_, PL_, S_, kRing>), dim3(grid, splits), dim3(convr::kThreads), 0, stream, x, w, \
                     y, bias, p, partial)
#define KG_CONV_RVF_MI(KW_, PL_, S_) \
  if (mi == 2) { KG_CONV_RVF(2, KW_, PL_, S_); } else { KG_CONV_RVF(1, KW_, PL_, S_); }
  if (s.kw == 3) {
    if (s.sh == 1) { KG_CONV_RVF_MI(3, 1, 1) } else { KG_CONV_RVF_MI(3, 1, 2) }
  } else {
    if (s.sh == 1) { KG_CONV_RVF_MI(1, 0, 1) } else { KG_CONV_RVF_MI(1, 0, 2) }
  }
#undef KG_CONV_RVF_MI
#undef KG_CONV_RVF
  if (splits > 1) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int nfp = p.NP * s.f;
    const int rgrid = (nfp + kConvReduceThreads - 1) / kConvReduceThreads;
    if (bias_kind == 0)
      hipLaunchKernelGGL((conv_splitk_reduce_kernel<F32Tag, 0>), dim3(rgrid), dim3(kConvReduceThreads), 0, stream,
                         partial, splits, y, bias, nfp, p.div_p, s.f);
    else
      hipLaunchKernelGGL((conv_splitk_reduce_kernel<F32Tag, 1>), dim3(rgrid), dim3(kConvReduceThreads), 0, stream,
                         partial, splits, y, bias, nfp, p.div_p, s.f);
  }
  return hipGetLastError();
}

template <typename Tag, int kRing>
hipError_t launch_conv2d_rowvec_ring(const uint16_t* x, const uint16_t* w, uint16_t* y, const void* bias, int bias_kind,
                                     const ConvShape& s, hipStream_t stream, float* partial, int splits, int kcs) {
  convr::Params p = conv_rowvec_params(s, bias_kind);
  if (splits > 1) p.kcs = kcs;
  else splits = 1;
  const int mi = conv_rowvec_mi(s);
  const int piece = conv_rowvec_piece(s);
  const int grid = ((s.f + 64 * mi - 1) / (64 * mi)) * ((p.NP + convr::kBN - 1) / convr::kBN);
#define KG_CONV_RV(MI, KW_, PL_, G_, S_)                                                                     \
  hipLaunchKernelGGL((conv2d_rowvec_kernel<Tag, MI, KW_, PL_, G_, S_, kRing>), dim3(grid, splits), dim3(convr::kThreads), 0, \
                     stream, x, w, y, bias, p, partial)
#define KG_CONV_RV_MI(KW_, PL_, G_, S_) \
  if (mi == 2) KG_CONV_RV(2, KW_, PL_, G_, S_); \
  else KG_CONV_RV(1, KW_, PL_, G_, S_)
#define KG_CONV_RV_G(KW_, PL_, S_) \
  if (piece == 8) { KG_CONV_RV_MI(KW_, PL_, 8, S_); } else { KG_CONV_RV_MI(KW_, PL_, 4, S_); }
  if (s.kw == 3) {
    if (s.sh == 1) { KG_CONV_RV_G(3, 1, 1) } else { KG_CONV_RV_G(3, 1, 2) }
  } else {
    if (s.sh == 1) { KG_CONV_RV_G(1, 0, 1) } else { KG_CONV_RV_G(1, 0, 2) }
  }
#undef KG_CONV_RV_G
#undef KG_CONV_RV_MI
#undef KG_CONV_RV
  if (splits > 1) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int nfp = p.NP * s.f;
    const int rgrid = (nfp + kConvReduceThreads - 1) / kConvReduceThreads;
    if (bias_kind == 0)
      hipLaunchKernelGGL((conv_splitk_reduce_kernel<Tag, 0>), dim3(rgrid), dim3(kConvReduceThreads), 0, stream, partial,
                         splits, y, bias, nfp, p.div_p, s.f);
    else if (bias_kind == 1)
      hipLaunchKernelGGL((conv_splitk_reduce_kernel<Tag, 1>), dim3(rgrid), dim3(kConvReduceThreads), 0, stream, partial,
                         splits, y, bias, nfp, p.div_p, s.f);
    else
      hipLaunchKernelGGL((conv_splitk_reduce_kernel<Tag, 2>), dim3(rgrid), dim3(kConvReduceThreads), 0, stream, partial,
                         splits, y, bias, nfp, p.div_p, s.f);
  }
  return hipGetLastError();
}

// ring: the LDS stage count (2, 3 or 4); the register sets stay two either way
inline hipError_t launch_conv2d_rowvec_f32(const float* x, const float* w, float* y, const float* bias, int bias_kind,
                                           const ConvShape& s, hipStream_t stream, float* partial = nullptr,
                                           int splits = 1, int kcs = 0, int ring = 2) {
  if (ring == 3) return launch_conv2d_rowvec_f32_ring<3>(x, w, y, bias, bias_kind, s, stream, partial, splits, kcs);
  if (ring == 4) return launch_conv2d_rowvec_f32_ring<4>(x, w, y, bias, bias_kind, s, stream, partial, splits, kcs);
  return launch_conv2d_rowvec_f32_ring<2>(x, w, y, bias, bias_kind, s, stream, partial, splits, kcs);
}

template <typename Tag>
hipError_t launch_conv2d_rowvec(const uint16_t* x, const uint16_t* w, uint16_t* y, const void* bias, int bias_kind,
                                const ConvShape& s, hipStream_t stream, float* partial = nullptr, int splits = 1,
                                int kcs = 0, int ring = 2) {
  if (ring == 3) return launch_conv2d_rowvec_ring<Tag, 3>(x, w, y, bias, bias_kind, s, stream, partial, splits, kcs);
  if (ring == 4) return launch_conv2d_rowvec_ring<Tag, 4>(x, w, y, bias, bias_kind, s, stream, partial, splits, kcs);
  return launch_conv2d_rowvec_ring<Tag, 2>(x, w, y, bias, bias_kind, s, stream, partial, splits, kcs);
}

}  // namespace kg_gfx950
