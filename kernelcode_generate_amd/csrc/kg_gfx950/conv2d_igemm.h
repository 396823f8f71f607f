// Implicit-GEMM conv2d on gfx950 matrix cores for any NCHW shape, kernel size, stride,
// dilation and padding: bf16/f16 (v_mfma_f32_32x32x16) or fp32 (v_mfma_f32_32x32x2_f32)
// operands, fp32 accumulation.
//
// GEMM view: Y[n][f][p] = sum_k W[f][k] Xcol[k][(n, p)], with k = (c, kh, kw) in the
// weight's own order (K = C KH KW, so W[F][K] is read as stored) and the columns running
// over all N Ho Wo output pixels. A workgroup (4 waves, 2 x 2) computes a BM x 128 tile
// (BM = 64 or 128 filters) and walks K in slices of 64 bytes per row (32 16-bit or 16 fp32
// values). Each thread owns one output column of the tile for the whole K loop (its
// image, input row/column origin and bounds are worked out once) and gathers that column's
// im2col values of the next slice into registers while the MFMAs of the current slice run;
// taps that fall in the padding read nothing and store zeros. Weights are staged the same
// way, as 16-byte row chunks when K allows. Both operands sit in LDS as 64-byte k-rows
// ([filter][k] and [column][k]) with 16-byte chunk c of row r at c ^ ((r >> 2) & 3), so every
// MFMA fragment is one conflict-free ds_read_b128; the MFMA runs as Y^T = Xcol^T W^T
// (columns as operand A) and each lane ends with 4 consecutive output pixels of one filter.
// Divisions by runtime extents (KH KW, KW, C, Ho Wo, Wo) use precomputed multipliers.
#pragma once

#include "common.h"
#include "conv2d.h"

namespace kg_gfx950 {

// n / d for 0 <= n < 2^32 and 1 <= d < 2^31: q = (umulhi(n, mul) + n) >> shift with
// shift = ceil(log2 d) and mul = floor(2^32 (2^shift - d) / d) + 1 (division by invariant
// integers using multiplication, Granlund and Montgomery, PLDI 1994).
struct FastDiv {
  uint32_t d, mul, shift;
};
inline FastDiv make_fast_div(uint32_t d) {
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  const unsigned long long mul = ((1ull << 32) * ((1ull << l) - d)) / d + 1;
  return FastDiv{d, (uint32_t)mul, l};
}
__device__ __forceinline__ uint32_t fdiv(uint32_t n, FastDiv f) {
  const uint32_t hi = __umulhi(n, f.mul);
  return (uint32_t)(((unsigned long long)hi + n) >> f.shift);
}

struct F32Tag {};

namespace convg {
constexpr int kBN = 128;  // output pixels per tile
constexpr int kThreads = 256;
__device__ __forceinline__ int slot(int row, int c) { return row * 4 + (c ^ ((row >> 2) & 3)); }

struct Params {
  int n, c, h, w, f, kh, kw, ho, wo, sh, sw, dh, dw, pt, pl;
  int K, P;   // C KH KW, Ho Wo
  int NP;     // N Ho Wo
  int w_vec;  // tap-major order with KH KW == 1 and 16-byte aligned weights: chunk loads
  int kcs;    // split-K: k slices per workgroup row (blockIdx.y); 0 = the whole K range
  FastDiv div_khw, div_kw, div_p, div_wo, div_c;
};

template <typename Tag>
struct IgElem {  // 16-bit operands: 8 values per 16-byte chunk, 32 per slice row
  using T = uint16_t;
  static constexpr int kPerChunk = 8;
  static __device__ __forceinline__ uint32_t bits(T v) { return v; }
  static __device__ __forceinline__ float to_float(T v) { return Half16<Tag>::to_float(v); }
};
template <>
struct IgElem<F32Tag> {  // fp32 operands: 4 values per chunk, 16 per slice row
  using T = float;
  static constexpr int kPerChunk = 4;
  static __device__ __forceinline__ uint32_t bits(T v) { return __builtin_bit_cast(uint32_t, v); }
  static __device__ __forceinline__ float to_float(T v) { return v; }
};
}  // namespace convg

// kMI: 32-row filter blocks per wave (BM = 64 kMI); kBias: 0 none, 1 fp32, 2 same dtype.
// kOrder: the contraction order. kChannelMajor: k = (c, kh, kw) as the weight is stored,
// weights read as scalars; kChannelMajorVecW: the same with K % (values per chunk) == 0 and
// 16-byte aligned weights, read as chunks; kTapMajor (C % values per chunk == 0): k =
// (kh, kw, c), so the values of one chunk share a tap: one bounds check and one address
// per chunk (channels H W apart), weights read as scalars KH KW apart (as chunks for 1x1).
enum ConvOrder { kChannelMajor = 0, kChannelMajorVecW = 1, kTapMajor = 2 };
// Split-K (s.kcs > 0, for grids of fewer than two workgroups per CU): workgroup row y of the
// grid runs k slices [y kcs, (y+1) kcs) and stores its fp32 sums, without bias, to
// partial[y][N][F][Ho Wo]; conv_splitk_reduce_kernel adds the rows in y order, adds the bias
// and rounds once.
template <typename Tag, int kMI, int kBias, int kOrder, int kRing>
__global__ __launch_bounds__(convg::kThreads) void conv2d_igemm_kernel(
    const typename convg::IgElem<Tag>::T* __restrict__ x, const typename convg::IgElem<Tag>::T* __restrict__ wt,
    typename convg::IgElem<Tag>::T* __restrict__ y, const void* __restrict__ bias, convg::Params s,
    float* __restrict__ partial) {
  using namespace convg;
  using E = IgElem<Tag>;
  using T = typename E::T;
  constexpr int V = E::kPerChunk;
  constexpr int BK = 4 * V;  // k per slice
  constexpr int BM = 64 * kMI;
  constexpr int kStage = (BM + kBN) * 64;  // bytes
  static_assert(kRing >= 2 && kRing <= 4, "LDS ring");
  // slice it is read from stage it % kRing; slice it + 1 is stored after its MFMAs into the
  // stage slice it + 1 - kRing was read from, before the previous step's barrier
  __shared__ __attribute__((aligned(1024))) u32x4 lds[kRing * kStage / 16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_m = (s.f + BM - 1) / BM;
  const int logical = xcd_logical_id(blockIdx.x, gridDim.x);
  const int m0 = (logical % tiles_m) * BM;  // the filter tiles of one column tile are adjacent
  const int n0 = (logical / tiles_m) * kBN;

  // ---- this thread's column: output pixel j = n0 + (tid & 127), chunks cb and cb + 2 ----
  const int jj = tid & (kBN - 1);
  const int cb = tid >> 7;
  const int j = n0 + jj;
  const bool col_ok = j < s.NP;
  const uint32_t jn = fdiv(col_ok ? j : 0, s.div_p);
  const uint32_t jp = (col_ok ? j : 0) - jn * s.P;
  const uint32_t jho = fdiv(jp, s.div_wo);
  const int hi0 = (int)jho * s.sh - s.pt;
  const int wi0 = (int)(jp - jho * s.wo) * s.sw - s.pl;
  const int hw = s.h * s.w;
  const T* xn = x + (long long)jn * s.c * hw;

  auto pack = [&](const T (&v)[V]) -> u32x4 {
    u32x4 out;
    if constexpr (V == 8) {
#pragma unroll
      for (int q = 0; q < 4; ++q) out[q] = E::bits(v[2 * q]) | (E::bits(v[2 * q + 1]) << 16);
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) out[q] = E::bits(v[q]);
    }
    return out;
  };
  auto gather_chunk = [&](int k0) -> u32x4 {  // Xcol[k0 .. k0+V-1][j]
    if constexpr (kOrder == kTapMajor) {
      const uint32_t tap = fdiv(k0, s.div_c);
      const uint32_t c0 = k0 - tap * s.c;
      const uint32_t kh = fdiv(tap, s.div_kw);
      const int hi = hi0 + (int)kh * s.dh, wi = wi0 + (int)(tap - kh * s.kw) * s.dw;
      const bool ok = col_ok && k0 < s.K && (unsigned)hi < (unsigned)s.h && (unsigned)wi < (unsigned)s.w;
      T v[V];
      const T* src = xn + (int)c0 * hw + hi * s.w + wi;
#pragma unroll
      for (int e = 0; e < V; ++e) v[e] = ok ? src[e * hw] : T(0);
      return pack(v);
    }
    uint32_t c = fdiv(k0, s.div_khw);
    const uint32_t r = k0 - c * (s.kh * s.kw);
    uint32_t kh = fdiv(r, s.div_kw);
    uint32_t kw = r - kh * s.kw;
    T v[V];
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const int hi = hi0 + (int)kh * s.dh, wi = wi0 + (int)kw * s.dw;
      const bool ok = col_ok && k0 + e < s.K && (unsigned)hi < (unsigned)s.h && (unsigned)wi < (unsigned)s.w;
      v[e] = ok ? xn[(int)c * hw + hi * s.w + wi] : T(0);
      if (++kw == (uint32_t)s.kw) {
        kw = 0;
        if (++kh == (uint32_t)s.kh) {
          kh = 0;
          ++c;
        }
      }
    }
    return pack(v);
  };
  auto weight_chunk = [&](int f, int k0) -> u32x4 {  // W in contraction order: k0 .. k0+V-1
    const bool row_ok = f < s.f;
    if constexpr (kOrder == kChannelMajorVecW) {
      if (row_ok && k0 < s.K) return ld16(wt + (long long)f * s.K + k0);
      return u32x4{0, 0, 0, 0};
    } else if constexpr (kOrder == kTapMajor) {
      if (s.w_vec) {  // KH KW == 1: the chunk is contiguous
        if (row_ok && k0 < s.K) return ld16(wt + (long long)f * s.K + k0);
        return u32x4{0, 0, 0, 0};
      }
      const uint32_t tap = fdiv(k0, s.div_c);
      const uint32_t c0 = k0 - tap * s.c;
      const int khw = s.kh * s.kw;
      const bool ok = row_ok && k0 < s.K;
      const T* src = wt + (long long)f * s.K + (long long)c0 * khw + tap;
      T v[V];
#pragma unroll
      for (int e = 0; e < V; ++e) v[e] = ok ? src[e * khw] : T(0);
      return pack(v);
    } else {
      T v[V];
#pragma unroll
      for (int e = 0; e < V; ++e) v[e] = (row_ok && k0 + e < s.K) ? wt[(long long)f * s.K + k0 + e] : T(0);
      return pack(v);
    }
  };

  u32x4 rb[2], ra[kMI];
  auto load_regs = [&](int kt) {
    const int kb = kt * BK;
#pragma unroll
    for (int i = 0; i < 2; ++i) rb[i] = gather_chunk(kb + (cb + 2 * i) * V);
#pragma unroll
    for (int i = 0; i < kMI; ++i) {
      const int ci = tid + kThreads * i;  // weight chunk: row ci >> 2, chunk ci & 3
      ra[i] = weight_chunk(m0 + (ci >> 2), kb + (ci & 3) * V);
    }
  };
  auto store_lds = [&](int buf) {
    u32x4* st = lds + buf * (kStage / 16);
#pragma unroll
    for (int i = 0; i < kMI; ++i) {
      const int ci = tid + kThreads * i;
      st[slot(ci >> 2, ci & 3)] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) st[BM * 4 + slot(jj, cb + 2 * i)] = rb[i];
  };

  f32x16 acc[kMI][2];
#pragma unroll
  for (int i = 0; i < kMI; ++i)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][b][e] = 0.f;

  const int frag = lane & 31, h = lane >> 5;
  int kt0 = 0, nk = (s.K + BK - 1) / BK;
  if (s.kcs > 0) {  // split-K: this workgroup row's slices
    kt0 = blockIdx.y * s.kcs;
    nk = min(nk - kt0, s.kcs);
    partial += (long long)blockIdx.y * s.NP * s.f;
  }
  load_regs(kt0);
  store_lds(0);
  __syncthreads();
  for (int it = 0; it < nk; ++it) {
    const int kt = kt0 + it;
    if (it + 1 < nk) load_regs(kt + 1);  // gathers in flight during the MFMAs below
    const u32x4* st = lds + ((unsigned)it % kRing) * (kStage / 16);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      u32x4 af[kMI], bf[2];
#pragma unroll
      for (int i = 0; i < kMI; ++i) af[i] = st[slot(wm * (BM / 2) + 32 * i + frag, 2 * ks + h)];
#pragma unroll
      for (int b = 0; b < 2; ++b) bf[b] = st[BM * 4 + slot(wn * 64 + 32 * b + frag, 2 * ks + h)];
#pragma unroll
      for (int i = 0; i < kMI; ++i)
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          if constexpr (V == 8) {
            acc[i][b] = Half16<Tag>::mfma32(bf[b], af[i], acc[i][b]);
          } else {
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
              const uint32_t bu = bf[b][kk], au = af[i][kk];
              acc[i][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(__builtin_bit_cast(float, bu),
                                                               __builtin_bit_cast(float, au), acc[i][b], 0, 0, 0);
            }
          }
        }
    }
    if (it + 1 < nk) store_lds((unsigned)(it + 1) % kRing);
    __syncthreads();
  }

  // ---- epilogue: lane holds Y[f][j0 .. j0+3], f = tile row wm*BM/2 + 32 i + lane % 32,
  // j0 = tile column wn*64 + 32 b + 8 q + 4 (lane / 32) ----
  const bool vec_out = (s.P & 3) == 0;  // then j0 .. j0+3 lie in one image, p % 4 == 0
#pragma unroll
  for (int i = 0; i < kMI; ++i) {
    const int f = m0 + wm * (BM / 2) + 32 * i + frag;
    if (f >= s.f) continue;
    float bv = 0.f;
    if constexpr (kBias == 1) bv = static_cast<const float*>(bias)[f];
    if constexpr (kBias == 2) bv = E::to_float(static_cast<const T*>(bias)[f]);
    if (s.kcs > 0) bv = 0.f;  // split-K: the reduction adds the bias
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int j0 = n0 + wn * 64 + 32 * b + 8 * q + 4 * h;
        if (j0 >= s.NP) continue;
        float r[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = acc[i][b][4 * q + e] + bv;
        if (s.kcs > 0) {  // fp32 partial sums in Y's layout
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int jv = j0 + e;
            if (jv >= s.NP) break;
            const uint32_t n = fdiv(jv, s.div_p);
            const uint32_t p = jv - n * s.P;
            partial[((long long)n * s.f + f) * s.P + p] = r[e];
          }
        } else if (vec_out) {
          const uint32_t n = fdiv(j0, s.div_p);
          const uint32_t p = j0 - n * s.P;
          T* yp = y + ((long long)n * s.f + f) * s.P + p;
          if constexpr (V == 8) {
            u32x2 packed;
            packed[0] = Half16<Tag>::pack2(r[0], r[1]);
            packed[1] = Half16<Tag>::pack2(r[2], r[3]);
            st8(yp, packed);
          } else {
            *reinterpret_cast<f32x4*>(yp) = f32x4{r[0], r[1], r[2], r[3]};
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int jv = j0 + e;
            if (jv >= s.NP) break;
            const uint32_t n = fdiv(jv, s.div_p);
            const uint32_t p = jv - n * s.P;
            T* yp = y + ((long long)n * s.f + f) * s.P + p;
            if constexpr (V == 8) {
              const uint32_t pk = Half16<Tag>::pack2(r[e], 0.f);
              *yp = (uint16_t)(pk & 0xffffu);
            } else {
              *yp = r[e];
            }
          }
        }
      }
  }
}

// y[e] = round(sum over the splits of partial[split][e] + bias[f]), e = (n F + f) P + p, in
// split order. N F P < 2^31.
constexpr int kConvReduceThreads = 256;
template <typename Tag, int kBias>
__global__ __launch_bounds__(kConvReduceThreads) void conv_splitk_reduce_kernel(
    const float* __restrict__ partial, int splits, typename convg::IgElem<Tag>::T* __restrict__ y,
    const void* __restrict__ bias, int nfp, FastDiv div_p, int f_count) {
  using E = convg::IgElem<Tag>;
  using T = typename E::T;
  const int e = blockIdx.x * kConvReduceThreads + threadIdx.x;
  if (e >= nfp) return;
  float v = partial[e];
  for (int sp = 1; sp < splits; ++sp) v += partial[(long long)sp * nfp + e];
  if constexpr (kBias != 0) {
    const uint32_t nf = fdiv((uint32_t)e, div_p);  // n F + f
    const int f = (int)(nf % (uint32_t)f_count);
    if constexpr (kBias == 1) v += static_cast<const float*>(bias)[f];
    else v += E::to_float(static_cast<const T*>(bias)[f]);
  }
  if constexpr (E::kPerChunk == 8) y[e] = (T)(Half16<Tag>::pack2(v, 0.f) & 0xffffu);
  else y[e] = v;
}

inline bool conv_igemm_supported(const ConvShape& s) {
  const long long K = (long long)s.c * s.kh * s.kw;
  const long long P = (long long)s.ho * s.wo;
  return K >= 1 && K < (1ll << 30) && (long long)s.n * P < (1ll << 31) && (long long)s.c * s.h * s.w < (1ll << 31) &&
         (long long)s.n * s.c * s.h * s.w < (1ll << 40);
}

inline convg::Params conv_igemm_params(const ConvShape& s) {
  convg::Params p;
  p.n = s.n; p.c = s.c; p.h = s.h; p.w = s.w; p.f = s.f; p.kh = s.kh; p.kw = s.kw; p.ho = s.ho; p.wo = s.wo;
  p.sh = s.sh; p.sw = s.sw; p.dh = s.dh; p.dw = s.dw; p.pt = s.pt; p.pl = s.pl;
  p.K = s.c * s.kh * s.kw;
  p.P = s.ho * s.wo;
  p.NP = s.n * p.P;
  p.div_khw = make_fast_div((uint32_t)(s.kh * s.kw));
  p.div_kw = make_fast_div((uint32_t)s.kw);
  p.div_p = make_fast_div((uint32_t)p.P);
  p.div_wo = make_fast_div((uint32_t)s.wo);
  p.div_c = make_fast_div((uint32_t)s.c);
  p.w_vec = 0;
  p.kcs = 0;
  return p;
}

// BM = 128 filters per tile when F > 64 and such tiles still give every CU of the MI355X
// (256) two workgroups; else 64 (more, smaller workgroups fill the chip).
inline int conv_igemm_mi(const ConvShape& s) {
  const long long cols = ((long long)s.n * s.ho * s.wo + convg::kBN - 1) / convg::kBN;
  return s.f > 64 && ((s.f + 127) / 128) * cols >= 512 ? 2 : 1;
}

// Split-K for grids of fewer than two workgroups per CU: the k slices are cut into chunks of
// at least 4 until the grid reaches 512 workgroups (or the fp32 partials would pass
// max_partial_bytes). Returns the split count (1: none) and the slices per chunk.
inline int conv_igemm_splits(const ConvShape& s, bool f32, long long max_partial_bytes, int* kcs) {
  const long long K = (long long)s.c * s.kh * s.kw;
  const long long bk = f32 ? 16 : 32;
  const long long nk = (K + bk - 1) / bk;
  const long long np = (long long)s.n * s.ho * s.wo;
  const long long nfp = np * s.f;
  const int mi = conv_igemm_mi(s);
  const long long grid = ((s.f + 64 * mi - 1) / (64 * mi)) * ((np + convg::kBN - 1) / convg::kBN);
  *kcs = 0;
  if (grid >= 512 || nk < 8 || nfp >= (1ll << 31)) return 1;
  long long splits = std::min((512 + grid - 1) / grid, nk / 4);
  splits = std::min(splits, max_partial_bytes / (nfp * 4));
  if (splits < 2) return 1;
  const long long c = (nk + splits - 1) / splits;
  *kcs = (int)c;
  return (int)((nk + c - 1) / c);
}

// splits > 1: split-K with kcs slices per chunk into the fp32 workspace `partial`
// (splits x N F Ho Wo floats), then the reduction into y.
template <typename Tag, int kRing>
hipError_t launch_conv2d_igemm_ring(const void* x, const void* w, void* y, const void* bias, int bias_kind, int order,
                                    bool w_vec, const ConvShape& s, hipStream_t stream, float* partial, int splits,
                                    int kcs) {
  using T = typename convg::IgElem<Tag>::T;
  convg::Params p = conv_igemm_params(s);
  p.w_vec = w_vec ? 1 : 0;
  if (splits > 1) p.kcs = kcs;
  else splits = 1;
  const int mi = conv_igemm_mi(s);
  const int grid = ((s.f + 64 * mi - 1) / (64 * mi)) * ((p.NP + convg::kBN - 1) / convg::kBN);
  const T* xp = static_cast<const T*>(x);
  const T* wp = static_cast<const T*>(w);
  T* yp = static_cast<T*>(y);
#define KG_CONV_IG(MI, B, O)                                                                                  \
  hipLaunchKernelGGL((conv2d_igemm_kernel<Tag, MI, B, O, kRing>), dim3(grid, splits), dim3(convg::kThreads), 0, stream, xp, wp, \
                     yp, bias, p, partial)
#define KG_CONV_IG_B(MI, O)                  \
  if (bias_kind == 0) KG_CONV_IG(MI, 0, O);   \
  else if (bias_kind == 1) KG_CONV_IG(MI, 1, O); \
  else KG_CONV_IG(MI, 2, O)
#define KG_CONV_IG_O(MI)                                                 \
  if (order == kTapMajor) { KG_CONV_IG_B(MI, kTapMajor); }                \
  else if (order == kChannelMajorVecW) { KG_CONV_IG_B(MI, kChannelMajorVecW); } \
  else { KG_CONV_IG_B(MI, kChannelMajor); }
  if (mi == 2) {
    KG_CONV_IG_O(2)
  } else {
    KG_CONV_IG_O(1)
  }
#undef KG_CONV_IG_O
#undef KG_CONV_IG_B
#undef KG_CONV_IG
  if (splits > 1) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int nfp = p.NP * s.f;
    const int rgrid = (nfp + kConvReduceThreads - 1) / kConvReduceThreads;
    if (bias_kind == 0)
      hipLaunchKernelGGL((conv_splitk_reduce_kernel<Tag, 0>), dim3(rgrid), dim3(kConvReduceThreads), 0, stream, partial,
                         splits, yp, bias, nfp, p.div_p, s.f);
    else if (bias_kind == 1)
      hipLaunchKernelGGL((conv_splitk_reduce_kernel<Tag, 1>), dim3(rgrid), dim3(kConvReduceThreads), 0, stream, partial,
                         splits, yp, bias, nfp, p.div_p, s.f);
    else
      hipLaunchKernelGGL((conv_splitk_reduce_kernel<Tag, 2>), dim3(rgrid), dim3(kConvReduceThreads), 0, stream, partial,
                         splits, yp, bias, nfp, p.div_p, s.f);
  }
  return hipGetLastError();
}

// ring: the LDS stage count (2, 3 or 4); the register set stays one slice ahead either way
template <typename Tag>
hipError_t launch_conv2d_igemm(const void* x, const void* w, void* y, const void* bias, int bias_kind, int order,
                               bool w_vec, const ConvShape& s, hipStream_t stream, float* partial = nullptr,
                               int splits = 1, int kcs = 0, int ring = 2) {
  if (ring == 3)
    return launch_conv2d_igemm_ring<Tag, 3>(x, w, y, bias, bias_kind, order, w_vec, s, stream, partial, splits, kcs);
  if (ring == 4)
    return launch_conv2d_igemm_ring<Tag, 4>(x, w, y, bias, bias_kind, order, w_vec, s, stream, partial, splits, kcs);
  return launch_conv2d_igemm_ring<Tag, 2>(x, w, y, bias, bias_kind, order, w_vec, s, stream, partial, splits, kcs);
}

}  // namespace kg_gfx950
