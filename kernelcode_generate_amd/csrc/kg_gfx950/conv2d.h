// NCHW conv2d kernels for the conv2d demos:
//   out[n,f,ho,wo] = sum_{c,kh,kw} x[n,c,ho*sh+kh*dh-pt, wo*sw+kw*dw-pl] * w[f,c,kh,kw] (+ bias[f])
// with zero padding (pt/pb top/bottom, pl/pr left/right) and
//   Ho = (H + pt + pb - dh*(KH-1) - 1) / sh + 1,  Wo = (W + pl + pr - dw*(KW-1) - 1) / sw + 1.
//
// conv2d_direct_kernel: any dtype/stride/dilation/padding; one thread per output element,
//   fp32 accumulation in (c, kh, kw) order, the img2col2d K order.
#pragma once

#include "common.h"

namespace kg_gfx950 {

struct ConvShape {
  int n, c, h, w;       // input
  int f, kh, kw;        // weight
  int ho, wo;           // output
  int sh, sw, dh, dw;   // stride, dilation
  int pt, pl;           // top/left padding (bottom/right only change Ho/Wo)
};

template <typename TX, typename TW, typename TO, typename TB>
__global__ __launch_bounds__(256) void conv2d_direct_kernel(const TX* __restrict__ x, const TW* __restrict__ w,
                                                            TO* __restrict__ out, const TB* __restrict__ bias,
                                                            ConvShape s) {
  const long long total = (long long)s.n * s.f * s.ho * s.wo;
  for (long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (long long)gridDim.x * blockDim.x) {
    const int wo = (int)(idx % s.wo);
    long long t = idx / s.wo;
    const int ho = (int)(t % s.ho);
    t /= s.ho;
    const int f = (int)(t % s.f);
    const int n = (int)(t / s.f);
    float acc = 0.f;
    const int h_base = ho * s.sh - s.pt;
    const int w_base = wo * s.sw - s.pl;
    for (int c = 0; c < s.c; ++c) {
      const TX* xc = x + ((long long)n * s.c + c) * s.h * s.w;
      const TW* wc = w + ((long long)f * s.c + c) * s.kh * s.kw;
      for (int r = 0; r < s.kh; ++r) {
        const int hh = h_base + r * s.dh;
        if (hh < 0 || hh >= s.h) continue;
        for (int q = 0; q < s.kw; ++q) {
          const int ww = w_base + q * s.dw;
          if (ww < 0 || ww >= s.w) continue;
          acc = __builtin_fmaf(Elem<TX>::load(xc + (long long)hh * s.w + ww), Elem<TW>::load(wc + r * s.kw + q), acc);
        }
      }
    }
    if (bias != nullptr) acc += Elem<TB>::load(bias + f);
    Elem<TO>::store(out + idx, acc);
  }
}

}  // namespace kg_gfx950
