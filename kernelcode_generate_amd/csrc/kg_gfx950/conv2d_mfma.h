// Implicit-GEMM conv2d on gfx950 MFMA (16-bit NCHW operands, fp32 accumulation).
#pragma once

#include "conv2d.h"

namespace kg_gfx950 {

inline bool conv_mfma_supported(const ConvShape&) { return false; }

template <typename Tag>
hipError_t launch_conv2d_mfma(const uint16_t*, const uint16_t*, uint16_t*, const void*, int, const ConvShape&,
                              hipStream_t) {
  return hipErrorNotSupported;
}

}  // namespace kg_gfx950
