// Flash-attention forward on gfx950 MFMA (16-bit Q/K/V, fp32 online softmax).
#pragma once

#include "flash_attn.h"

namespace kg_gfx950 {

inline bool fa_mfma_supported(const FaShape&) { return false; }

template <typename Tag>
hipError_t launch_fa_fwd_mfma(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, const FaShape&,
                              hipStream_t) {
  return hipErrorNotSupported;
}

}  // namespace kg_gfx950
