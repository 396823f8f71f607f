// Explicit instantiations of the launchers of the large kernel families. Each family is
// compiled in a translation unit of its own (kg_gfx950_<family>.hip defines KG_INSTANTIATE
// and KG_INSTANTIATE_<FAMILY>), in parallel; every other translation unit, the entry's
// included, sees `extern template` declarations and so neither instantiates the launchers
// nor compiles their kernels.
#pragma once

#include "conv2d_igemm.h"
#include "conv2d_mfma.h"
#include "conv2d_rowvec.h"
#include "flash_attn_mfma.h"
#include "gemm.h"
#include "gemm_quad.h"

#ifdef KG_INSTANTIATE
#define KG_INSTANCE template
#else
#define KG_INSTANCE extern template
#endif

namespace kg_gfx950 {

#if !defined(KG_INSTANTIATE) || defined(KG_INSTANTIATE_GEMM)
#define KG_GEMM_PIPE_INSTANCE(TAG, TM, ST, RAG)                                                                          \
  KG_INSTANCE hipError_t launch_gemm_pipe<TAG, TM, ST, RAG>(const uint16_t*, const uint16_t*, uint16_t*, const void*, int, \
                                                            int, int, int, long long, long long, long long, float*, int,  \
                                                            int, int, hipStream_t);
#define KG_GEMM_PIPE_INSTANCES(TAG, TM, RAG) \
  KG_GEMM_PIPE_INSTANCE(TAG, TM, 2, RAG) KG_GEMM_PIPE_INSTANCE(TAG, TM, 3, RAG) KG_GEMM_PIPE_INSTANCE(TAG, TM, 4, RAG)
KG_GEMM_PIPE_INSTANCES(Bf16Tag, 128, false)
KG_GEMM_PIPE_INSTANCES(Bf16Tag, 128, true)
KG_GEMM_PIPE_INSTANCES(Bf16Tag, 256, false)
KG_GEMM_PIPE_INSTANCES(Bf16Tag, 256, true)
KG_GEMM_PIPE_INSTANCES(F16Tag, 128, false)
KG_GEMM_PIPE_INSTANCES(F16Tag, 128, true)
KG_GEMM_PIPE_INSTANCES(F16Tag, 256, false)
KG_GEMM_PIPE_INSTANCES(F16Tag, 256, true)
#undef KG_GEMM_PIPE_INSTANCES
#undef KG_GEMM_PIPE_INSTANCE
#endif

#if !defined(KG_INSTANTIATE) || defined(KG_INSTANTIATE_GEMM_QUAD)
#define KG_GEMM_QUAD_INSTANCE(TAG, ST, TM)                                                                              \
  KG_INSTANCE hipError_t launch_gemm_quad<TAG, ST, TM>(const uint16_t*, const uint16_t*, uint16_t*, const void*, int, int, \
                                                       int, int, long long, long long, long long, hipStream_t);
#define KG_GEMM_QUAD_INSTANCES(TAG, TM) \
  KG_GEMM_QUAD_INSTANCE(TAG, 2, TM) KG_GEMM_QUAD_INSTANCE(TAG, 3, TM) KG_GEMM_QUAD_INSTANCE(TAG, 4, TM)
KG_GEMM_QUAD_INSTANCES(Bf16Tag, 256)
KG_GEMM_QUAD_INSTANCES(Bf16Tag, 128)
KG_GEMM_QUAD_INSTANCES(F16Tag, 256)
KG_GEMM_QUAD_INSTANCES(F16Tag, 128)
#undef KG_GEMM_QUAD_INSTANCES
#undef KG_GEMM_QUAD_INSTANCE
#endif

// The persistent attention form: its own translation unit; every other one, the attention
// family's included, sees `extern template` declarations (ahead of the attention launchers
// that call it).
#ifdef KG_INSTANTIATE_FA_PERSIST
#define KG_FA_PERSIST_INSTANCE(TAG, D, W)                                                                          \
  template hipError_t launch_fa_fwd_mfma_persist<TAG, D, W>(const uint16_t*, const uint16_t*, const uint16_t*,     \
                                                            uint16_t*, const FaShape&, int, hipStream_t);
#else
#define KG_FA_PERSIST_INSTANCE(TAG, D, W)                                                                          \
  extern template hipError_t launch_fa_fwd_mfma_persist<TAG, D, W>(const uint16_t*, const uint16_t*,              \
                                                                   const uint16_t*, uint16_t*, const FaShape&, int, \
                                                                   hipStream_t);
#endif
KG_FA_PERSIST_INSTANCE(Bf16Tag, 128, 8)
KG_FA_PERSIST_INSTANCE(Bf16Tag, 64, 4)
KG_FA_PERSIST_INSTANCE(F16Tag, 128, 8)
KG_FA_PERSIST_INSTANCE(F16Tag, 64, 4)
#undef KG_FA_PERSIST_INSTANCE

#if !defined(KG_INSTANTIATE) || defined(KG_INSTANTIATE_FA)
#define KG_FA_INSTANCE(TAG, ST)                                                                                      \
  KG_INSTANCE hipError_t launch_fa_fwd_mfma_st<TAG, ST>(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, \
                                                        const FaShape&, hipStream_t);
KG_FA_INSTANCE(Bf16Tag, 2)
KG_FA_INSTANCE(Bf16Tag, 3)
KG_FA_INSTANCE(Bf16Tag, 4)
KG_FA_INSTANCE(F16Tag, 2)
KG_FA_INSTANCE(F16Tag, 3)
KG_FA_INSTANCE(F16Tag, 4)
#undef KG_FA_INSTANCE
#endif

#if !defined(KG_INSTANTIATE) || defined(KG_INSTANTIATE_CONV_ROWVEC)
#define KG_ROWVEC_INSTANCE(TAG, R)                                                                                      \
  KG_INSTANCE hipError_t launch_conv2d_rowvec_ring<TAG, R>(const uint16_t*, const uint16_t*, uint16_t*, const void*, int, \
                                                           const ConvShape&, hipStream_t, float*, int, int);
#define KG_ROWVEC_F32_INSTANCE(R)                                                                                       \
  KG_INSTANCE hipError_t launch_conv2d_rowvec_f32_ring<R>(const float*, const float*, float*, const float*, int,         \
                                                          const ConvShape&, hipStream_t, float*, int, int);
KG_ROWVEC_INSTANCE(Bf16Tag, 2)
KG_ROWVEC_INSTANCE(Bf16Tag, 3)
KG_ROWVEC_INSTANCE(Bf16Tag, 4)
KG_ROWVEC_INSTANCE(F16Tag, 2)
KG_ROWVEC_INSTANCE(F16Tag, 3)
KG_ROWVEC_INSTANCE(F16Tag, 4)
KG_ROWVEC_F32_INSTANCE(2)
KG_ROWVEC_F32_INSTANCE(3)
KG_ROWVEC_F32_INSTANCE(4)
#undef KG_ROWVEC_F32_INSTANCE
#undef KG_ROWVEC_INSTANCE
KG_INSTANCE hipError_t launch_conv2d_mfma<Bf16Tag>(const uint16_t*, const uint16_t*, uint16_t*, const void*, int,
                                                    const ConvShape&, hipStream_t);
KG_INSTANCE hipError_t launch_conv2d_mfma<F16Tag>(const uint16_t*, const uint16_t*, uint16_t*, const void*, int,
                                                   const ConvShape&, hipStream_t);
#endif

#if !defined(KG_INSTANTIATE) || defined(KG_INSTANTIATE_CONV_IGEMM)
#define KG_IGEMM_INSTANCE(TAG, R)                                                                                      \
  KG_INSTANCE hipError_t launch_conv2d_igemm_ring<TAG, R>(const void*, const void*, void*, const void*, int, int, bool, \
                                                          const ConvShape&, hipStream_t, float*, int, int);
KG_IGEMM_INSTANCE(F32Tag, 2)
KG_IGEMM_INSTANCE(F32Tag, 3)
KG_IGEMM_INSTANCE(F32Tag, 4)
KG_IGEMM_INSTANCE(Bf16Tag, 2)
KG_IGEMM_INSTANCE(Bf16Tag, 3)
KG_IGEMM_INSTANCE(Bf16Tag, 4)
KG_IGEMM_INSTANCE(F16Tag, 2)
KG_IGEMM_INSTANCE(F16Tag, 3)
KG_IGEMM_INSTANCE(F16Tag, 4)
#undef KG_IGEMM_INSTANCE
#endif

}  // namespace kg_gfx950

#undef KG_INSTANCE
