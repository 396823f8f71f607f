// Shared CDNA4 (gfx950) device helpers: vector types, MFMA wrappers, conversions,
// wave64 reductions. Everything here is written for gfx950 only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kg_gfx950 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

// Element tags: the MFMA paths move 16-bit data as raw bits and only the MFMA
// instruction and the final conversion depend on the format.
struct Bf16Tag {};
struct F16Tag {};

template <typename Tag>
struct Half16;

template <>
struct Half16<Bf16Tag> {
  static constexpr uint32_t kOnePair = 0x3F803F80u;  // two bf16 1.0
  // D(16x16,f32) += A(16x32) * B(32x16); lane l supplies A[l%16][8*(l/16)+0..7] and
  // B[8*(l/16)+0..7][l%16]; D[4*(l/16)+i][l%16] lands in element i.
  static __device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // D(32x32,f32) += A(32x16) * B(16x32); lane l supplies A[l%32][8*(l/32)+0..7].
  static __device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // Round-to-nearest-even float -> bf16 bits (NaN stays NaN).
  static __device__ __forceinline__ uint32_t from_float(float x) {
    uint32_t u = __builtin_bit_cast(uint32_t, x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
  }
  static __device__ __forceinline__ float to_float(uint32_t bits) {
    return __builtin_bit_cast(float, bits << 16);
  }
  // Two floats -> two bf16 (RNE) in one dword: v_cvt_pk_bf16_f32; `a` in the low half.
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
  }
  // acc + (both halves of a packed pair), fp32 accumulate: v_dot2c_f32_bf16 with (1, 1).
  static __device__ __forceinline__ float sum2(uint32_t packed, float acc) {
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, packed), one, acc, false);
  }
};

template <>
struct Half16<F16Tag> {
  static constexpr uint32_t kOnePair = 0x3C003C00u;  // two fp16 1.0
  static __device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t from_float(float x) {
    _Float16 h = (_Float16)x;  // v_cvt_f16_f32: round to nearest even
    return (uint32_t)__builtin_bit_cast(uint16_t, h);
  }
  static __device__ __forceinline__ float to_float(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
  }
  // Two floats -> two fp16 (RNE) in one dword: v_cvt_pk_f16_f32; `a` in the low half.
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
  }
  // acc + (both halves of a packed pair), fp32 accumulate: v_dot2c_f32_f16 with (1, 1).
  static __device__ __forceinline__ float sum2(uint32_t packed, float acc) {
    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, packed), one, acc, false);
  }
};

// Pack two 16-bit values: low half of the result from `lo`, high half from `hi`.
__device__ __forceinline__ uint32_t pack16(uint32_t lo, uint32_t hi) {
  return (lo & 0xffffu) | (hi << 16);
}

// Byte permute: v_perm_b32 picks bytes of {hi:lo} by selector.
// Low 16-bit halves of x (bits 0-15) and y (to bits 16-31).
__device__ __forceinline__ uint32_t lo_halves(uint32_t x, uint32_t y) {
  return __builtin_amdgcn_perm(y, x, 0x05040100u);
}
// High 16-bit halves of x (to bits 0-15) and y (to bits 16-31).
__device__ __forceinline__ uint32_t hi_halves(uint32_t x, uint32_t y) {
  return __builtin_amdgcn_perm(y, x, 0x07060302u);
}

// Transpose an 8x8 block of 16-bit elements held as 8 rows of 16 bytes.
// in[r] holds row r (8 elements, element e in dword e/2, half e%2).
// out[c] holds column c: element r of column c = in[r] element c.
__device__ __forceinline__ void transpose8x8_b16(const u32x4 in[8], u32x4 out[8]) {
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int dw = c >> 1;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t x = in[2 * q][dw];
      const uint32_t y = in[2 * q + 1][dw];
      out[c][q] = (c & 1) ? hi_halves(x, y) : lo_halves(x, y);
    }
  }
}

// Global -> register 16-byte load/store helpers (plain vector memory ops).
// The lane id from an asm statement the compiler may not move or merge: values computed from
// it inside a loop are not hoisted out of that loop (and held in registers across it).
__device__ __forceinline__ int lane_id_volatile() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ void st8(void* p, u32x2 v) { *reinterpret_cast<u32x2*>(p) = v; }

// Wave64 butterfly reductions through ds_swizzle/ds_bpermute (via __shfl_xor).
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Element load/store in a generic 16/32-bit format, converting to/from fp32.
template <typename E>
struct Elem;
template <>
struct Elem<float> {
  static __device__ __forceinline__ float load(const float* p) { return *p; }
  static __device__ __forceinline__ void store(float* p, float v) { *p = v; }
};
template <>
struct Elem<__bf16> {
  static __device__ __forceinline__ float load(const __bf16* p) {
    return Half16<Bf16Tag>::to_float(*reinterpret_cast<const uint16_t*>(p));
  }
  static __device__ __forceinline__ void store(__bf16* p, float v) {
    *reinterpret_cast<uint16_t*>(p) = (uint16_t)Half16<Bf16Tag>::from_float(v);
  }
};
template <>
struct Elem<_Float16> {
  static __device__ __forceinline__ float load(const _Float16* p) { return (float)*p; }
  static __device__ __forceinline__ void store(_Float16* p, float v) { *p = (_Float16)v; }
};

// Maps a workgroup id onto the chip so that consecutive logical ids share one XCD
// (workgroups are dealt to the 8 XCDs round-robin; each XCD has its own L2).
__device__ __forceinline__ int xcd_logical_id(int pid, int num) {
  constexpr int kXcds = 8;
  if (num % kXcds != 0) return pid;
  return (pid % kXcds) * (num / kXcds) + pid / kXcds;
}

}  // namespace kg_gfx950
