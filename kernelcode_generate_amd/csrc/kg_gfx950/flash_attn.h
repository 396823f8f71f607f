// Flash-attention forward kernels for the flash_attention demos:
//   O[b,h] = softmax(scale * Q[b,h] K[b,h]^T (+ causal mask)) V[b,h],  layout [B,H,S,D].
// The reference demo computes the online softmax per key block: running row max m,
// running row sum l, P = exp(S - m_new), l' = l*exp(m - m_new) + rowsum(P),
// acc' = acc*exp(m - m_new) + P V, O = acc / l (scale 1, no mask).
//
// fa_fwd_simt_kernel: any dtype, any S and D <= 512; one 128-thread block per (b*h, query
//   row), on a one-dimensional grid, keys processed in blocks of 128 with the same online-softmax recurrence.
#pragma once

#include "common.h"

namespace kg_gfx950 {

struct FaShape {
  int bh;        // B*H
  int s_q;       // query length
  int s_kv;      // key length
  int d;         // head dim
  float scale;   // multiplies Q K^T
  int causal;    // key j visible to query i iff j <= i
};

template <typename T>
__global__ __launch_bounds__(128) void fa_fwd_simt_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                          const T* __restrict__ v, T* __restrict__ o,
                                                          FaShape s) {
  constexpr int kThreads = 128;
  constexpr int kMaxD = 512;
  constexpr int kDPer = kMaxD / kThreads;
  __shared__ float qs[kMaxD];
  __shared__ float ps[kThreads];
  __shared__ float red[kThreads / 64];

  // one-dimensional grid: block b is query row b % S_q of head b / S_q
  const int row = (int)(blockIdx.x % (unsigned)s.s_q);
  const int bh = (int)(blockIdx.x / (unsigned)s.s_q);
  const int tid = threadIdx.x;
  const long long base_q = ((long long)bh * s.s_q + row) * s.d;
  const long long base_kv = (long long)bh * s.s_kv * s.d;
  for (int d = tid; d < s.d; d += kThreads) qs[d] = Elem<T>::load(q + base_q + d);
  __syncthreads();

  float acc[kDPer];
#pragma unroll
  for (int i = 0; i < kDPer; ++i) acc[i] = 0.f;
  float m_state = -INFINITY;
  float l_state = 0.f;
  const int kv_end = s.causal ? min(s.s_kv, row + 1) : s.s_kv;

  for (int n0 = 0; n0 < kv_end; n0 += kThreads) {
    const int n = n0 + tid;
    float score = -INFINITY;
    if (n < kv_end) {
      const T* kr = k + base_kv + (long long)n * s.d;
      float dot = 0.f;
      for (int d = 0; d < s.d; ++d) dot = __builtin_fmaf(qs[d], Elem<T>::load(kr + d), dot);
      score = dot * s.scale;
    }
    // block max
    float mx = wave_max(score);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(red[0], red[1]);
    __syncthreads();
    const float m_new = fmaxf(m_state, mx);
    const float p = (n < kv_end) ? expf(score - m_new) : 0.f;
    float sm = wave_sum(p);
    if ((tid & 63) == 0) red[tid >> 6] = sm;
    ps[tid] = p;
    __syncthreads();
    sm = red[0] + red[1];
    const float alpha = expf(m_state - m_new);  // exp(-inf) = 0 on the first block
    l_state = l_state * alpha + sm;
    m_state = m_new;
    const int cnt = min(kThreads, kv_end - n0);
#pragma unroll
    for (int i = 0; i < kDPer; ++i) {
      const int d = tid + i * kThreads;
      if (d < s.d) {
        float a = acc[i] * alpha;
        const T* vc = v + base_kv + (long long)n0 * s.d + d;
        for (int j = 0; j < cnt; ++j) a = __builtin_fmaf(ps[j], Elem<T>::load(vc + (long long)j * s.d), a);
        acc[i] = a;
      }
    }
    __syncthreads();
  }
  const float inv = 1.f / l_state;
#pragma unroll
  for (int i = 0; i < kDPer; ++i) {
    const int d = tid + i * kThreads;
    if (d < s.d) Elem<T>::store(o + base_q + d, acc[i] * inv);
  }
}

}  // namespace kg_gfx950
