// Flash-attention forward for fp32 Q/K/V/O [B,H,S,D], D in {64, 128}, on gfx950 matrix
// cores (v_mfma_f32_32x32x2_f32: fp32 products, fp32 accumulation), fp32 online softmax,
// optional scale and causal mask.
//
// The fp32 MFMA issues once per 64 cycles, so per 32 keys a wave spends D x 64 cycles in
// MFMAs against a few dozen VALU and LDS instructions: the kernel is simply kept MFMA-bound.
// A workgroup is 4 waves x 32 queries of one (b,h); 32-key K and V tiles are copied
// HBM -> LDS (global buffer loads straight into LDS, two buffers each), one tile ahead.
//
// S^T = K Q^T: operand A = 32 keys of the K tile, operand B = Q^T held in registers for the
// whole kernel. The contraction order over d is permuted: lane half h of k-step kk of group
// g covers d = 8g + 4h + kk, so one ds_read_b128 of a K row feeds four k-steps and lane l
// keeps Q[q][8g + 4h .. +3] as one float4 per g. In the 32x32 result lane l holds query
// l % 32 against keys 8(e/4) + 4(l/32) + e%4 (element e): the row max and sum are
// lane-local plus one exchange with lane l ^ 32.
// O^T += V^T P^T: the k-step (e', i) pairs key 8e' + i (lane half 0) with key 8e' + 4 + i
// (half 1), which is exactly score element 4e' + i of each lane, so P feeds the MFMA from
// the registers it was computed in; the V^T operand is one ds_read_b32 (V[key][d], 32
// consecutive d per lane half). Lane l ends with O[l % 32][32 b + 8(e/4) + 4(l/32) + e%4].
//
// LDS swizzles (16-byte chunks, 64 banks of 4 bytes): K chunk c of key row r at slot
// c ^ (r & 15) (the 16 lanes of a b128 read cycle read 16 rows at one chunk); V chunk c at
// c ^ 8((r >> 2) & 1) (the two lane halves read rows r and r + 4). Every copy lane fetches
// the HBM chunk that belongs at its LDS slot; keys past S_kv are out of the buffer range
// and land zeros (their scores are masked to -inf).
#pragma once

#include "flash_attn.h"
#include "flash_attn_mfma.h"
#include "lds_dma.h"

namespace kg_gfx950 {

namespace faf {
constexpr int kWaves = 4;
constexpr int kBM = 32 * kWaves;  // queries per workgroup
constexpr int kBC = 32;           // keys per tile
constexpr int kThreads = 64 * kWaves;
__host__ __device__ constexpr int k_slot(int r, int c) { return c ^ (r & 15); }
__host__ __device__ constexpr int v_slot(int r, int c) { return c ^ (8 * ((r >> 2) & 1)); }
}  // namespace faf

template <int D, bool kCausal>
__global__ __launch_bounds__(faf::kThreads, D == 128 ? 2 : 4) void fa_fwd_f32_mfma_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V, float* __restrict__ O,
    int bh_count, int s_q, int s_kv, float scale_log2) {
  using namespace faf;
  static_assert(D == 64 || D == 128, "head dim");
  constexpr int kTileBytes = kBC * D * 4;  // 8 or 16 KiB
  constexpr int kChunks = D / 4;           // 16-byte chunks per row
  constexpr int kRowsPerCopy = 64 / kChunks;
  constexpr int kCopies = kTileBytes / 1024 / kWaves;  // per wave per tile, for K and again for V
  constexpr int G = D / 8;                 // b128 groups of the QK contraction
  constexpr int NB = D / 32;               // 32-wide d blocks of O
  __shared__ __attribute__((aligned(1024))) char lds[4 * kTileBytes];  // K0 K1 V0 V1

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nqb = (s_q + kBM - 1) / kBM;
  const int logical = fa::xcd_block(blockIdx.x, gridDim.x);
  const int bh = logical / nqb;
  int qb = logical - bh * nqb;
  if (kCausal) qb = nqb - 1 - qb;  // longest query blocks of a (b,h) first
  const int q_wg = qb * kBM;
  const int q0 = q_wg + 32 * wave;
  const int frag = lane & 31;
  const int h = lane >> 5;
  const bool active = q0 < s_q;  // wave-uniform: waves past the last query only copy

  // ---- Q^T operand: Q[q][8g + 4h .. +3], rows past S_q read the last row (never stored) ----
  const int q_row = min(q0 + frag, s_q - 1);
  f32x4 qf[G];
  {
    const float* qp = Q + ((long long)bh * s_q + q_row) * D + 4 * h;
#pragma unroll
    for (int g = 0; g < G; ++g) qf[g] = *reinterpret_cast<const f32x4*>(qp + 8 * g);
  }

  // ---- copies: instruction p of a wave covers tile rows (wave*kCopies + p)*kRowsPerCopy +
  // lane / kChunks, LDS slot lane % kChunks ----
  const int n_tiles_all = (s_kv + kBC - 1) / kBC;
  const int n_tiles = kCausal ? min(n_tiles_all, (min(q_wg + kBM, s_q) + kBC - 1) / kBC) : n_tiles_all;
  uint32_t k_off[kCopies], v_off[kCopies];
  int c_row[kCopies];
#pragma unroll
  for (int p = 0; p < kCopies; ++p) {
    const int r = (wave * kCopies + p) * kRowsPerCopy + lane / kChunks;
    const int slot = lane % kChunks;
    c_row[p] = r;
    k_off[p] = (uint32_t)((r * D + 4 * k_slot(r, slot)) * 4);  // k_slot is an involution
    v_off[p] = (uint32_t)((r * D + 4 * v_slot(r, slot)) * 4);
  }
  const float* k_bh = K + (long long)bh * s_kv * D;
  const float* v_bh = V + (long long)bh * s_kv * D;
  const uint32_t lds0 = lds_addr(lds);
  auto issue = [&](int t) {
    const int buf = t & 1;
    const float* kb = k_bh + (long long)t * kBC * D;
    const float* vb = v_bh + (long long)t * kBC * D;
#pragma unroll
    for (int p = 0; p < kCopies; ++p) {
      const bool ok = t * kBC + c_row[p] < s_kv;
      const uint32_t dst = (wave * kCopies + p) * 1024;
      buf2lds16_s(ok ? k_off[p] : kBufOOB, kb, lds0 + buf * kTileBytes + dst);
      buf2lds16_s(ok ? v_off[p] : kBufOOB, vb, lds0 + (2 + buf) * kTileBytes + dst);
    }
  };

  // ---- fragment addresses (bytes within a tile buffer) ----
  uint32_t k_rd[G];
#pragma unroll
  for (int g = 0; g < G; ++g) k_rd[g] = (uint32_t)(frag * D * 4 + 16 * k_slot(frag, 2 * g + h));
  // V[key][d] for key 8e' + 4h + i, d = 32 b + frag: chunk (32 b + frag) / 4, slot via
  // v_slot(key) whose value depends on h only ((key >> 2) & 1 == h)
  uint32_t v_rd[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int d = 32 * b + frag;
    v_rd[b] = (uint32_t)((4 * h) * D * 4 + 16 * v_slot(4 * h, d >> 2) + 4 * (d & 3));
  }

  f32x16 o[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[b][e] = 0.f;
  float m_run = -INFINITY;  // running max of scale_log2 * s (log2 units)
  float l_run = 0.f;        // this lane's part of the row sum

  issue(0);
  for (int t = 0; t < n_tiles; ++t) {
    wait_and_barrier<0>();  // tile t landed; every wave is done with tile t-1's buffers
    if (t + 1 < n_tiles) issue(t + 1);
    const int key0 = t * kBC;
    if (!active || (kCausal && key0 > q0 + 31)) continue;  // no key of this tile is visible
    const uint32_t kb = lds0 + (t & 1) * kTileBytes;
    const uint32_t vb = lds0 + (2 + (t & 1)) * kTileBytes;

    // Operands are read one step ahead of their MFMAs, so an LDS read's latency overlaps the
    // MFMAs of the step before instead of stalling its own.
    f32x16 s;
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] = 0.f;
    auto read_k = [&](int g) {
      return *(const __attribute__((address_space(3))) f32x4*)(uintptr_t)(kb + k_rd[g]);
    };
    f32x4 kf = read_k(0);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const f32x4 kn = g + 1 < G ? read_k(g + 1) : kf;
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[kk], qf[g][kk], s, 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      kf = kn;
    }

    // mask: keys past S_kv, and (causal) keys after the query
    const int q = q0 + frag;
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int key = key0 + 8 * (e >> 2) + 4 * h + (e & 3);
      const bool dead = key >= s_kv || (kCausal && key > q);
      s[e] = dead ? -INFINITY : s[e] * scale_log2;
      mx = __builtin_elementwise_maximum(mx, s[e]);
    }
    mx = __builtin_elementwise_maximum(mx, __shfl_xor(mx, 32));
    const float m_new = __builtin_elementwise_maximum(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;  // a row with no visible key yet
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      s[e] = __builtin_amdgcn_exp2f(s[e] - m_use);
      sum += s[e];
    }
    l_run = l_run * alpha + sum;
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[b][e] *= alpha;

    // PV step t = 4 ep + i pairs keys 8 ep + i and 8 ep + 4 + i
    auto read_v = [&](int t, int b) {
      return *(const __attribute__((address_space(3))) float*)(uintptr_t)(vb + v_rd[b] + (8 * (t >> 2) + (t & 3)) * D * 4);
    };
    float vc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) vc[b] = read_v(0, b);
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      float vn[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) vn[b] = t + 1 < 16 ? read_v(t + 1, b) : vc[b];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int b = 0; b < NB; ++b) o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vc[b], s[t], o[b], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int b = 0; b < NB; ++b) vc[b] = vn[b];
    }
  }

  if (!active) return;
  const float l_row = l_run + __shfl_xor(l_run, 32);
  const int q = q0 + frag;
  if (q >= s_q) return;
  const float inv = 1.f / l_row;
  float* op = O + ((long long)bh * s_q + q) * D + 4 * h;
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int ep = 0; ep < 4; ++ep) {
      f32x4 r;
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = o[b][4 * ep + e] * inv;
      *reinterpret_cast<f32x4*>(op + 32 * b + 8 * ep) = r;
    }
}

inline bool fa_f32_mfma_supported(const FaShape& s) {
  return (s.d == 64 || s.d == 128) && s.s_q >= 1 && s.s_kv >= 1 &&
         (long long)s.bh * ((s.s_q + faf::kBM - 1) / faf::kBM) < (1ll << 31) &&
         (long long)faf::kBC * s.d * 4 * 2 < (1ll << 31);
}

inline hipError_t launch_fa_fwd_f32_mfma(const float* q, const float* k, const float* v, float* o, const FaShape& s,
                                         hipStream_t stream) {
  const int grid = s.bh * ((s.s_q + faf::kBM - 1) / faf::kBM);
  const float scale_log2 = s.scale * 1.4426950408889634f;
#define KG_FA_F32(D, C)                                                                                         \
  hipLaunchKernelGGL((fa_fwd_f32_mfma_kernel<D, C>), dim3(grid), dim3(faf::kThreads), 0, stream, q, k, v, o, s.bh, \
                     s.s_q, s.s_kv, scale_log2)
  if (s.d == 128) {
    if (s.causal) KG_FA_F32(128, true); else KG_FA_F32(128, false);
  } else {
    if (s.causal) KG_FA_F32(64, true); else KG_FA_F32(64, false);
  }
#undef KG_FA_F32
  return hipGetLastError();
}

}  // namespace kg_gfx950
