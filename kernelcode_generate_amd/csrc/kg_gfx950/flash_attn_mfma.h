// Flash-attention forward on gfx950 MFMA: 16-bit Q/K/V/O [B,H,S,D], D in {64, 128},
// fp32 online softmax, optional scale and causal mask.
//
// Work split: one workgroup = 128 query rows of one (b,h), 4 waves x 32 queries; key/value
// tiles of 64 keys are staged through LDS (double buffered) and shared by the 4 waves.
//
// Per wave and key tile the kernel computes S^T = K Q^T with v_mfma_f32_32x32x16 (operand A
// = 32 keys x 16 d from LDS, operand B = Q^T kept in registers for the whole kernel). In
// the 32x32 MFMA result lane l holds column l%32 (one query) and rows {8j + 4(l/32) + r};
// the K rows are read in the permuted order pi(8j + 4h + r) = 16h + 4j + r, so lane l ends
// up with the scores of ITS query against 16 CONSECUTIVE keys (16h .. 16h+15 of the
// 32-key block). The row max/sum are therefore lane-local plus one exchange with lane
// l^32, and P (converted to 16-bit) is already laid out as the B operand of
// O^T += V^T P^T: lane half h supplies keys 16h+8t .. 16h+8t+7 of MFMA t, which is one
// 16-byte read of the transposed V tile. O^T keeps one query per lane column as well, so
// the rescale by exp(m_old - m_new) is lane-local.
//
// Softmax works in base 2: p = exp2(s * scale*log2(e) - m) with m tracked in the same
// units; exp2 is v_exp_f32. P is rounded to the input format before the PV product.
//
// K tiles are copied HBM -> LDS by global_load_lds_dwordx4 (no registers); each lane
// fetches the 16-byte chunk that belongs at its LDS slot under the swizzle. V arrives
// key-major; each thread loads a 4-key x 8-d block with 16-byte loads, transposes it in
// registers (v_perm_b32) and writes d-major 8-byte pieces to LDS. Both LDS tiles use
// XOR-swizzled 16-byte chunks so the fragment reads are bank-conflict free.
#pragma once

#include "flash_attn.h"

namespace kg_gfx950 {

namespace fa {

constexpr int kBM = 128;  // queries per workgroup
constexpr int kBC = 64;   // keys per tile
constexpr int kThreads = 256;

// Row of the K tile that MFMA row r reads (see header comment).
__device__ __forceinline__ int key_perm(int r) { return 16 * ((r >> 2) & 1) + 4 * (r >> 3) + (r & 3); }
// 16-byte chunk swizzle of the K tile: distinct for each group of 8 MFMA rows.
__device__ __forceinline__ int k_swz(int key) { return (key & 3) | ((key >> 2) & 4); }
// 16-byte chunk swizzle of the V^T tile (8 key-chunks per d row).
__device__ __forceinline__ int v_swz(int d) { return (d & 7) ^ ((d >> 3) & 7); }

}  // namespace fa

template <typename Tag, int D, bool kCausal, bool kMasked>
__global__ __launch_bounds__(fa::kThreads, 2) void fa_fwd_mfma_kernel(const uint16_t* __restrict__ Q,
                                                                      const uint16_t* __restrict__ K,
                                                                      const uint16_t* __restrict__ V,
                                                                      uint16_t* __restrict__ O, int bh_count, int s_q,
                                                                      int s_kv, float scale_log2) {
  using namespace fa;
  using H = Half16<Tag>;
  constexpr int DCH = D / 8;           // 16-byte chunks per K row
  constexpr int KVEC = kBC * DCH;      // u32x4 per K tile
  constexpr int VVEC = D * (kBC / 8);  // u32x4 per V^T tile
  constexpr int NDB = D / 32;          // 32-wide d blocks of O^T
  constexpr int NKK = D / 16;          // 16-wide d steps of S^T

  __shared__ u32x4 k_lds[2][KVEC];
  __shared__ u32x4 v_lds[2][VVEC];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int ql = lane & 31;

  const int nmb = (s_q + kBM - 1) / kBM;
  const int pid = blockIdx.x;
  const int bh = pid % bh_count;
  int mb = pid / bh_count;
  if (kCausal) mb = nmb - 1 - mb;  // longest query blocks first
  const int m0 = mb * kBM;
  const uint16_t* Qh = Q + (long long)bh * s_q * D;
  const uint16_t* Kh = K + (long long)bh * s_kv * D;
  const uint16_t* Vh = V + (long long)bh * s_kv * D;
  uint16_t* Oh = O + (long long)bh * s_q * D;

  const int q_row = m0 + 32 * wave + ql;
  u32x4 qf[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk)
    qf[kk] = (!kMasked || q_row < s_q) ? ld16(Qh + (long long)q_row * D + 16 * kk + 8 * half) : u32x4{0, 0, 0, 0};

  f32x16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.f;
  float m_run = -INFINITY;
  float l_run = 0.f;

  const int n_end = kCausal ? min(s_kv, m0 + kBM) : s_kv;
  const int ntiles = (n_end + kBC - 1) / kBC;

  // V: each thread owns a 4-key x 8-d block: key group va (0..15), d chunk ve.
  constexpr int VTHREADS = (kBC / 4) * (D / 8);
  const int ve = tid % (D / 8);
  const int va = tid / (D / 8);
  // K: wave-level direct global->LDS copies, KROWS rows of the tile per instruction.
  constexpr int KROWS = 64 / DCH;
  constexpr int KINST = kBC / KROWS / 4;  // instructions per wave
  static_assert(kBC % (KROWS * 4) == 0, "K tile must split over 4 waves");

  u32x4 vpre[4];

  auto load_tile = [&](int j, int buf) {
    const int n0 = j * kBC;
#pragma unroll
    for (int i = 0; i < KINST; ++i) {
      const int slab = wave * KINST + i;  // KROWS rows per slab
      const int row = slab * KROWS + lane / DCH;
      const int pc = lane % DCH;
      int grow = n0 + row;
      if (kMasked) grow = min(grow, s_kv - 1);  // clamped rows are masked out of S below
      const uint16_t* src = Kh + (long long)grow * D + 8 * (pc ^ k_swz(row));
      __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)&k_lds[buf][slab * 64], 16, 0, 0);
    }
    if (tid < VTHREADS) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = n0 + 4 * va + r;
        vpre[r] = (!kMasked || row < s_kv) ? ld16(Vh + (long long)row * D + 8 * ve) : u32x4{0, 0, 0, 0};
      }
    }
  };
  auto store_v = [&](int buf) {
    if (tid < VTHREADS) {
      uint32_t* vrow = reinterpret_cast<uint32_t*>(&v_lds[buf][0]);
#pragma unroll
      for (int jd = 0; jd < 8; ++jd) {
        const int dw = jd >> 1;
        u32x2 col;
        if (jd & 1) {
          col[0] = hi_halves(vpre[0][dw], vpre[1][dw]);
          col[1] = hi_halves(vpre[2][dw], vpre[3][dw]);
        } else {
          col[0] = lo_halves(vpre[0][dw], vpre[1][dw]);
          col[1] = lo_halves(vpre[2][dw], vpre[3][dw]);
        }
        const int d = 8 * ve + jd;
        const int chunk = (va >> 1) ^ v_swz(d);
        *reinterpret_cast<u32x2*>(vrow + (d * 8 + chunk) * 4 + (va & 1) * 2) = col;
      }
    }
  };

  load_tile(0, 0);
  store_v(0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  const int wave_q_lo = m0 + 32 * wave;
  const int wave_q_hi = wave_q_lo + 31;

  for (int j = 0; j < ntiles; ++j) {
    const int cur = j & 1;
    const int n0 = j * kBC;
    if (j + 1 < ntiles) load_tile(j + 1, cur ^ 1);

    // A causal tile that starts past every query of this wave contributes nothing.
    const bool active = !kCausal || n0 <= wave_q_hi;
    if (active) {
      f32x16 s[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) s[kb][i] = 0.f;
        const int key = kb * 32 + key_perm(ql);
        const int sw = k_swz(key);
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
          const u32x4 kf = k_lds[cur][key * DCH + ((2 * kk + half) ^ sw)];
          s[kb] = H::mfma32(kf, qf[kk], s[kb]);
        }
      }
      // lane holds S[q_row][n0 + 32kb + 16*half + i]
      const bool need_mask = (kMasked && n0 + kBC > s_kv) || (kCausal && n0 + kBC - 1 > wave_q_lo);
      if (need_mask) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = n0 + 32 * kb + 16 * half + i;
            const bool dead = (kMasked && key >= s_kv) || (kCausal && key > q_row);
            if (dead) s[kb][i] = -INFINITY;
          }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[kb][i]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx * scale_log2);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      float rs = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][i], scale_log2, -m_new));
          s[kb][i] = p;
          rs += p;
        }
      l_run = l_run * alpha + rs;
      m_run = m_new;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[db][i] *= alpha;

#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          u32x4 pp;
#pragma unroll
          for (int e = 0; e < 4; ++e) pp[e] = H::pack2(s[kb][8 * t + 2 * e], s[kb][8 * t + 2 * e + 1]);
          const int kc = 4 * kb + 2 * half + t;
#pragma unroll
          for (int db = 0; db < NDB; ++db) {
            const int d = 32 * db + ql;
            const u32x4 vf = v_lds[cur][d * 8 + (kc ^ v_swz(d))];
            o[db] = H::mfma32(vf, pp, o[db]);
          }
        }
      }
    }
    if (j + 1 < ntiles) store_v(cur ^ 1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = 1.f / l_tot;
  if (!kMasked || q_row < s_q) {
    uint16_t* orow = Oh + (long long)q_row * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        // lane holds O^T[32db + 8jj + 4*half + r][q_row], r = 0..3
        u32x2 packed;
        packed[0] = H::pack2(o[db][4 * jj] * inv, o[db][4 * jj + 1] * inv);
        packed[1] = H::pack2(o[db][4 * jj + 2] * inv, o[db][4 * jj + 3] * inv);
        st8(orow + 32 * db + 8 * jj + 4 * half, packed);
      }
  }
}

inline bool fa_mfma_supported(const FaShape& s) {
  return (s.d == 64 || s.d == 128) && s.scale > 0.f && s.s_q >= 1 && s.s_kv >= 1 && (!s.causal || s.s_q == s.s_kv) &&
         (long long)((s.s_q + fa::kBM - 1) / fa::kBM) * s.bh < (1ll << 31);
}

template <typename Tag, int D>
hipError_t launch_fa_fwd_mfma_d(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, const FaShape& s,
                                hipStream_t stream) {
  const int nmb = (s.s_q + fa::kBM - 1) / fa::kBM;
  const dim3 grid(nmb * s.bh);
  const bool masked = (s.s_q % fa::kBM) != 0 || (s.s_kv % fa::kBC) != 0;
  const float scale_log2 = s.scale * 1.4426950408889634f;
  if (s.causal) {
    if (masked)
      hipLaunchKernelGGL((fa_fwd_mfma_kernel<Tag, D, true, true>), grid, dim3(fa::kThreads), 0, stream, q, k, v, o, s.bh,
                         s.s_q, s.s_kv, scale_log2);
    else
      hipLaunchKernelGGL((fa_fwd_mfma_kernel<Tag, D, true, false>), grid, dim3(fa::kThreads), 0, stream, q, k, v, o, s.bh,
                         s.s_q, s.s_kv, scale_log2);
  } else {
    if (masked)
      hipLaunchKernelGGL((fa_fwd_mfma_kernel<Tag, D, false, true>), grid, dim3(fa::kThreads), 0, stream, q, k, v, o, s.bh,
                         s.s_q, s.s_kv, scale_log2);
    else
      hipLaunchKernelGGL((fa_fwd_mfma_kernel<Tag, D, false, false>), grid, dim3(fa::kThreads), 0, stream, q, k, v, o, s.bh,
                         s.s_q, s.s_kv, scale_log2);
  }
  return hipGetLastError();
}

template <typename Tag>
hipError_t launch_fa_fwd_mfma(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, const FaShape& s,
                              hipStream_t stream) {
  if (s.d == 128) return launch_fa_fwd_mfma_d<Tag, 128>(q, k, v, o, s, stream);
  return launch_fa_fwd_mfma_d<Tag, 64>(q, k, v, o, s, stream);
}

}  // namespace kg_gfx950
