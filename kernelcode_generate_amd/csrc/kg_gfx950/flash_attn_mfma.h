// Flash-attention forward on gfx950 MFMA: 16-bit Q/K/V/O [B,H,S,D], D in {64, 128},
// fp32 online softmax, optional scale and causal mask.
//
// Work split: a workgroup holds query rows of one (b,h), 32 per wave (Cfg<D>: 8 waves for
// D=128, 4 for D=64 and for D=128 grids too small to give every CU an 8-wave workgroup;
// two waves per SIMD either way). Key/value tiles of 64 keys are copied
// HBM -> LDS (two buffers each for K and V) and shared by the workgroup's waves. Workgroup
// ids are dealt to the 8 XCDs round-robin; they are remapped so that each XCD runs the query
// blocks of the same (b,h) together and its L2 serves their K/V.
//
// Per wave and key tile the kernel computes S^T = K Q^T with v_mfma_f32_32x32x16 (operand A
// = 32 keys x 16 d from LDS, operand B = Q^T kept in registers for the whole kernel). In
// the 32x32 MFMA result lane l holds column l%32 (one query) and rows {8j + 4(l/32) + r};
// the K rows are read in the permuted order pi(8j + 4h + r) = 16h + 4j + r, so lane l ends
// up with the scores of ITS query against 16 CONSECUTIVE keys (16h .. 16h+15 of the
// 32-key block). Row max/sum are lane-local plus one exchange with lane l^32
// (v_permlane32_swap), and P (rounded to 16 bits) is already laid out as the B operand of
// O^T += V^T P^T: lane half h supplies keys 16h+8t .. 16h+8t+7 of MFMA t. The V^T operand
// (8 consecutive keys of one d per lane) comes from the key-major V tile through two
// ds_read_b64_tr_b16: within each 16-lane group, lane j addresses 4 consecutive d of key
// row j/4 and lane i receives key rows 0..3 of column i.
//
// Softmax works in base 2: p = exp2(s * scale*log2(e) - m) with m tracked in the same
// units (v_exp_f32). The running max is raised only when a tile's max exceeds it by more
// than kRescaleSlack, so the O rescale is skipped on most tiles; numerator and denominator
// use the same m, so the result does not depend on it. Row sums add the rounded P pairs
// with v_dot2c_f32_{bf16,f16}: the same P values the PV product uses.
//
// Software pipeline per wave, tile j (S(j) computed and its max known on entry):
//   block 1: the S(j+1) MFMAs, with the exp/pack of 3/4 of S(j) and the K(j+1) fragment
//            reads slotted between them;
//   block 2: the PV(j) MFMAs, with the last quarter of softmax(j), the V(j) fragment reads
//            and the max of S(j+1) slotted between them.
// The copies of K(j+2) and V(j+1) (into the buffers iteration j-1 finished with) are
// slotted between the block-1 MFMAs of iteration j; one wait + barrier ends the iteration.
//
// LDS chunk swizzles (16-byte chunks, 64 banks of 4 bytes; ds_read_b128 serves 16 lanes per
// cycle, 64-bit reads 32): K chunk c of key row r sits at slot c ^ k_mask(r) and V chunk c
// at c ^ v_mask(r). Each copy lane fetches the HBM chunk that belongs at its LDS slot.
#pragma once

#include "flash_attn.h"
#include "lds_dma.h"

namespace kg_gfx950 {

namespace fa {

constexpr int kBC = 64;  // keys per tile
// Waves per workgroup (32 queries each): D=128 uses one 8-wave workgroup per CU (K/V tiles
// shared by 256 queries halve the HBM/L2 -> LDS copy traffic per query), D=64 two 4-wave
// workgroups per CU. Either way two waves share each SIMD.
// A D=128 launch whose 8-wave grid would leave CUs without a workgroup takes 4-wave
// workgroups (two per CU) instead: twice the workgroups for the same queries.
template <int D, int W = (D == 128 ? 8 : 4)>
struct Cfg {
  static constexpr int kWaves = W;
  static constexpr int kBM = 32 * kWaves;  // queries per workgroup
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kPerCU = 8 / kWaves;
};
// Running-max slack (log2 units): P <= 2^8 between rescales.
constexpr float kRescaleSlack = 8.0f;

// Row of the K tile that MFMA row r reads (see header comment).
__host__ __device__ constexpr int key_perm(int r) { return 16 * ((r >> 2) & 1) + 4 * (r >> 3) + (r & 3); }
// The 16 lanes of one b128 read cycle read keys pi(0..15) = {0-3, 16-19, 4-7, 20-23} (+8)
// at the same chunk; D=128 rows are 256 bytes (one bank row), D=64 rows 128 bytes.
template <int D>
__host__ __device__ constexpr int k_mask(int key) {
  return D == 128 ? ((key & 7) | ((key >> 1) & 8)) : (((key >> 1) & 3) | ((key >> 2) & 4));
}
// Transposed reads: the 32 lanes of a cycle read 4 key rows x two 32-byte pieces.
template <int D>
__host__ __device__ constexpr int v_mask(int key) {
  return D == 128 ? 4 * (key & 3) : 4 * ((key >> 1) & 1);
}

// Copy instruction p of wave w covers tile rows (w*PW + p)*RPP + lane/DCH. K keeps a
// per-lane HBM offset for every p; V keeps the one of p = 0 and moves the wave-uniform base
// by whole KiB, which needs the V masks of the rows to repeat (the tail tile uses the same
// offsets).
template <int D, int W>
constexpr bool v_copy_masks_repeat() {
  constexpr int RB = 2 * D, PW = kBC * RB / 1024 / W, RPP = 1024 / RB, DCH = D / 8;
  for (int w = 0; w < W; ++w)
    for (int lane = 0; lane < 64; ++lane)
      for (int p = 0; p < PW; ++p) {
        const int row = (w * PW + p) * RPP + lane / DCH;
        if (v_mask<D>(row) != v_mask<D>((w * PW) * RPP + lane / DCH)) return false;
      }
  return true;
}
static_assert(v_copy_masks_repeat<128, 8>() && v_copy_masks_repeat<128, 4>() && v_copy_masks_repeat<64, 4>(),
              "copy offsets");

// Bijection of workgroup ids: XCD x (ids with id % 8 == x) gets one contiguous range.
__device__ __forceinline__ int xcd_block(int pid, int total) {
  constexpr int kX = 8;
  const int q = total / kX, r = total % kX;
  const int x = pid % kX;
  return x * q + min(x, r) + pid / kX;
}

__device__ __forceinline__ float max3f(float a, float b, float c) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

}  // namespace fa

template <typename Tag, int D, bool kCausal, bool kMasked, int W>
__global__ __launch_bounds__((fa::Cfg<D, W>::kThreads), (fa::Cfg<D, W>::kPerCU)) void fa_fwd_mfma_kernel(const uint16_t* __restrict__ Q,
                                                                      const uint16_t* __restrict__ K,
                                                                      const uint16_t* __restrict__ V,
                                                                      uint16_t* __restrict__ O, int bh_count, int s_q,
                                                                      int s_kv, float scale_log2) {
  using namespace fa;
  using H = Half16<Tag>;
  constexpr int kWaves = Cfg<D, W>::kWaves;
  constexpr int kBM = Cfg<D, W>::kBM;
  constexpr int RB = 2 * D;          // bytes per K/V row
  constexpr int TB = kBC * RB;       // bytes per K or V tile
  constexpr int DCH = D / 8;         // 16-byte chunks per row
  constexpr int NKK = D / 16;        // S^T MFMAs per 32-key block
  constexpr int NDB = D / 32;        // 32-row d blocks of O^T
  constexpr int NS = 2 * NKK;        // S^T MFMAs per tile
  constexpr int NP = 4 * NDB;        // PV MFMAs per tile
  constexpr int PW = TB / 1024 / kWaves;  // copy instructions per wave, tile and operand
  static_assert(PW >= 1 && 2 * PW <= NS, "copy slots");
  constexpr int RPP = 1024 / RB;     // rows per copy instruction

  __shared__ __attribute__((aligned(1024))) u32x4 lds[4 * TB / 16];  // K0 K1 V0 V1

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int ql = lane & 31;

  const int nmb = (s_q + kBM - 1) / kBM;
  const int lin = xcd_block(blockIdx.x, nmb * bh_count);
  const int bh = lin / nmb;
  int mb = lin - bh * nmb;
  if (kCausal) mb = nmb - 1 - mb;  // longest query blocks of a (b,h) first
  const int m0 = mb * kBM;
  const long long kv_base = (long long)bh * s_kv * D;
  const uint16_t* Qh = Q + (long long)bh * s_q * D;
  const char* Kb = reinterpret_cast<const char*>(K + kv_base);
  const char* Vb = reinterpret_cast<const char*>(V + kv_base);
  uint16_t* Oh = O + (long long)bh * s_q * D;

  const int q_row = m0 + 32 * wave + ql;
  u32x4 qf[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk)
    qf[kk] = (!kMasked || q_row < s_q) ? ld16(Qh + (long long)q_row * D + 16 * kk + 8 * half) : u32x4{0, 0, 0, 0};

  const int n_end = kCausal ? min(s_kv, m0 + kBM) : s_kv;
  const int ntiles = (n_end + kBC - 1) / kBC;
  const int wave_q_lo = m0 + 32 * wave;

  // ---- HBM -> LDS copies: K tile t into K buffer b (LDS bytes b*TB), V into 2*TB + b*TB ----
  const uint32_t lds0 = lds_addr(&lds[0]);
  const int c_row0 = wave * PW * RPP + lane / DCH;
  const int c_slot = lane % DCH;
  uint32_t k_goff[PW];
#pragma unroll
  for (int p = 0; p < PW; ++p) {
    const int row = c_row0 + p * RPP;
    k_goff[p] = (uint32_t)(row * RB + 16 * (c_slot ^ k_mask<D>(row)));
  }
  const uint32_t v_goff = (uint32_t)(c_row0 * RB + 16 * (c_slot ^ v_mask<D>(c_row0)));

  // Copy instruction p (< PW) of tile t of K (kV false) or V into the LDS buffer at lds_buf.
  auto copy_piece = [&](const char* src, int t, uint32_t lds_buf, bool kV, int p) {
    const int n0 = t * kBC;
    const uint32_t m = lds_buf + (wave * PW + p) * 1024;
    if constexpr (kMasked) {
      // ragged S: every tile through a raw buffer resource that ends at row s_kv, so the rows
      // of the tail tile past s_kv land zeros (their scores are masked in S: P is 0 there)
      const char* base = src + (long long)n0 * RB + (kV ? p * 1024 : 0);
      const long long left = (long long)(s_kv - n0) * RB - (kV ? p * 1024 : 0);
      const uint32_t range = (uint32_t)max(0ll, min(left, (long long)TB));
      buf2lds16_r(kV ? v_goff : k_goff[p], base, range, m);
    } else {
      const char* base = src + (long long)n0 * RB;
      if (kV) g2lds16_s(v_goff, base + p * 1024, m);
      else g2lds16_s(k_goff[p], base, m);
    }
  };
  auto copy_k = [&](int t, int buf) {
#pragma unroll
    for (int p = 0; p < PW; ++p) copy_piece(Kb, t, lds0 + buf * TB, false, p);
  };
  auto copy_v = [&](int t, int buf) {
#pragma unroll
    for (int p = 0; p < PW; ++p) copy_piece(Vb, t, lds0 + (2 + buf) * TB, true, p);
  };

  // ---- fragment reads ----
  // K: MFMA step i (block kb = i&1, d step kk = i>>1) reads key key_perm(ql) + 32kb, chunk
  // 2kk + half; k_mask(key + 32) == k_mask(key), so kb is an immediate offset.
  uint32_t k_rd[NKK];
  {
    const int key = key_perm(ql);
    const int km = k_mask<D>(key);
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) k_rd[kk] = lds0 + key * RB + 16 * ((2 * kk + half) ^ km);
  }
  // V^T: PV MFMA i = (2kb + t)*NDB + db; lane group g = lane/16 reads key rows
  // 32kb + 16*half + 8t + {0..3} (then +4) and d columns 32db + 16(g&1) .. +15. v_mask of
  // those rows equals that of row 16*half + (j>>2), so kb and t are immediate offsets.
  uint32_t v_rd[NDB];
  {
    const int g = lane >> 4, jj = lane & 15;
    const int row = 16 * half + (jj >> 2);
    const int vm = v_mask<D>(row);
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int c16 = 4 * db + 2 * (g & 1) + ((jj & 3) >> 1);
      v_rd[db] = lds0 + 2 * TB + row * RB + 16 * (c16 ^ vm) + 8 * (jj & 1);
    }
  }
  auto read_k = [&](int buf, int i) -> u32x4 {
    return *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)(k_rd[i >> 1] + buf * TB + (i & 1) * 32 * RB);
  };
  auto read_v = [&](int buf, int i) -> u32x4 {
    const int grp = i / NDB, db = i % NDB;
    const uint32_t a = v_rd[db] + buf * TB + (32 * (grp >> 1) + 8 * (grp & 1)) * RB;
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(uintptr_t)a);
    const s16x4 hi =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(uintptr_t)(a + 4 * RB));
    const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
    return u32x4{l2[0], l2[1], h2[0], h2[1]};
  };

  // ---- softmax state ----
  f32x16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.f;
  float m_run = -INFINITY;  // max used by exp2 (log2 units)
  float l_run = 0.f;        // this lane's share of the row sum
  float m_cur = -INFINITY;  // max of the S tile about to be exponentiated (log2 units)
  u32x4 pp[4];              // P of group 2kb + t (keys 32kb + 16*half + 8t + 0..7)
  const f32x16 zero16 = {};

  auto need_mask = [&](int t) {
    const int n0 = t * kBC;
    return (kMasked && n0 + kBC > s_kv) || (kCausal && n0 + kBC - 1 > wave_q_lo);
  };
  // Ragged S: keys past key_lim_h + 16*half are dead, past s_kv or (causal) past the query;
  // one limit per lane keeps the masked variants within their registers. Unmasked causal
  // kernels compare each key with the query row.
  const int key_lim_h = (kCausal ? min(q_row, s_kv - 1) : s_kv - 1) - 16 * half;
  auto apply_mask = [&](f32x16(&s)[2], int t) {
    if constexpr (kMasked) {
      const int rel = key_lim_h - t * kBC;  // element i of block kb is dead if 32kb + i > rel
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (32 * kb + i > rel) s[kb][i] = -INFINITY;
    } else {
      const int key0 = t * kBC + 16 * half;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (kCausal && key0 + 32 * kb + i > q_row) s[kb][i] = -INFINITY;
    }
  };
  // max op k (0..15) over the 32 scores of a lane: v_maximum3_f32 chains
  auto max_op = [&](const f32x16(&s)[2], int k, float& mx) {
    auto e = [&](int x) { return s[x >> 4][x & 15]; };
    if (k == 0) mx = max3f(e(0), e(1), e(2));
    else if (k < 15) mx = max3f(mx, e(1 + 2 * k), e(2 + 2 * k));
    else mx = __builtin_elementwise_maximum(mx, e(31));
  };
  auto rescale = [&]() {
    const bool raise = m_cur > m_run + kRescaleSlack;
    if (__builtin_amdgcn_ballot_w64(raise)) {
      const float alpha = raise ? __builtin_amdgcn_exp2f(m_run - m_cur) : 1.f;  // 0 on the first tile
      m_run = raise ? m_cur : m_run;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
    }
  };
  auto sm_elem = [&](f32x16(&s)[2], int e) {
    s[e >> 4][e & 15] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[e >> 4][e & 15], scale_log2, -m_run));
  };
  auto sm_pack = [&](const f32x16(&s)[2], int g) {
    const int kb = g >> 1, t = g & 1;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      pp[g][q] = H::pack2(s[kb][8 * t + 2 * q], s[kb][8 * t + 2 * q + 1]);
      l_run = H::sum2(pp[g][q], l_run);
    }
  };
  auto pv = [&](int i, u32x4 vf) {
    const int db = i % NDB;
    o[db] = H::mfma32(vf, pp[i / NDB], o[db]);
  };
  auto s_mfma = [&](f32x16(&s)[2], int i, u32x4 kf) {
    s[i & 1] = H::mfma32(kf, qf[i >> 1], i < 2 ? zero16 : s[i & 1]);
  };

  // One key tile. par = j & 1 (K(j+1) sits in K buffer par^1, V(j) in V buffer par);
  // kNext: tile j+1 exists, its S is computed here into sn.
  auto iteration = [&](int j, auto par_tag, auto next_tag, f32x16(&sc)[2], f32x16(&sn)[2]) {
    constexpr int par = decltype(par_tag)::value;
    constexpr bool kNext = decltype(next_tag)::value != 0;
    const bool copy_k2 = j + 2 < ntiles;  // K(j+2) exists (only if kNext)
    rescale();
    if constexpr (!kNext) {
      u32x4 vf[NP];
#pragma unroll
      for (int i = 0; i < NP; ++i) vf[i] = read_v(par, i);
#pragma unroll
      for (int e = 0; e < 32; ++e) {
        sm_elem(sc, e);
        if ((e & 7) == 7) sm_pack(sc, e >> 3);
      }
#pragma unroll
      for (int i = 0; i < NP; ++i) pv(i, vf[i]);
    } else {
      u32x4 kf[NS];
      u32x4 vf[NP];
#pragma unroll
      for (int i = 0; i < 3; ++i) kf[i] = read_k(par ^ 1, i);
      __builtin_amdgcn_sched_barrier(0);
      // block 1: S(j+1) MFMAs; softmax elements 0..23 of S(j)
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        s_mfma(sn, i, kf[i]);
        // this wave's 2*PW copies of K(j+2) and V(j+1), spread over the steps: a burst of
        // copies from all waves right after the barrier stalls their issue for hundreds of
        // cycles (the HBM/L2 -> LDS path moves about 64-80 bytes per clock per CU)
        constexpr int kGap = NS / (2 * PW);
        if (i % kGap == kGap - 1) {
          const int c = i / kGap;
          if (c < PW) {
            if (copy_k2) copy_piece(Kb, j + 2, lds0 + par * TB, false, c);
          } else {
            copy_piece(Vb, j + 1, lds0 + (2 + (par ^ 1)) * TB, true, c - PW);
          }
        }
        if (i + 3 < NS) kf[i + 3] = read_k(par ^ 1, i + 3);
        if (i == NS - 2) vf[0] = read_v(par, 0);
        if (i == NS - 1) vf[1] = read_v(par, 1);
        const int lo = 24 * i / NS, hi = 24 * (i + 1) / NS;
#pragma unroll
        for (int e = lo; e < hi; ++e) sm_elem(sc, e);
#pragma unroll
        for (int g = 0; g < 3; ++g)
          if (8 * (g + 1) > lo && 8 * (g + 1) <= hi) sm_pack(sc, g);
        __builtin_amdgcn_sched_barrier(0);
      }
      // block 2, first half: PV of key block 0; softmax elements 24..31
#pragma unroll
      for (int i = 0; i < 2 * NDB; ++i) {
        pv(i, vf[i]);
        vf[i + 2] = read_v(par, i + 2);
        const int lo = 24 + 8 * i / (2 * NDB), hi = 24 + 8 * (i + 1) / (2 * NDB);
#pragma unroll
        for (int e = lo; e < hi; ++e) sm_elem(sc, e);
        if (i == 2 * NDB - 1) sm_pack(sc, 3);
        __builtin_amdgcn_sched_barrier(0);
      }
      // block 2, second half: PV of key block 1; max of S(j+1)
      float mx = 0.f;
      if (!need_mask(j + 1)) {
#pragma unroll
        for (int i = 2 * NDB; i < NP; ++i) {
          pv(i, vf[i]);
          if (i + 2 < NP) vf[i + 2] = read_v(par, i + 2);
          const int r = i - 2 * NDB;
          const int lo = 16 * r / (2 * NDB), hi = 16 * (r + 1) / (2 * NDB);
#pragma unroll
          for (int k = lo; k < hi; ++k) max_op(sn, k, mx);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int i = 2 * NDB; i < NP; ++i) {
          pv(i, vf[i]);
          if (i + 2 < NP) vf[i + 2] = read_v(par, i + 2);
        }
        apply_mask(sn, j + 1);
#pragma unroll
        for (int k = 0; k < 16; ++k) max_op(sn, k, mx);
      }
      m_cur = halves_max(mx) * scale_log2;
      wait_and_barrier<0>();
    }
  };

  // ---- prologue: tiles 0 (K, V) and 1 (K); S(0) and its max ----
  copy_k(0, 0);
  copy_v(0, 0);
  if (ntiles > 1) copy_k(1, 1);
  wait_and_barrier<0>();
  f32x16 sa[2], sb[2];
  {
    u32x4 kf[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) kf[i] = read_k(0, i);
#pragma unroll
    for (int i = 0; i < NS; ++i) s_mfma(sa, i, kf[i]);
    if (need_mask(0)) apply_mask(sa, 0);
    float mx = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) max_op(sa, k, mx);
    m_cur = halves_max(mx) * scale_log2;
  }
  wait_and_barrier<0>();  // every wave is done with K(0) before K(2) replaces it

  int j = 0;
  for (; j + 2 < ntiles; j += 2) {
    iteration(j, Int<0>{}, Int<1>{}, sa, sb);
    iteration(j + 1, Int<1>{}, Int<1>{}, sb, sa);
  }
  if (j + 1 < ntiles) {
    iteration(j, Int<0>{}, Int<1>{}, sa, sb);
    iteration(j + 1, Int<1>{}, Int<0>{}, sb, sa);
  } else {
    iteration(j, Int<0>{}, Int<0>{}, sa, sb);
  }

  const float inv = 1.f / halves_sum(l_run);
  // masked variants take the output row and lane half from the lane id again: kept live
  // across the loop they would take registers the loop needs (the compiler cannot tie
  // __lane_id() to threadIdx.x)
  const int lane_out = kMasked ? (int)__lane_id() : lane;
  const int q_out = kMasked ? m0 + 32 * wave + (lane_out & 31) : q_row;
  const int half_out = kMasked ? lane_out >> 5 : half;
  if (!kMasked || q_out < s_q) {
    uint16_t* orow = Oh + (long long)q_out * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        // lane holds O^T[32db + 8jj + 4*half + r][q_row], r = 0..3
        u32x2 packed;
        packed[0] = H::pack2(o[db][4 * jj] * inv, o[db][4 * jj + 1] * inv);
        packed[1] = H::pack2(o[db][4 * jj + 2] * inv, o[db][4 * jj + 3] * inv);
        st8(orow + 32 * db + 8 * jj + 4 * half_out, packed);
      }
  }
}

inline bool fa_mfma_supported(const FaShape& s) {
  return (s.d == 64 || s.d == 128) && s.scale > 0.f && s.s_q >= 1 && s.s_kv >= 1 && (!s.causal || s.s_q == s.s_kv) &&
         (long long)((s.s_q + fa::Cfg<64>::kBM - 1) / fa::Cfg<64>::kBM) * s.bh < (1ll << 31);
}

template <typename Tag, int D, int W>
hipError_t launch_fa_fwd_mfma_dw(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, const FaShape& s,
                                 hipStream_t stream) {
  using C = fa::Cfg<D, W>;
  const int nmb = (s.s_q + C::kBM - 1) / C::kBM;
  const dim3 grid(nmb * s.bh);
  const bool masked = (s.s_q % C::kBM) != 0 || (s.s_kv % fa::kBC) != 0;
  const float scale_log2 = s.scale * 1.4426950408889634f;
#define KG_FA(CAUSAL, MASKED)                                                                                    \
  hipLaunchKernelGGL((fa_fwd_mfma_kernel<Tag, D, CAUSAL, MASKED, W>), grid, dim3(C::kThreads), 0, stream, q, k, v, o, \
                     s.bh, s.s_q, s.s_kv, scale_log2)
  if (s.causal) {
    if (masked) KG_FA(true, true); else KG_FA(true, false);
  } else {
    if (masked) KG_FA(false, true); else KG_FA(false, false);
  }
#undef KG_FA
  return hipGetLastError();
}

// Waves per workgroup the launch uses: D=128 drops to 4 when 8-wave workgroups would not
// give every CU of the MI355X (256) one.
inline int fa_mfma_waves(const FaShape& s) {
  if (s.d != 128) return fa::Cfg<64>::kWaves;
  const long long wg8 = (long long)s.bh * ((s.s_q + fa::Cfg<128, 8>::kBM - 1) / fa::Cfg<128, 8>::kBM);
  return wg8 < 256 ? 4 : 8;
}

template <typename Tag>
hipError_t launch_fa_fwd_mfma(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, const FaShape& s,
                              hipStream_t stream) {
  if (s.d == 128) {
    if (fa_mfma_waves(s) == 4) return launch_fa_fwd_mfma_dw<Tag, 128, 4>(q, k, v, o, s, stream);
    return launch_fa_fwd_mfma_dw<Tag, 128, 8>(q, k, v, o, s, stream);
  }
  return launch_fa_fwd_mfma_dw<Tag, 64, 4>(q, k, v, o, s, stream);
}

}  // namespace kg_gfx950
