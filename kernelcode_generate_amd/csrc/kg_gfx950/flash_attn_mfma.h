// Flash-attention forward on gfx950 MFMA: 16-bit Q/K/V/O [B,H,S,D], D in {64, 128},
// fp32 online softmax, optional scale and causal mask.
//
// Work split: a workgroup holds query rows of one (b,h), 32 per wave (Cfg<D>: 8 waves for
// D=128, 4 for D=64 and for D=128 grids too small to give every CU an 8-wave workgroup;
// two waves per SIMD either way; large non-causal grids run persistent workgroups, kPersist
// below). Key/value tiles of 64 keys are copied
// HBM -> LDS into rings of kStages buffers each for K and V (2 by default; 3 or 4 when the
// lowering's memory_stage asks for a deeper ring) and shared by the workgroup's waves. Workgroup
// ids are dealt to the 8 XCDs round-robin; they are remapped so that each XCD runs the query
// blocks of the same (b,h) together and its L2 serves their K/V.
//
// Matrix cores: v_mfma_f32_16x16x32 (16x16 blocks, 32-deep contraction; the same FLOP per
// cycle as 32x32x16, and under the part's power limit it holds a higher clock). A wave's 32
// queries are two query blocks qb (16 each), a key tile four key blocks kb (16 keys).
//   S^T = K Q^T: operand A = 16 keys x 32 d of K from LDS (lane l: key l%16, d 8(l/16)..+7),
//     operand B = Q^T kept in registers for the whole kernel (lane l: query l%16 of qb, the
//     same d). Each K fragment feeds the MFMAs of both query blocks. Lane l ends up with
//     S[query l%16 of qb][keys 16kb + 4(l/16) + 0..3] for every (qb, kb): 16 scores of each
//     of its two queries, so the row max combines the four lanes l%16 + 16r (three
//     v_permlane{16,32}_swap for both queries together).
//   O^T += V^T P^T over 32-key chunks c: the contraction index k = 8r + j of lane row r stands
//     for key 32c + 4r + j (j < 4) and 32c + 16 + 4r + j - 4 (j >= 4), exactly the keys whose
//     scores lane row r holds, so P (rounded to 16 bits) feeds operand B from its own
//     registers; operand A (lane l: d 16db + l%16, those 8 keys) is two ds_read_b64_tr_b16
//     from the key-major V tile: within each 16-lane group, lane j addresses 4 consecutive d
//     of key row j/4 and lane i receives key rows 0..3 of column i. Each V fragment feeds
//     both query blocks.
//
// Softmax works in base 2: p = exp2(s * scale*log2(e) - m) with m tracked in the same
// units (v_exp_f32). The running max is raised only when a tile's max exceeds it by more
// than kRescaleSlack, so the O rescale is skipped on most tiles; numerator and denominator
// use the same m, so the result does not depend on it. Row sums are one more MFMA per key
// chunk and query block, the chunk's P (rounded to 16 bits: the same values the PV product
// uses) against a fragment of ones, so every lane ends up with its query's whole sum and no
// lane combine is needed; against a chain of 16 dependent v_dot2c per tile this cut a C4
// iteration from 3644 to 3320 cycles (D=64 causal: equal), for 4 more MFMAs per wave and tile.
//
// Software pipeline per wave, tile j (S(j) computed and its max known on entry):
//   block 1: the S(j+1) MFMAs, with the exp/pack of 3/4 of S(j) and the K(j+1) fragment
//            reads slotted between them;
//   block 2: the PV(j) MFMAs, with the last quarter of softmax(j), the V(j) fragment reads
//            and the max of S(j+1) slotted between them.
// The copies of K(j+S) and V(j+S-1), S = kStages (into the buffers iteration j-1 finished
// with: K(j) and V(j-1)), are slotted between the block-1 MFMAs of iteration j; one wait +
// barrier ends the iteration. With two buffers it waits for every copy; with deeper rings
// only for the copies issued before this iteration (the next one needs K(j+2) and V(j+1),
// issued at least one iteration earlier), so a copy may take S-1 iterations to land.
//
// LDS chunk swizzles (16-byte chunks, 64 banks of 4 bytes; ds_read_b128 serves 16 lanes per
// cycle, 64-bit reads 32): K chunk c of key row r sits at slot c ^ k_mask(r) and V chunk c
// at c ^ v_mask(r). Each copy lane fetches the HBM chunk that belongs at its LDS slot.
#pragma once

#include <atomic>

#include "flash_attn.h"
#include "lds_dma.h"

namespace kg_gfx950 {

namespace fa {

constexpr int kBC = 64;  // keys per tile
constexpr int kDefaultStages = 2;  // K/V ring depth unless the lowering asks for another
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

// K fragment reads: the 16 lanes of a b128 read cycle read key rows 16kb + 0..15 at the same
// chunk. D=128 rows are 256 bytes (one bank row): slot c ^ (r & 15) puts them in 16 distinct
// chunks. D=64 rows are 128 bytes (two per bank row): rows of one parity need distinct
// chunks, c ^ ((r >> 1) & 7).
template <int D>
__host__ __device__ constexpr int k_mask(int key) {
  return D == 128 ? (key & 15) : ((key >> 1) & 7);
}
// V^T reads: the 32 lanes of a 64-bit read cycle read key rows 8i + 0..7, 32 contiguous bytes
// (chunks 2db, 2db+1) each. D=128: slot c ^ 2(r & 7) gives the 8 rows 8 distinct chunk
// pairs; D=64: rows of one parity (4 of them) distinct pairs, c ^ 2((r >> 1) & 3).
template <int D>
__host__ __device__ constexpr int v_mask(int key) {
  return D == 128 ? 2 * (key & 7) : 2 * ((key >> 1) & 3);
}

// The copy rows of one lane (kWaves * RPP apart, RPP = 1024 / (2D) rows per KiB) share
// their K and V masks.
template <int D, int W>
constexpr bool copy_masks_repeat() {
  constexpr int RPP = 1024 / (2 * D), PW = 64 * 2 * D / 1024 / W;
  for (int w = 0; w < W; ++w)
    for (int lane = 0; lane < 64; ++lane)
      for (int p = 0; p < PW; ++p) {
        const int r0 = w * RPP + lane / (D / 8), r = r0 + W * p * RPP;
        if (k_mask<D>(r) != k_mask<D>(r0) || v_mask<D>(r) != v_mask<D>(r0)) return false;
      }
  return true;
}
static_assert(copy_masks_repeat<128, 8>() && copy_masks_repeat<128, 4>() && copy_masks_repeat<64, 4>(),
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

// a and b combined over the four 16-lane rows (lanes with the same lane % 16), both results
// in every lane. v_permlane16_swap(x, y) swaps the odd rows of x with the even rows of y:
// it returns [x0 y0 x2 y2] and [x1 y1 x3 y3]; v_permlane32_swap(x, y) swaps the high half of
// x with the low half of y: with x = y it returns [x0 x1 x0 x1] and [x2 x3 x2 x3].
template <bool kMax>
__device__ __forceinline__ void rows4_combine(float& a, float& b) {
  auto op = [](float x, float y) { return kMax ? __builtin_elementwise_maximum(x, y) : x + y; };
  auto f = [](uint32_t u) { return __builtin_bit_cast(float, u); };
  const auto r1 = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                                   false, false);
  const uint32_t r10 = r1[0], r11 = r1[1];
  const float m = op(f(r10), f(r11));  // rows: a01 b01 a23 b23
  const uint32_t um = __builtin_bit_cast(uint32_t, m);
  const auto r2 = __builtin_amdgcn_permlane32_swap(um, um, false, false);
  const uint32_t r20 = r2[0], r21 = r2[1];
  const float t = op(f(r20), f(r21));  // rows: A B A B
  const uint32_t ut = __builtin_bit_cast(uint32_t, t);
  const auto r3 = __builtin_amdgcn_permlane16_swap(ut, ut, false, false);
  const uint32_t r30 = r3[0], r31 = r3[1];
  a = f(r30);
  b = f(r31);
}

// Whole query blocks: a wave packs its 32 output rows (o: O^T accumulators, lane holding
// O^T[16db + 4lr + i][query l16 of block qb]; inv: the row sums' inverses) into an LDS region of
// its own and writes them back as whole 2D-byte rows, 16 bytes per lane, with nontemporal
// stores, instead of 32-byte pieces of 16 rows (measured on C4: shorter launches, as for the
// GEMMs' C). 16-byte chunk c of region row r sits at slot c ^ (r % CPR): the packing writes of
// 16 rows at one chunk pair and the row reads both spread over the bank groups.
template <typename H, int D, int NDB>
__device__ __forceinline__ void write_rows(const f32x4 (&o)[NDB][2], const float (&inv)[2], uint32_t region, int lane,
                                           uint16_t* rows) {
  constexpr int RB = 2 * D;
  constexpr int CPR = RB / 16;  // 16-byte chunks per output row
  constexpr int RPI = 64 / CPR;  // rows per read instruction
  const int l16 = lane & 15, lr = lane >> 4;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      u32x2 packed;
      packed[0] = H::pack2(o[db][qb][0] * inv[qb], o[db][qb][1] * inv[qb]);
      packed[1] = H::pack2(o[db][qb][2] * inv[qb], o[db][qb][3] * inv[qb]);
      const int r = 16 * qb + l16;
      const int c = 2 * db + (lr >> 1);
      const uint32_t ad = region + r * RB + 16 * (c ^ (r & (CPR - 1))) + 8 * (lr & 1);
      *(__attribute__((address_space(3))) u32x2*)(uintptr_t)ad = packed;
    }
#pragma unroll
  for (int t = 0; t < 32 / RPI; ++t) {
    const int r = RPI * t + lane / CPR;
    const int c = lane % CPR;
    const u32x4 v = *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)(region + r * RB + 16 * (c ^ (r & (CPR - 1))));
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(rows + (long long)r * D + 8 * c));
  }
}

}  // namespace fa

// kPersist: a grid of kPerCU workgroups per CU walks the work items (query blocks) blockIdx.x,
// blockIdx.x + gridDim.x, ... as one sequence of key tiles: each wave copies its rows of the
// next item's Q into a staging region of its own during tiles nt-4 and nt-3 and reads them
// into its Q registers in tile nt-2, the next item's K tiles 0-1 and V tile 0 take the ring
// slots of the tiles that would follow this item's last, and the last tile's S MFMAs compute
// the next item's first S tile. An item boundary then costs only the output write, where a
// new workgroup waits for its launch and its first tiles (non-causal whole tiles, an even
// tile count of at least 4 and a two-deep ring).
template <typename Tag, int D, bool kCausal, bool kMasked, int W, int kStages, bool kPersist = false>
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
  constexpr int NDS = D / 32;        // 32-deep d steps of S^T
  constexpr int NKF = 4 * NDS;       // K fragments per tile: 4 key blocks x NDS
  constexpr int NS = 2 * NKF;        // S^T MFMAs per tile (both query blocks per fragment)
  constexpr int NDB = D / 16;        // 16-row d blocks of O^T
  constexpr int NVF = 2 * NDB;       // V^T fragments per tile: 2 key chunks x NDB
  constexpr int NP = 2 * NVF;        // PV MFMAs per tile
  constexpr int PW = TB / 1024 / kWaves;  // copy instructions per wave, tile and operand
  static_assert(PW >= 1 && 2 * PW <= NS, "copy slots");
  constexpr int RPP = 1024 / RB;     // rows per copy instruction
  constexpr int kKAhead = 3;         // K fragments read ahead of their MFMAs
  static_assert(kStages >= 2 && kStages <= 4, "K/V ring depth");
  static_assert(!kPersist || (!kCausal && !kMasked && kStages == 2), "persistent form: whole non-causal tiles");
  // persistent form: each wave's staging region of 32 rows follows the ring; it takes the
  // next item's Q rows, then this item's output rows (the ring holds the next item's first
  // tiles while the outputs leave)
  constexpr int kStagingBytes = kPersist ? kWaves * 32 * RB : 0;

  __shared__ __attribute__((aligned(1024))) u32x4 lds[(2 * kStages * TB + kStagingBytes) / 16];  // K ring, V ring, staging

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15;
  const int lr = lane >> 4;  // lane row (16 lanes)

  const int nmb = (s_q + kBM - 1) / kBM;
  const int items = nmb * bh_count;
  int item = blockIdx.x;  // work item (query block): the workgroup id, or for kPersist the first
  if (kPersist && item >= items) return;  // (the launcher gives every workgroup at least two)
  const int lin = xcd_block(item, items);
  const int bh = lin / nmb;
  int mb = lin - bh * nmb;
  if (kCausal) mb = nmb - 1 - mb;  // longest query blocks of a (b,h) first
  int m0 = mb * kBM;
  const long long kv_base = (long long)bh * s_kv * D;
  const uint16_t* Qh = Q + (long long)bh * s_q * D;
  const char* Kb = reinterpret_cast<const char*>(K + kv_base);
  const char* Vb = reinterpret_cast<const char*>(V + kv_base);
  uint16_t* Oh = O + (long long)bh * s_q * D;
  // the next item of a persistent workgroup (has_next false: none, or not persistent; the
  // persistent form is non-causal, so query blocks keep their order). Only the persistent
  // form's copies and Q staging read these; the masks and the masked epilogue use
  // wave_q_lo / q_row0 below, which stay those of the first item.
  bool has_next = false;
  int m0_next = 0;
  const uint16_t* Qn = Q;
  const char* Kn = nullptr;
  const char* Vn = nullptr;
  uint16_t* On = O;
  auto find_next = [&]() {
    const int it = item + (int)gridDim.x;
    has_next = it < items;
    if (has_next) {
      const int lin_n = xcd_block(it, items);
      const long long bhn = lin_n / nmb;
      m0_next = (lin_n - (int)bhn * nmb) * kBM;
      Qn = Q + bhn * s_q * D;
      Kn = reinterpret_cast<const char*>(K + bhn * s_kv * D);
      Vn = reinterpret_cast<const char*>(V + bhn * s_kv * D);
      On = O + bhn * s_q * D;
    }
  };
  if constexpr (kPersist) find_next();

  const int wave_q_lo = m0 + 32 * wave;
  const int q_row0 = wave_q_lo + l16;  // query of block qb: q_row0 + 16 qb
  u32x4 qf[2][NDS];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int s = 0; s < NDS; ++s) {
      const int q = q_row0 + 16 * qb;
      qf[qb][s] = (!kMasked || q < s_q) ? ld16(Qh + (long long)q * D + 32 * s + 8 * lr) : u32x4{0, 0, 0, 0};
    }

  const int n_end = kCausal ? min(s_kv, m0 + kBM) : s_kv;
  const int ntiles = (n_end + kBC - 1) / kBC;

  // ---- HBM -> LDS copies: K tile t into K buffer b (LDS bytes b*TB), V into (kStages+b)*TB ----
  // Copy instruction p of wave w covers the KiB (w + kWaves*p) of the tile: rows
  // (w + kWaves*p)*RPP + lane/DCH, LDS slot lane%DCH. The rows of one lane's copies lie
  // kWaves*RPP (at least 32) rows apart, so they share their K and V masks: one per-lane
  // offset each, and p moves the wave-uniform source base by whole KiB.
  const uint32_t lds0 = lds_addr(&lds[0]);
  const int c_row0 = wave * RPP + lane / DCH;
  const int c_slot = lane % DCH;
  const uint32_t k_goff = (uint32_t)(c_row0 * RB + 16 * (c_slot ^ k_mask<D>(c_row0)));
  const uint32_t v_goff = (uint32_t)(c_row0 * RB + 16 * (c_slot ^ v_mask<D>(c_row0)));

  // Copy instruction p (< PW) of tile t of K (kV false) or V into the LDS buffer at lds_buf.
  auto copy_piece = [&](const char* src, int t, uint32_t lds_buf, bool kV, int p) {
    const int n0 = t * kBC;
    const uint32_t m = lds_buf + (wave + kWaves * p) * 1024;
    const char* base = src + (long long)n0 * RB + kWaves * p * 1024;
    if constexpr (kMasked) {
      // ragged S: every tile through a raw buffer resource that ends at row s_kv, so the rows
      // of the tail tile past s_kv land zeros (their scores are masked in S: P is 0 there)
      const long long left = (long long)(s_kv - n0) * RB - kWaves * p * 1024;
      const uint32_t range = (uint32_t)max(0ll, min(left, (long long)TB));
      buf2lds16_r(kV ? v_goff : k_goff, base, range, m);
    } else {
      g2lds16_s(kV ? v_goff : k_goff, base, m);
    }
  };
  auto copy_k = [&](int t, int buf) {
#pragma unroll
    for (int p = 0; p < PW; ++p) copy_piece(Kb, t, lds0 + buf * TB, false, p);
  };
  auto copy_v = [&](int t, int buf) {
#pragma unroll
    for (int p = 0; p < PW; ++p) copy_piece(Vb, t, lds0 + (kStages + buf) * TB, true, p);
  };
  // Persistent form: this wave's 32 rows of the next item's Q into its staging region (after
  // the ring), laid out like a K tile (chunk c of row r at slot c ^ k_mask(r)), so that the Q
  // fragments are read at the K fragment offsets; QPW copies of RPP rows. The lane id is taken
  // afresh: offsets derived from a value that lives through the item loop would be hoisted out
  // of it and held in registers across the main loop.
  constexpr int QPW = 32 * RB / 1024;
  const uint32_t q_stage = lds0 + 2 * kStages * TB + wave * 32 * RB;
  auto copy_q = [&](int p) {
    const int ln = lane_id_volatile();
    const int row = p * RPP + ln / DCH;
    const uint32_t voff = (uint32_t)(row * RB + 16 * ((ln % DCH) ^ k_mask<D>(row)));
    g2lds16_s(voff, reinterpret_cast<const char*>(Qn + (long long)(m0_next + 32 * wave) * D), q_stage + p * 1024);
  };

  // ---- fragment reads ----
  // K fragment f = kb*NDS + s: key row 16kb + l16, chunk 4s + lr; k_mask(16kb + l16) ==
  // k_mask(l16), so kb is an immediate offset.
  uint32_t k_rd[NDS];
  {
    const int km = k_mask<D>(l16);
#pragma unroll
    for (int s = 0; s < NDS; ++s) k_rd[s] = lds0 + l16 * RB + 16 * ((4 * s + lr) ^ km);
  }
  // V^T fragment f = c*NDB + db: lane row lr reads key rows 32c + 4lr + {0..3} (then +16) and
  // d columns 16db .. 16db+15, lane j of the row addressing row j/4 and d 4(j%4) .. +3.
  // v_mask of those rows equals that of row 4lr + j/4, so c and the +16 are immediate offsets.
  uint32_t v_rd[NDB];
  {
    const int row = 4 * lr + (l16 >> 2);
    const int vm = v_mask<D>(row);
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int c16 = 2 * db + ((l16 & 3) >> 1);
      v_rd[db] = lds0 + kStages * TB + row * RB + 16 * (c16 ^ vm) + 8 * (l16 & 1);
    }
  }
  // boff: the byte offset of the tile's ring buffer (buffer index x TB)
  auto read_k = [&](uint32_t boff, int f) -> u32x4 {
    const int kb = f / NDS, s = f % NDS;
    return *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)(k_rd[s] + boff + kb * 16 * RB);
  };
  // Q fragment (query block qb, d step s) of the staged next item: row 16qb + l16, chunk 4s + lr,
  // whose slot is the K fragment's (k_mask(16qb + l16) == k_mask(l16))
  auto read_q = [&](int qb, int s) -> u32x4 {
    return *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)(k_rd[s] + (q_stage - lds0) + qb * 16 * RB);
  };
  auto read_v = [&](uint32_t boff, int f) -> u32x4 {
    const int c = f / NDB, db = f % NDB;
    const uint32_t a = v_rd[db] + boff + 32 * c * RB;
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(uintptr_t)a);
    const s16x4 hi =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(uintptr_t)(a + 16 * RB));
    const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
    return u32x4{l2[0], l2[1], h2[0], h2[1]};
  };

  // ---- softmax state (per query block) ----
  f32x4 o[NDB][2];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) o[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {-INFINITY, -INFINITY};  // max used by exp2 (log2 units)
  f32x4 l_run[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};  // row sums (each element: the query's)
  const u32x4 ones = {H::kOnePair, H::kOnePair, H::kOnePair, H::kOnePair};
  float m_cur[2] = {-INFINITY, -INFINITY};  // max of the S tile about to be exponentiated
  u32x4 pp[2][2];                           // P of chunk c, query block qb (keys as above)
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
  using Scores = f32x4[2][4];               // [qb][kb], lane holds keys 16kb + 4lr + 0..3

  auto need_mask = [&](int t) {
    const int n0 = t * kBC;
    return (kMasked && n0 + kBC > s_kv) || (kCausal && n0 + kBC - 1 > wave_q_lo);
  };
  // Ragged S: a score of query block qb and tile-relative key 16kb + 4lr + i is dead if
  // 16kb + i > key_lim[qb] - t*kBC (keys past s_kv or, causal, past the query). Unmasked
  // causal kernels compare each key with the query row.
  auto apply_mask = [&](Scores& s, int t) {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int q = q_row0 + 16 * qb;
      if constexpr (kMasked) {
        const int rel = (kCausal ? min(q, s_kv - 1) : s_kv - 1) - 4 * lr - t * kBC;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (16 * kb + i > rel) s[qb][kb][i] = -INFINITY;
      } else {
        const int key0 = t * kBC + 4 * lr;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (kCausal && key0 + 16 * kb + i > q) s[qb][kb][i] = -INFINITY;
      }
    }
  };
  // max op k (0..7) over the 16 scores of query block qb: v_maximum3_f32 chains
  auto max_op = [&](const Scores& s, int qb, int k, float& mx) {
    auto e = [&](int x) { return s[qb][x >> 2][x & 3]; };
    if (k == 0) mx = max3f(e(0), e(1), e(2));
    else if (k < 7) mx = max3f(mx, e(1 + 2 * k), e(2 + 2 * k));
    else mx = __builtin_elementwise_maximum(mx, e(15));
  };
  auto tile_max = [&](float (&mx)[2]) {
    rows4_combine<true>(mx[0], mx[1]);
    m_cur[0] = mx[0] * scale_log2;
    m_cur[1] = mx[1] * scale_log2;
  };
  // kAlways: scale without the wave-uniform branch (alpha 1 where nothing is raised)
  auto rescale = [&](auto always_tag) {
    constexpr bool kAlways = decltype(always_tag)::value != 0;
    const bool raise0 = m_cur[0] > m_run[0] + kRescaleSlack;
    const bool raise1 = m_cur[1] > m_run[1] + kRescaleSlack;
    if (kAlways || __builtin_amdgcn_ballot_w64(raise0 || raise1)) {
      // alpha is 0 on the first tile (m_run = -inf)
      const float a0 = raise0 ? __builtin_amdgcn_exp2f(m_run[0] - m_cur[0]) : 1.f;
      const float a1 = raise1 ? __builtin_amdgcn_exp2f(m_run[1] - m_cur[1]) : 1.f;
      m_run[0] = raise0 ? m_cur[0] : m_run[0];
      m_run[1] = raise1 ? m_cur[1] : m_run[1];
      l_run[0] *= a0;
      l_run[1] *= a1;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        o[db][0] *= a0;
        o[db][1] *= a1;
      }
    }
  };
  // softmax element e (0..31): pack group G = e/8 = 2c + qb, in the order the PV MFMAs use
  // them (chunk 0 of both query blocks first); within a group, kb = 2c + (e/4)%2, i = e%4
  auto sm_elem = [&](Scores& s, int e) {
    const int G = e >> 3, c = G >> 1, qb = G & 1, kb = 2 * c + ((e >> 2) & 1), i = e & 3;
    s[qb][kb][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qb][kb][i], scale_log2, -m_run[qb]));
  };
  auto sm_pack = [&](const Scores& s, int G) {
    const int c = G >> 1, qb = G & 1;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        pp[c][qb][2 * h + q] = H::pack2(s[qb][2 * c + h][2 * q], s[qb][2 * c + h][2 * q + 1]);
      }
  };
  // PV MFMA i: V fragment i/2 (chunk c, d block db), query block i%2
  auto pv = [&](int i, u32x4 vf) {
    const int f = i >> 1, qb = i & 1;
    const int c = f / NDB, db = f % NDB;
    o[db][qb] = H::mfma16(vf, pp[c][qb], o[db][qb]);
    if (db == NDB - 1) l_run[qb] = H::mfma16(ones, pp[c][qb], l_run[qb]);  // the chunk's row sums
  };
  // S MFMA i: K fragment i/2 (key block kb, d step s), query block i%2
  auto s_mfma = [&](Scores& s, int i, u32x4 kf) {
    const int f = i >> 1, qb = i & 1;
    const int kb = f / NDS, st = f % NDS;
    s[qb][kb] = H::mfma16(kf, qf[qb][st], st == 0 ? zero4 : s[qb][kb]);
  };

  // One key tile. par = j & 1 selects the score registers (and, with two buffers, the ring
  // buffers as immediates: K(j+1) sits in K buffer par^1, V(j) in V buffer par; deeper rings
  // take tile t's buffer t % kStages); kNext: tile j+1 exists, its S is computed here into sn.
  // kTail: the iterations after the loop, which rescale without a branch (a branch there
  // leaves the compiler short of registers where its two paths meet)
  auto iteration = [&](int j, auto par_tag, auto next_tag, Scores& sc, Scores& sn, auto tail_tag) {
    constexpr int par = decltype(par_tag)::value;
    constexpr bool kNext = decltype(next_tag)::value != 0;
    // tail_tag: 0 main loop, 1 the last two tiles, 2 (persistent form) tiles nt-4 and nt-3
    constexpr bool kTailIt = decltype(tail_tag)::value == 1;
    constexpr bool kQStage = kPersist && decltype(tail_tag)::value == 2;
    const bool copy_k2 = j + kStages < ntiles;      // K(j+S) exists (only if kNext)
    const bool copy_v1 = kStages == 2 || j + kStages - 1 < ntiles;  // V(j+S-1) exists
    // ring buffers: with two they are immediates; deeper rings keep the fragment addresses
    // k_rd / v_rd on K(j+1)'s and V(j)'s buffers (advanced at the end of each iteration),
    // and only the copies' destinations (wave-uniform) are computed here
    const uint32_t kb_next = kStages == 2 ? (par ^ 1) * TB : 0;                    // K(j+1)
    const uint32_t kb_copy = (kStages == 2 ? par : j % kStages) * TB;              // K(j+S): where K(j) was
    const uint32_t vb_cur = kStages == 2 ? par * TB : 0;                            // V(j)
    const uint32_t vb_copy = (kStages == 2 ? (par ^ 1) : (j + kStages - 1) % kStages) * TB;  // V(j+S-1)
    rescale(tail_tag);
    if constexpr (!kNext) {
      // last tile: the first two V fragments are read under the softmax, the rest two
      // fragments ahead of their MFMAs (all 16 at once would not fit the registers)
      u32x4 vf[NVF];
      vf[0] = read_v(vb_cur, 0);
      vf[1] = read_v(vb_cur, 1);
#pragma unroll
      for (int e = 0; e < 32; ++e) {
        sm_elem(sc, e);
        if ((e & 7) == 7) sm_pack(sc, e >> 3);
      }
#pragma unroll
      for (int i = 0; i < NP; ++i) {
        pv(i, vf[i >> 1]);
        if ((i & 1) == 0 && (i >> 1) + 2 < NVF) vf[(i >> 1) + 2] = read_v(vb_cur, (i >> 1) + 2);
      }
    } else {
      u32x4 kf[NKF];
      u32x4 vf[NVF];
#pragma unroll
      for (int f = 0; f < kKAhead; ++f) kf[f] = read_k(kb_next, f);
      __builtin_amdgcn_sched_barrier(0);
      // block 1: S(j+1) MFMAs; softmax elements 0..23 of S(j)
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        s_mfma(sn, i, kf[i >> 1]);
        // this wave's 2*PW copies of K(j+S) and V(j+S-1), spread over the steps: a burst of
        // copies from all waves right after the barrier stalls their issue for hundreds of
        // cycles (the HBM/L2 -> LDS path moves about 64-80 bytes per clock per CU)
        constexpr int kGap = NS / (2 * PW);
        if (i % kGap == kGap - 1) {
          const int c = i / kGap;
          if (c < PW) {
            if constexpr (kPersist && kTailIt) {
              // the last two tiles copy the next item's K tiles 0 and 1, into the buffers of
              // their position in the sequence of tiles (the tile count is even)
              if (has_next) copy_piece(Kn, par, lds0 + kb_copy, false, c);
            } else {
              if (copy_k2) copy_piece(Kb, j + kStages, lds0 + kb_copy, false, c);
            }
          } else {
            if constexpr (kPersist && kTailIt && par == 1) {
              copy_piece(Vn, 0, lds0 + kStages * TB + vb_copy, true, c - PW);  // (a next item exists here)
            } else {
              if (copy_v1) copy_piece(Vb, j + kStages - 1, lds0 + kStages * TB + vb_copy, true, c - PW);
            }
          }
        }
        if constexpr (kQStage) {
          // tiles nt-4 and nt-3 copy this wave's rows of the next item's Q into its staging
          // region, half in each
          if (i % kGap == kGap / 2 - 1 && i / kGap < QPW / 2 && has_next) copy_q(par * (QPW / 2) + i / kGap);
        }
        if ((i & 1) == 0 && (i >> 1) + kKAhead < NKF) kf[(i >> 1) + kKAhead] = read_k(kb_next, (i >> 1) + kKAhead);
        if (i == NS - 2) vf[0] = read_v(vb_cur, 0);
        if (i == NS - 1) vf[1] = read_v(vb_cur, 1);
        const int lo = 24 * i / NS, hi = 24 * (i + 1) / NS;
#pragma unroll
        for (int e = lo; e < hi; ++e) sm_elem(sc, e);
#pragma unroll
        for (int G = 0; G < 3; ++G)
          if (8 * (G + 1) > lo && 8 * (G + 1) <= hi) sm_pack(sc, G);
        __builtin_amdgcn_sched_barrier(0);
      }
      // block 2, first half: PV of key chunk 0; softmax elements 24..31
#pragma unroll
      for (int i = 0; i < NP / 2; ++i) {
        pv(i, vf[i >> 1]);
        if ((i & 1) == 0) vf[(i >> 1) + 2] = read_v(vb_cur, (i >> 1) + 2);
        if constexpr (kPersist && kTailIt && par == 0) {
          // the second-to-last tile is done with Q after block 1: the next item's Q comes in
          // from the staging region (unconditionally: without a next item it is not used)
          static_assert(2 * NDS <= NP / 4, "Q read slots");
          if ((i & 1) == 1 && (i >> 1) < 2 * NDS) qf[(i >> 1) / NDS][(i >> 1) % NDS] = read_q((i >> 1) / NDS, (i >> 1) % NDS);
        }
        const int lo = 24 + 8 * i / (NP / 2), hi = 24 + 8 * (i + 1) / (NP / 2);
#pragma unroll
        for (int e = lo; e < hi; ++e) sm_elem(sc, e);
        if (i == NP / 2 - 1) sm_pack(sc, 3);
        __builtin_amdgcn_sched_barrier(0);
      }
      // block 2, second half: PV of key chunk 1; max of S(j+1)
      float mx[2] = {0.f, 0.f};
      if (!need_mask(j + 1)) {
#pragma unroll
        for (int i = NP / 2; i < NP; ++i) {
          pv(i, vf[i >> 1]);
          if ((i & 1) == 0 && (i >> 1) + 2 < NVF) vf[(i >> 1) + 2] = read_v(vb_cur, (i >> 1) + 2);
          const int r = i - NP / 2;
          const int lo = 16 * r / (NP / 2), hi = 16 * (r + 1) / (NP / 2);
#pragma unroll
          for (int k = lo; k < hi; ++k) max_op(sn, k >> 3, k & 7, mx[k >> 3]);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int i = NP / 2; i < NP; ++i) {
          pv(i, vf[i >> 1]);
          if ((i & 1) == 0 && (i >> 1) + 2 < NVF) vf[(i >> 1) + 2] = read_v(vb_cur, (i >> 1) + 2);
        }
        apply_mask(sn, j + 1);
#pragma unroll
        for (int k = 0; k < 16; ++k) max_op(sn, k >> 3, k & 7, mx[k >> 3]);
      }
      tile_max(mx);
      if constexpr (kStages != 2) {
        // next iteration reads K(j+2) and V(j+1): one buffer on, wrapping at the ring's end
        const uint32_t k_step = (j + 2) % kStages == 0 ? (uint32_t)(-(kStages - 1) * TB) : (uint32_t)TB;
        const uint32_t v_step = (j + 1) % kStages == 0 ? (uint32_t)(-(kStages - 1) * TB) : (uint32_t)TB;
#pragma unroll
        for (int s = 0; s < NDS; ++s) k_rd[s] += k_step;
#pragma unroll
        for (int db = 0; db < NDB; ++db) v_rd[db] += v_step;
      }
      if constexpr (kStages == 2) {
        wait_and_barrier<0>();
      } else {
        // leave this iteration's copies in flight: every older one has landed after this
        if (copy_k2 && copy_v1) wait_and_barrier<2 * PW>();
        else if (copy_k2 || copy_v1) wait_and_barrier<PW>();
        else wait_and_barrier<0>();
      }
    }
  };

  // ---- prologue: K tiles 0..S-1 and V tiles 0..S-2 (those that exist); S(0) and its max ----
#pragma unroll
  for (int t = 0; t < kStages; ++t) {
    if (t < ntiles) copy_k(t, t);
    if (t < kStages - 1 && t < ntiles) copy_v(t, t);
  }
  wait_and_barrier<0>();
  Scores sa, sb;
  {
    u32x4 kf[NKF];
#pragma unroll
    for (int f = 0; f < NKF; ++f) kf[f] = read_k(0, f);
#pragma unroll
    for (int i = 0; i < NS; ++i) s_mfma(sa, i, kf[i >> 1]);
    if (need_mask(0)) apply_mask(sa, 0);
    float mx[2] = {0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 16; ++k) max_op(sa, k >> 3, k & 7, mx[k >> 3]);
    tile_max(mx);
  }
  if constexpr (kStages != 2) {
#pragma unroll
    for (int s = 0; s < NDS; ++s) k_rd[s] += TB;  // iteration 0 reads K(1) from buffer 1
  }
  wait_and_barrier<0>();  // every wave is done with K(0) before K(S) replaces it

  if constexpr (kPersist) {
    for (;;) {  // work items
      int j = 0;
      for (; j + 4 < ntiles; j += 2) {
        iteration(j, Int<0>{}, Int<1>{}, sa, sb, Int<0>{});
        iteration(j + 1, Int<1>{}, Int<1>{}, sb, sa, Int<0>{});
      }
      // An even tile count of at least 4: tiles nt-4 and nt-3 stage the next item's Q, then
      // the last two. With a next item the last one runs as a middle tile of one sequence of
      // tiles: its S MFMAs compute the next item's first S tile (into sa, with the Q read from
      // the staging region in the tile before) and its copies bring the next item's K tile 1
      // and V tile 0, so the next item starts at its first iteration once this one's outputs
      // are written.
      iteration(j, Int<0>{}, Int<1>{}, sa, sb, Int<2>{});
      iteration(j + 1, Int<1>{}, Int<1>{}, sb, sa, Int<2>{});
      j += 2;
      iteration(j, Int<0>{}, Int<1>{}, sa, sb, Int<1>{});
      if (!has_next) break;
      iteration(j + 1, Int<1>{}, Int<1>{}, sb, sa, Int<1>{});
      {
        // the lane id afresh (see copy_q); the staging region is free again (the Q read of
        // the tile before has completed: LDS ops of one wave complete in order)
        const float inv[2] = {1.f / l_run[0][0], 1.f / l_run[1][0]};
        fa::write_rows<H, D>(o, inv, q_stage, lane_id_volatile(), Oh + (long long)(m0 + 32 * wave) * D);
      }
      item += (int)gridDim.x;
      m0 = m0_next;
      Kb = Kn;
      Vb = Vn;
      Oh = On;
      find_next();
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) o[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
      m_run[0] = m_run[1] = -INFINITY;
      l_run[0] = l_run[1] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    iteration(ntiles - 1, Int<1>{}, Int<0>{}, sb, sa, Int<1>{});
    const float inv[2] = {1.f / l_run[0][0], 1.f / l_run[1][0]};
    fa::write_rows<H, D>(o, inv, q_stage, lane_id_volatile(), Oh + (long long)(m0 + 32 * wave) * D);
    return;
  }

  int j = 0;
  for (; j + 2 < ntiles; j += 2) {
    iteration(j, Int<0>{}, Int<1>{}, sa, sb, Int<0>{});
    iteration(j + 1, Int<1>{}, Int<1>{}, sb, sa, Int<0>{});
  }
  if (j + 1 < ntiles) {
    iteration(j, Int<0>{}, Int<1>{}, sa, sb, Int<1>{});
    iteration(j + 1, Int<1>{}, Int<0>{}, sb, sa, Int<1>{});
  } else {
    iteration(j, Int<0>{}, Int<0>{}, sa, sb, Int<1>{});
  }

  const float inv[2] = {1.f / l_run[0][0], 1.f / l_run[1][0]};
  if constexpr (!kMasked) {
    // Whole query blocks: fa::write_rows's packing and row stores, written out here (the call
    // changed the register allocation of these kernels), through the wave's part of the K/V
    // ring (free once every wave is past its last fragment read).
    constexpr int CPR = RB / 16;       // 16-byte chunks per output row
    constexpr int RPI = 64 / CPR;      // rows per read instruction
    static_assert(kWaves * 32 * RB <= 2 * kStages * TB, "the output regions fit in the ring");
    wait_and_barrier<0>();
    const uint32_t region = lds0 + wave * 32 * RB;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        // lane holds O^T[16db + 4lr + i][q], i = 0..3
        u32x2 packed;
        packed[0] = H::pack2(o[db][qb][0] * inv[qb], o[db][qb][1] * inv[qb]);
        packed[1] = H::pack2(o[db][qb][2] * inv[qb], o[db][qb][3] * inv[qb]);
        const int r = 16 * qb + l16;
        const int c = 2 * db + (lr >> 1);
        const uint32_t ad = region + r * RB + 16 * (c ^ (r & (CPR - 1))) + 8 * (lr & 1);
        *(__attribute__((address_space(3))) u32x2*)(uintptr_t)ad = packed;
      }
#pragma unroll
    for (int t = 0; t < 32 / RPI; ++t) {
      const int r = RPI * t + lane / CPR;
      const int c = lane % CPR;
      const u32x4 v = *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)(region + r * RB + 16 * (c ^ (r & (CPR - 1))));
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(Oh + (long long)(m0 + 32 * wave + r) * D + 8 * c));
    }
    return;
  }
  // masked variants take the output rows and lane row from the lane id again: kept live
  // across the loop they would take registers the loop needs (the compiler cannot tie
  // __lane_id() to threadIdx.x)
  const int lane_out = kMasked ? (int)__lane_id() : lane;
  const int q_out0 = kMasked ? m0 + 32 * wave + (lane_out & 15) : q_row0;
  const int lr_out = kMasked ? lane_out >> 4 : lr;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int q = q_out0 + 16 * qb;
    if (!kMasked || q < s_q) {
      uint16_t* orow = Oh + (long long)q * D;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        // lane holds O^T[16db + 4lr + i][q], i = 0..3
        u32x2 packed;
        packed[0] = H::pack2(o[db][qb][0] * inv[qb], o[db][qb][1] * inv[qb]);
        packed[1] = H::pack2(o[db][qb][2] * inv[qb], o[db][qb][3] * inv[qb]);
        st8(orow + 16 * db + 4 * lr_out, packed);
      }
    }
  }
}

inline bool fa_mfma_supported(const FaShape& s) {
  return (s.d == 64 || s.d == 128) && s.scale > 0.f && s.s_q >= 1 && s.s_kv >= 1 && (!s.causal || s.s_q == s.s_kv) &&
         (long long)((s.s_q + fa::Cfg<64>::kBM - 1) / fa::Cfg<64>::kBM) * s.bh < (1ll << 31);
}

// Compute units of the current device, read once per device.
inline int fa_device_cus() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 0;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// The persistent form (kPerCU workgroups per CU for `slots` workgroups in all). Compiled in a
// translation unit of its own: next to the other instantiations it changed their register
// allocation (spills in the causal D=128 kernels).
template <typename Tag, int D, int W>
hipError_t launch_fa_fwd_mfma_persist(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o,
                                      const FaShape& s, int slots, hipStream_t stream) {
  hipLaunchKernelGGL((fa_fwd_mfma_kernel<Tag, D, false, false, W, 2, true>), dim3(slots), dim3(fa::Cfg<D, W>::kThreads),
                     0, stream, q, k, v, o, s.bh, s.s_q, s.s_kv, s.scale * 1.4426950408889634f);
  return hipGetLastError();
}

template <typename Tag, int D, int W, int kStages>
hipError_t launch_fa_fwd_mfma_dw(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, const FaShape& s,
                                 hipStream_t stream) {
  using C = fa::Cfg<D, W>;
  const int nmb = (s.s_q + C::kBM - 1) / C::kBM;
  const dim3 grid(nmb * s.bh);
  const bool masked = (s.s_q % C::kBM) != 0 || (s.s_kv % fa::kBC) != 0;
  const float scale_log2 = s.scale * 1.4426950408889634f;
  if constexpr (kStages == 2 && (D == 64 || W == 8)) {
    // Non-causal whole tiles, an even tile count of at least 4 and at least two items per
    // workgroup slot: the persistent form, kPerCU workgroups per CU (a multiple of the 8
    // XCDs, so an item's XCD is its workgroup's).
    const long long items = (long long)nmb * s.bh;
    const int slots = fa_device_cus() * C::kPerCU / 8 * 8;
    const int ntiles = s.s_kv / fa::kBC;
    if (!s.causal && !masked && ntiles % 2 == 0 && ntiles >= 4 && slots >= 8 && items >= 2ll * slots)
      return launch_fa_fwd_mfma_persist<Tag, D, W>(q, k, v, o, s, slots, stream);
  }
#define KG_FA(CAUSAL, MASKED)                                                                                    \
  hipLaunchKernelGGL((fa_fwd_mfma_kernel<Tag, D, CAUSAL, MASKED, W, kStages>), grid, dim3(C::kThreads), 0, stream, q, k, v, o, \
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

template <typename Tag, int kStages>
hipError_t launch_fa_fwd_mfma_st(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, const FaShape& s,
                                 hipStream_t stream) {
  if (s.d == 128) {
    if (fa_mfma_waves(s) == 4) return launch_fa_fwd_mfma_dw<Tag, 128, 4, kStages>(q, k, v, o, s, stream);
    return launch_fa_fwd_mfma_dw<Tag, 128, 8, kStages>(q, k, v, o, s, stream);
  }
  return launch_fa_fwd_mfma_dw<Tag, 64, 4, kStages>(q, k, v, o, s, stream);
}

// stages: the K/V ring depth (2, 3 or 4)
template <typename Tag>
hipError_t launch_fa_fwd_mfma(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, const FaShape& s,
                              hipStream_t stream, int stages = fa::kDefaultStages) {
  if (stages == 3) return launch_fa_fwd_mfma_st<Tag, 3>(q, k, v, o, s, stream);
  if (stages == 4) return launch_fa_fwd_mfma_st<Tag, 4>(q, k, v, o, s, stream);
  return launch_fa_fwd_mfma_st<Tag, 2>(q, k, v, o, s, stream);
}

}  // namespace kg_gfx950
