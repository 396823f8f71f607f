// extern "C" entry points of libkg_gfx950.so (declared in include/kg_gfx950.h).
//
// Each entry validates the reference's slot contract (kind, rank, dtype, shape
// consistency; kernel_gen/execute_engine/builtin_strategy/common.py:925-931 returns -1 on
// any mismatch), picks the gfx950 kernel for the dtype/shape, launches it on the
// configured stream and, in the default synchronous mode, waits for it.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <vector>

#include "kg_gfx950.h"
#include "kg_gfx950/common.h"
#include "kg_gfx950/conv2d.h"
#include "kg_gfx950/flash_attn.h"
#include "kg_gfx950/gemm.h"
#include "kg_gfx950/gemm_f32.h"
#include "kg_gfx950/conv2d_mfma.h"
#include "kg_gfx950/conv2d_igemm.h"
#include "kg_gfx950/conv2d_rowvec.h"
#include "kg_gfx950/flash_attn_mfma.h"
#include "kg_gfx950/flash_attn_f32.h"
#include "kg_gfx950/instances.h"  // the heavy kernel families are compiled in their own translation units

namespace {

using namespace kg_gfx950;

constexpr int kOk = 0;
constexpr int kInvalid = -1;
constexpr int kHipFailure = -2;
constexpr int kUnsupported = -3;

// Per-thread state: the last failure text and the launch mode. Two host threads calling
// the entries concurrently (ctypes releases the GIL) each keep their own mode and stream,
// so a synchronous caller never has its kernel moved onto another thread's stream.
thread_local char g_last_error[512] = "";
thread_local bool g_synchronous = true;
thread_local hipStream_t g_stream = nullptr;

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int finish_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(kHipFailure, "%s: launch failed: %s", what, hipGetErrorString(err));
  if (g_synchronous) {
    err = hipStreamSynchronize(g_stream);
    if (err != hipSuccess) return fail(kHipFailure, "%s: hip_runtime_failed: %s", what, hipGetErrorString(err));
  }
  g_last_error[0] = '\0';
  return kOk;
}

// Cost queries (kg_gfx950_cost) run the entries' validation and dispatch with this set:
// pointers are not dereferenced or checked, and each dispatch point records the chosen
// kernel's per-launch cost instead of launching.
struct CostOut {
  long long v[KG_COST_KINDS];
};
thread_local CostOut* g_cost = nullptr;

// A memory slot viewed with its element shape/strides.
struct Mem {
  void* data = nullptr;
  int rank = 0;
  long long shape[8] = {0};
  long long stride[8] = {0};
  int dtype = 0;
  bool present = false;

  bool contiguous() const {
    if (numel() == 0) return true;  // no elements: any strides describe the same (empty) view
    long long expect = 1;
    for (int i = rank - 1; i >= 0; --i) {
      if (shape[i] != 1 && stride[i] != expect) return false;
      expect *= shape[i];
    }
    return true;
  }
  long long numel() const {
    long long n = 1;
    for (int i = 0; i < rank; ++i) n *= shape[i];
    return n;
  }
};

bool known_dtype(int code) {
  return code == KG_DTYPE_F32 || code == KG_DTYPE_F16 || code == KG_DTYPE_BF16;
}

const char* dtype_name(int code) {
  switch (code) {
    case KG_DTYPE_F32: return "f32";
    case KG_DTYPE_F64: return "f64";
    case KG_DTYPE_I32: return "i32";
    case KG_DTYPE_I64: return "i64";
    case KG_DTYPE_F16: return "f16";
    case KG_DTYPE_BF16: return "bf16";
    default: return "unknown";
  }
}

int read_mem(const KgArgSlot* slots, int idx, int rank, bool allow_absent, const char* name, Mem* out) {
  const KgArgSlot& s = slots[idx];
  if (s.kind != KG_ARG_MEMORY) return fail(kInvalid, "slot %d (%s): expected memory slot, got kind %d", idx, name, s.kind);
  if (s.data == nullptr) {
    if (allow_absent) {
      out->present = false;
      out->dtype = s.dtype_code;
      return kOk;
    }
    // an empty view may carry a null pointer (torch's zero-size tensors do); it is never
    // dereferenced, so it is accepted like any other empty operand
    bool empty_view = (int)s.rank == rank && s.shape != nullptr && s.stride != nullptr;
    bool has_zero = false;
    for (int i = 0; empty_view && i < rank; ++i) {
      if (s.shape[i] < 0) empty_view = false;
      if (s.shape[i] == 0) has_zero = true;
    }
    if (!empty_view || !has_zero) return fail(kInvalid, "slot %d (%s): memory slot has no data", idx, name);
  }
  if ((int)s.rank != rank) return fail(kInvalid, "slot %d (%s): expected rank %d, got %llu", idx, name, rank, s.rank);
  if (s.shape == nullptr || s.stride == nullptr) return fail(kInvalid, "slot %d (%s): missing shape/stride", idx, name);
  if (!known_dtype(s.dtype_code))
    return fail(kInvalid, "slot %d (%s): unsupported dtype_code %d (%s)", idx, name, s.dtype_code, dtype_name(s.dtype_code));
  out->data = s.data;
  out->rank = rank;
  out->dtype = s.dtype_code;
  out->present = true;
  bool empty = false;
  long long last = 0;  // largest element offset addressed by the view
  for (int i = 0; i < rank; ++i) {
    if (s.shape[i] < 0) return fail(kInvalid, "slot %d (%s): negative extent", idx, name);
    if (s.stride[i] < 0) return fail(kInvalid, "slot %d (%s): negative stride", idx, name);
    out->shape[i] = s.shape[i];
    out->stride[i] = s.stride[i];
    if (s.shape[i] == 0) empty = true;
    else last += (s.shape[i] - 1) * s.stride[i];
  }
  if (empty || g_cost != nullptr) return kOk;
  // The kernels dereference these pointers on the GPU: refuse host memory and views that
  // run past the end of their device allocation instead of faulting the device.
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, s.data) != hipSuccess || attr.type != hipMemoryTypeDevice) {
    (void)hipGetLastError();
    return fail(kInvalid, "slot %d (%s): data is not a device pointer", idx, name);
  }
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)s.data) != hipSuccess) {
    (void)hipGetLastError();
    return fail(kInvalid, "slot %d (%s): cannot query device allocation", idx, name);
  }
  const size_t elem = s.dtype_code == KG_DTYPE_F32 ? 4 : 2;
  const size_t need = (size_t)((const char*)s.data - (const char*)base) + (size_t)(last + 1) * elem;
  if (need > size)
    return fail(kInvalid, "slot %d (%s): view needs %zu bytes but the allocation holds %zu", idx, name, need, size);
  return kOk;
}

int read_int(const KgArgSlot* slots, int idx, const char* name, long long* out) {
  const KgArgSlot& s = slots[idx];
  if (s.kind != KG_ARG_INT) return fail(kInvalid, "slot %d (%s): expected int slot, got kind %d", idx, name, s.kind);
  *out = s.int_value;
  return kOk;
}

int read_float(const KgArgSlot* slots, int idx, const char* name, double* out) {
  const KgArgSlot& s = slots[idx];
  if (s.kind == KG_ARG_FLOAT) {
    *out = s.float_value;
    return kOk;
  }
  if (s.kind == KG_ARG_INT) {
    *out = (double)s.int_value;
    return kOk;
  }
  return fail(kInvalid, "slot %d (%s): expected float slot, got kind %d", idx, name, s.kind);
}

// (cost queries model device buffers, which are always 256-byte aligned)
bool aligned16(const void* p) { return g_cost != nullptr || ((uintptr_t)p & 15u) == 0; }

// mfma_cycles: SIMD cycles one of the kernel's MFMA instructions occupies (32 for
// 32x32x16, 16 for 16x16x32, 64 for the fp32 32x32x2).
int record_cost(long long mac, long long mfma, long long mfma_cycles, long long read, long long write) {
  g_cost->v[KG_COST_MAC] = mac;
  g_cost->v[KG_COST_MFMA] = mfma;
  g_cost->v[KG_COST_HBM_READ] = read;
  g_cost->v[KG_COST_HBM_WRITE] = write;
  g_cost->v[KG_COST_MFMA_CYCLES] = mfma * mfma_cycles;
  return kOk;
}
long long esize(int dtype) { return dtype == KG_DTYPE_F32 ? 4 : 2; }

int grid_1d(long long total, int threads) {
  long long blocks = (total + threads - 1) / threads;
  if (blocks > (1ll << 20)) blocks = 1ll << 20;
  if (blocks < 1) blocks = 1;
  return (int)blocks;
}

// ---------------------------------------------------------------------------------------
// matmul
// ---------------------------------------------------------------------------------------

template <typename TA, typename TBias>
int launch_gemm_simt(const Mem& out, const Mem& lhs, const Mem& rhs, const Mem& bias, int M, int N, int K) {
  const long long sbias = bias.present ? bias.stride[0] : 0;
  auto blocks = [&](int t) { return (long long)((N + t - 1) / t) * ((M + t - 1) / t); };
  // the largest tile that still gives every CU a block (256-thread blocks of T x T outputs)
  const int t = blocks(64) >= 256 ? 64 : blocks(32) >= 256 ? 32 : 16;
  // one-dimensional grid (gridDim.y is limited to 65535; x to 2^31 - 1)
  if (blocks(t) > 0x7fffffffLL) return fail(kUnsupported, "matmul(simt): %lld tiles exceed the grid limit", blocks(t));
#define KG_GEMM_SIMT(T)                                                                                          \
  hipLaunchKernelGGL((gemm_simt_kernel<TA, TA, TA, TBias, T>), dim3((unsigned)blocks(T)), dim3(256), 0, \
                     g_stream, static_cast<const TA*>(lhs.data), static_cast<const TA*>(rhs.data),                   \
                     static_cast<TA*>(out.data), static_cast<const TBias*>(bias.present ? bias.data : nullptr), M, N, \
                     K, lhs.stride[0], lhs.stride[1], rhs.stride[0], rhs.stride[1], out.stride[0], out.stride[1],   \
                     sbias)
  if (t == 64) KG_GEMM_SIMT(64);
  else if (t == 32) KG_GEMM_SIMT(32);
  else KG_GEMM_SIMT(16);
#undef KG_GEMM_SIMT
  return finish_launch("matmul(simt)");
}

// MI355X has 256 CUs: the pipelined GEMM takes 128-row tiles when 256-row tiles would not
// give every CU one.
constexpr long long kNumCUs = 256;
long long cdiv(long long a, long long b) { return (a + b - 1) / b; }
long long pipe_tile_m(long long M, long long N) {
  return cdiv(M, gemmp::kBM) * cdiv(N, gemmp::kBN) < kNumCUs ? 128 : 256;
}
// Shapes the pipelined kernel covers without its ragged-edge copies.
bool pipe_aligned(long long M, long long N, long long K) {
  return M % pipe_tile_m(M, N) == 0 && N % gemmp::kBN == 0 && K % gemmp::kBK == 0;
}
// Row strides up to 2^22 elements keep every copy lane's byte offset within a tile below
// 2^31 (the buffer range of the ragged copies; 255 rows x 2^23 bytes + 64).
constexpr long long kMaxPipeLd = 1LL << 22;

// Split-K for outputs of few tiles (skinny M or N: 16 x 4096 is 16 tiles of 128 x 256): the
// K range is cut into chunks (multiples of the 32-deep slice, at least 256 deep) until the
// grid covers the CUs, each workgroup row stores fp32 partial sums to a workspace, and a
// second kernel adds them in chunk order. Returns the chunk count (1: no split). The decision
// depends on the shape only, so every LDS ring depth gives the same bits.
constexpr long long kSplitMaxTiles = 64;                 // split below a quarter of the CUs, or
constexpr long long kSplitMaxTilesLongK = 128;           // below half of them when K is long:
constexpr long long kSplitLongK = 4096;                  // the fp32 partials then cost less than half the K loop
constexpr long long kSplitMinChunk = 256;                // k per chunk, at least 8 slices
constexpr long long kSplitMaxWorkspace = 64LL << 20;     // bytes of fp32 partials
int pipe_splits(long long M, long long N, long long K, long long* chunk) {
  const long long tiles = cdiv(M, pipe_tile_m(M, N)) * cdiv(N, gemmp::kBN);
  *chunk = K;
  const bool few = tiles <= kSplitMaxTiles || (tiles <= kSplitMaxTilesLongK && K >= kSplitLongK);
  if (!few || K < 2 * kSplitMinChunk) return 1;
  long long splits = std::min(cdiv(kNumCUs, tiles), K / kSplitMinChunk);
  splits = std::min(splits, kSplitMaxWorkspace / (M * N * 4));
  if (splits < 2) return 1;
  const long long c = cdiv(cdiv(K, splits), gemmp::kBK) * gemmp::kBK;
  *chunk = c;
  return (int)cdiv(K, c);
}

// Split-K workspaces, one per (device, stream) and kept for the life of the process: work
// enqueued on one stream runs in order, so its calls can share one buffer, and calls on
// different streams never do. A split call enqueues two kernels (the partial sums, then
// their reduction), and a call holds its slot's lock (the lease) from the lookup until both
// are enqueued: two host threads on one stream (every thread's default is the null stream)
// therefore enqueue whole pairs, never A's partials, B's partials, A's reduction. A larger
// request replaces the buffer (the old one is released in stream order, after the work
// already enqueued). At most kSplitCachedStreams buffers are kept per device: a call on
// another stream then takes the least recently used slot, waits for that slot's lease (so no
// call is between its two launches) and releases its buffer with hipFree, which waits for
// the device's pending work (the stream the buffer was used on may no longer exist). Lock
// order: the table's mutex, then a slot's. An allocation per call (hipMallocAsync /
// hipFreeAsync) cost about 60 us of host time per matmul. Calls that split allocate on the
// first use per stream (or a larger shape): they are not capturable in a HIP graph then.
constexpr int kSplitCachedStreams = 8;
struct SplitWorkspace {
  int device;
  hipStream_t stream;
  void* ptr;
  size_t bytes;
  unsigned long long last_use;
  std::shared_ptr<std::mutex> busy;  // the lease: held from the lookup through the reduction's launch
};
struct SplitLease {
  void* ptr = nullptr;
  std::unique_lock<std::mutex> hold;
};
std::mutex g_split_ws_mutex;
std::vector<SplitWorkspace> g_split_ws;
unsigned long long g_split_ws_clock = 0;

SplitLease split_workspace(size_t bytes, hipStream_t stream) {
  SplitLease lease;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return lease;
  std::lock_guard<std::mutex> lock(g_split_ws_mutex);
  int slot = -1, lru = -1, on_device = 0;
  for (int i = 0; i < (int)g_split_ws.size(); ++i) {
    const auto& w = g_split_ws[i];
    if (w.device != device) continue;
    ++on_device;
    if (w.stream == stream) slot = i;
    if (lru < 0 || w.last_use < g_split_ws[lru].last_use) lru = i;
  }
  if (slot >= 0) {
    lease.hold = std::unique_lock<std::mutex>(*g_split_ws[slot].busy);
    if (g_split_ws[slot].bytes >= bytes) {
      g_split_ws[slot].last_use = ++g_split_ws_clock;
      lease.ptr = g_split_ws[slot].ptr;
      return lease;
    }
  }
  void* ptr = nullptr;
  const size_t want = std::max(bytes, (size_t)(4u << 20));
  if (hipMalloc(&ptr, want) != hipSuccess) {
    (void)hipGetLastError();
    lease.hold = {};
    return lease;
  }
  if (slot >= 0) {
    (void)hipFreeAsync(g_split_ws[slot].ptr, stream);
  } else if (on_device >= kSplitCachedStreams) {
    slot = lru;
    lease.hold = std::unique_lock<std::mutex>(*g_split_ws[slot].busy);  // the evicted call has launched both kernels
    (void)hipFree(g_split_ws[slot].ptr);                                 // waits for the device's pending work
  } else {
    g_split_ws.push_back({device, stream, nullptr, 0, 0, std::make_shared<std::mutex>()});
    slot = (int)g_split_ws.size() - 1;
    lease.hold = std::unique_lock<std::mutex>(*g_split_ws[slot].busy);
  }
  SplitWorkspace& w = g_split_ws[slot];
  w.device = device;
  w.stream = stream;
  w.ptr = ptr;
  w.bytes = want;
  w.last_use = ++g_split_ws_clock;
  lease.ptr = ptr;
  return lease;
}

template <typename Tag>
int launch_gemm_mfma(const Mem& out, const Mem& lhs, const Mem& rhs, const Mem& bias, int M, int N, int K,
                     int stages) {
  const uint16_t* A = static_cast<const uint16_t*>(lhs.data);
  const uint16_t* B = static_cast<const uint16_t*>(rhs.data);
  uint16_t* C = static_cast<uint16_t*>(out.data);
  const void* bp = bias.present ? bias.data : nullptr;
  const int bias_kind = !bias.present ? 0 : (bias.dtype == KG_DTYPE_F32 ? 1 : 2);
  const long long lda = lhs.stride[0], ldb = rhs.stride[0], ldc = out.stride[0];
  // 128-row tiles when 256-row ones would leave CUs idle (C2': 8192x1024 is 128 tiles)
  const long long tm = pipe_tile_m(M, N);
  const bool ragged = !pipe_aligned(M, N, K);
  const int grid = (int)(cdiv(M, tm) * cdiv(N, gemmp::kBN));
  long long chunk = K;
  int splits = pipe_splits(M, N, K, &chunk);
  float* partial = nullptr;
  SplitLease lease;  // held until both kernels of a split call are enqueued (this function's return)
  if (splits > 1) {
    lease = split_workspace((size_t)splits * M * N * sizeof(float), g_stream);
    partial = static_cast<float*>(lease.ptr);
    if (partial == nullptr) splits = 1;  // no workspace: the whole K range in one pass
  }
  const int k_chunk = splits > 1 ? (int)chunk : 0;
  if (!ragged && splits == 1 && (tm == 256 || grid >= kNumCUs)) {
    // whole tiles that fill the chip: four waves of (tm/2) x 128 (same MFMA sequence per
    // output block as the eight-wave kernel, so the same bits)
    hipError_t e = hipSuccess;
#define KG_GEMM_QUAD(TM)                                                                                          \
  if (stages == 2) e = launch_gemm_quad<Tag, 2, TM>(A, B, C, bp, bias_kind, M, N, K, lda, ldb, ldc, g_stream);      \
  else if (stages == 3) e = launch_gemm_quad<Tag, 3, TM>(A, B, C, bp, bias_kind, M, N, K, lda, ldb, ldc, g_stream); \
  else e = launch_gemm_quad<Tag, 4, TM>(A, B, C, bp, bias_kind, M, N, K, lda, ldb, ldc, g_stream);
    if (tm == 256) { KG_GEMM_QUAD(256) } else { KG_GEMM_QUAD(128) }
#undef KG_GEMM_QUAD
    if (e != hipSuccess) return fail(kHipFailure, "matmul(mfma-quad): %s", hipGetErrorString(e));
    return finish_launch("matmul(mfma-quad)");
  }
#define KG_GEMM_PIPE(TM, ST, RAG)                                                                          \
  e = launch_gemm_pipe<Tag, TM, ST, RAG>(A, B, C, bp, bias_kind, M, N, K, lda, ldb, ldc, partial, k_chunk, grid, splits, \
                                         g_stream)
#define KG_GEMM_PIPE_DEPTH(TM, RAG)                  \
  if (stages == 2) { KG_GEMM_PIPE(TM, 2, RAG); }      \
  else if (stages == 3) { KG_GEMM_PIPE(TM, 3, RAG); } \
  else { KG_GEMM_PIPE(TM, 4, RAG); }
  hipError_t e = hipSuccess;
  if (tm == 128) {
    if (ragged) { KG_GEMM_PIPE_DEPTH(128, true) } else { KG_GEMM_PIPE_DEPTH(128, false) }
  } else {
    if (ragged) { KG_GEMM_PIPE_DEPTH(256, true) } else { KG_GEMM_PIPE_DEPTH(256, false) }
  }
#undef KG_GEMM_PIPE_DEPTH
#undef KG_GEMM_PIPE
  if (e != hipSuccess) return fail(kHipFailure, "matmul(mfma-pipe): %s", hipGetErrorString(e));
  if (splits > 1) {
    const int rgrid = (int)cdiv((long long)M * (N / 4), kSplitReduceThreads);
    if (bias_kind == 0)
      hipLaunchKernelGGL((gemm_splitk_reduce_kernel<Tag, 0>), dim3(rgrid), dim3(kSplitReduceThreads), 0, g_stream, partial, splits, C, bp,
                         M, N, ldc);
    else if (bias_kind == 1)
      hipLaunchKernelGGL((gemm_splitk_reduce_kernel<Tag, 1>), dim3(rgrid), dim3(kSplitReduceThreads), 0, g_stream, partial, splits, C, bp,
                         M, N, ldc);
    else
      hipLaunchKernelGGL((gemm_splitk_reduce_kernel<Tag, 2>), dim3(rgrid), dim3(kSplitReduceThreads), 0, g_stream, partial, splits, C, bp,
                         M, N, ldc);
    return finish_launch("matmul(mfma-pipe-splitk)");
  }
  return finish_launch(ragged ? "matmul(mfma-pipe-ragged)" : "matmul(mfma-pipe)");
}

// fp32 on matrix cores: 64-cycle MFMAs on 128 x 128 tiles. Below 32 tiles (e.g. C1's
// 256^3 is 4) the SIMT kernel, which spreads small problems over every CU, finishes first.
constexpr long long kF32MfmaMinTiles = 32;
bool gemm_f32_mfma_pays(long long M, long long N, long long K) {
  return cdiv(M, gemmf::kTile) * cdiv(N, gemmf::kTile) >= kF32MfmaMinTiles && K >= 4 * gemmf::kBK;
}

int launch_gemm_f32_mfma(const Mem& out, const Mem& lhs, const Mem& rhs, const Mem& bias, int M, int N, int K,
                         int stages) {
  const float* A = static_cast<const float*>(lhs.data);
  const float* B = static_cast<const float*>(rhs.data);
  float* C = static_cast<float*>(out.data);
  const float* bp = bias.present ? static_cast<const float*>(bias.data) : nullptr;
  const bool ragged = M % gemmf::kTile || N % gemmf::kTile || K % gemmf::kBK;
  const int grid = (int)(cdiv(M, gemmf::kTile) * cdiv(N, gemmf::kTile));
  const long long lda = lhs.stride[0], ldb = rhs.stride[0], ldc = out.stride[0];
#define KG_GEMM_F32(BIAS, RAG, ST)                                                                                   \
  hipLaunchKernelGGL((gemm_f32_mfma_kernel<BIAS, RAG, ST>), dim3(grid), dim3(gemmf::kThreads), 0, g_stream, A, B, C, bp, \
                     M, N, K, lda, ldb, ldc)
#define KG_GEMM_F32_ST(BIAS, RAG)                                       \
  if (stages == 2) { KG_GEMM_F32(BIAS, RAG, 2); }                       \
  else if (stages == 4) { KG_GEMM_F32(BIAS, RAG, 4); }                  \
  else { KG_GEMM_F32(BIAS, RAG, 3); }
  if (ragged) {
    if (bp) { KG_GEMM_F32_ST(1, true) } else { KG_GEMM_F32_ST(0, true) }
  } else {
    if (bp) { KG_GEMM_F32_ST(1, false) } else { KG_GEMM_F32_ST(0, false) }
  }
#undef KG_GEMM_F32_ST
#undef KG_GEMM_F32
  return finish_launch(ragged ? "matmul(f32-mfma-ragged)" : "matmul(f32-mfma)");
}

// Small fp32 outputs (fewer than kF32MfmaMinTiles tiles of 128 x 128) with 32-aligned
// extents: split-K inside a workgroup per 32 x 32 block.
bool gemm_f32_splitk_ok(const Mem& out, const Mem& lhs, const Mem& rhs, long long M, long long N, long long K) {
  return M % 32 == 0 && N % 32 == 0 && K % 16 == 0 && K > 0 && M > 0 && N > 0 && lhs.stride[1] == 1 &&
         rhs.stride[1] == 1 && out.stride[1] == 1 && lhs.stride[0] % 4 == 0 && aligned16(lhs.data) &&
         (M / 32) * (N / 32) < (1LL << 31);
}

int launch_gemm_f32_splitk(const Mem& out, const Mem& lhs, const Mem& rhs, const Mem& bias, int M, int N, int K) {
  const int grid = (M / 32) * (N / 32);
  const float* A = static_cast<const float*>(lhs.data);
  const float* B = static_cast<const float*>(rhs.data);
  float* C = static_cast<float*>(out.data);
  const float* bp = bias.present ? static_cast<const float*>(bias.data) : nullptr;
  if (bp)
    hipLaunchKernelGGL((gemm_f32_splitk_kernel<1>), dim3(grid), dim3(gemmk::kThreads), 0, g_stream, A, B, C, bp, M, N, K,
                       lhs.stride[0], rhs.stride[0], out.stride[0]);
  else
    hipLaunchKernelGGL((gemm_f32_splitk_kernel<0>), dim3(grid), dim3(gemmk::kThreads), 0, g_stream, A, B, C, bp, M, N, K,
                       lhs.stride[0], rhs.stride[0], out.stride[0]);
  return finish_launch("matmul(f32-splitk)");
}

int matmul_impl(const KgArgSlot* args, unsigned long long n) {
  if (args == nullptr) return fail(kInvalid, "ordered_args is null");
  if (n != 4 && n != 7 && n != 8) return fail(kInvalid, "matmul expects 4, 7 or 8 slots, got %llu", n);
  Mem out, lhs, rhs, bias;
  int rc;
  if ((rc = read_mem(args, 0, 2, false, "out", &out))) return rc;
  if ((rc = read_mem(args, 1, 2, false, "lhs", &lhs))) return rc;
  if ((rc = read_mem(args, 2, 2, false, "rhs", &rhs))) return rc;
  if ((rc = read_mem(args, 3, 1, true, "bias", &bias))) return rc;
  if (n >= 7) {
    long long t;
    const char* names[3] = {"tile_m", "tile_n", "tile_k"};
    for (int i = 0; i < 3; ++i) {
      if ((rc = read_int(args, 4 + i, names[i], &t))) return rc;
      if (t <= 0) return fail(kInvalid, "%s must be positive, got %lld", names[i], t);
    }
  }
  long long stages = gemmp::kDefaultStages;  // LDS ring depth of the pipelined MFMA kernel
  long long stages_f32 = gemmf::kDefaultStages;  // and of the fp32 MFMA kernel
  const bool staged = n == 8;
  if (staged) {
    if ((rc = read_int(args, 7, "memory_stage", &stages))) return rc;
    if (stages < 2 || stages > 4) return fail(kInvalid, "matmul: memory_stage must be 2, 3 or 4, got %lld", stages);
    stages_f32 = stages;
  }
  const long long M = lhs.shape[0], K = lhs.shape[1], N = rhs.shape[1];
  if (rhs.shape[0] != K) return fail(kInvalid, "matmul: lhs K=%lld != rhs K=%lld", K, rhs.shape[0]);
  if (out.shape[0] != M || out.shape[1] != N)
    return fail(kInvalid, "matmul: out shape [%lld,%lld] != [%lld,%lld]", out.shape[0], out.shape[1], M, N);
  if (bias.present && bias.shape[0] != N) return fail(kInvalid, "matmul: bias extent %lld != N=%lld", bias.shape[0], N);
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff) return fail(kUnsupported, "matmul: extent exceeds int32");
  if (lhs.dtype != out.dtype || rhs.dtype != out.dtype)
    return fail(kInvalid, "matmul: lhs/rhs/out dtypes must match (%s, %s, %s)", dtype_name(lhs.dtype),
                dtype_name(rhs.dtype), dtype_name(out.dtype));
  if (bias.present && bias.dtype != out.dtype && bias.dtype != KG_DTYPE_F32)
    return fail(kInvalid, "matmul: bias dtype %s must be f32 or match out", dtype_name(bias.dtype));
  const int m = (int)M, nn = (int)N, k = (int)K;
  const bool mfma_ok = out.dtype != KG_DTYPE_F32 && k > 0 && (k % 8 == 0) && (nn % 8 == 0) && lhs.stride[1] == 1 &&
                       rhs.stride[1] == 1 && out.stride[1] == 1 && lhs.stride[0] % 8 == 0 && rhs.stride[0] % 8 == 0 &&
                       out.stride[0] % 8 == 0 && lhs.stride[0] <= kMaxPipeLd && rhs.stride[0] <= kMaxPipeLd &&
                       aligned16(lhs.data) && aligned16(rhs.data) && aligned16(out.data) &&
                       (!bias.present || bias.stride[0] == 1);
  const bool f32_mfma_ok = out.dtype == KG_DTYPE_F32 && k % 4 == 0 && nn % 4 == 0 && lhs.stride[1] == 1 &&
                           rhs.stride[1] == 1 && out.stride[1] == 1 && lhs.stride[0] % 4 == 0 &&
                           rhs.stride[0] % 4 == 0 && out.stride[0] % 4 == 0 && lhs.stride[0] <= kMaxPipeLd &&
                           rhs.stride[0] <= kMaxPipeLd && aligned16(lhs.data) && aligned16(rhs.data) &&
                           aligned16(out.data) && (!bias.present || bias.stride[0] == 1) && gemm_f32_mfma_pays(M, N, K);
  if (g_cost) {
    long long mfma = 0, cyc = 64;
    if (f32_mfma_ok)  // 4 waves x 2 x 2 blocks x 8 k-steps (32x32x2) per 16-deep slice of a 128 x 128 tile
      mfma = cdiv(M, gemmf::kTile) * cdiv(N, gemmf::kTile) * cdiv(K, gemmf::kBK) * 128;
    else if (out.dtype == KG_DTYPE_F32 && gemm_f32_splitk_ok(out, lhs, rhs, M, N, K) &&
             (!bias.present || bias.stride[0] == 1))  // 8 MFMAs (32x32x2) per 32 x 32 block and 16-deep slice
      mfma = (M / 32) * (N / 32) * (K / 16) * 8;
    if (mfma_ok && M > 0 && N > 0) {
      // tm MFMAs (16x16x32) per 32-deep slice of a tm x 256 tile: 8 waves x tm/8, or for
      // whole 256 x 256 tiles 4 waves x 64; ragged edges are covered by whole tiles and slices
      const long long tm = pipe_tile_m(M, N);
      mfma = cdiv(M, tm) * cdiv(N, gemmp::kBN) * cdiv(K, gemmp::kBK) * tm;
      cyc = 16;
    }
    const long long es = esize(out.dtype);
    return record_cost(M * N * K, mfma, cyc, (M * K + K * N) * es + (bias.present ? N * esize(bias.dtype) : 0),
                       M * N * es);
  }
  if (M == 0 || N == 0) return finish_launch("matmul(empty)");

  if (out.dtype == KG_DTYPE_F32) {
    if (f32_mfma_ok) return launch_gemm_f32_mfma(out, lhs, rhs, bias, m, nn, k, (int)stages_f32);
    if (staged)
      return fail(kUnsupported, "matmul: memory_stage sets the LDS ring depth of the MFMA kernels; this fp32 call takes "
                                "a kernel that loads its operands straight into registers");
    if (gemm_f32_splitk_ok(out, lhs, rhs, M, N, K) && (!bias.present || bias.stride[0] == 1))
      return launch_gemm_f32_splitk(out, lhs, rhs, bias, m, nn, k);
    return launch_gemm_simt<float, float>(out, lhs, rhs, bias, m, nn, k);
  }
  if (staged && !mfma_ok)
    return fail(kUnsupported, "matmul: memory_stage sets the LDS ring depth of the MFMA kernels; this call takes the "
                              "SIMT kernel, which stages nothing through an LDS ring");
  if (out.dtype == KG_DTYPE_BF16) {
    if (mfma_ok) return launch_gemm_mfma<Bf16Tag>(out, lhs, rhs, bias, m, nn, k, (int)stages);
    if (bias.present && bias.dtype == KG_DTYPE_F32) return launch_gemm_simt<__bf16, float>(out, lhs, rhs, bias, m, nn, k);
    return launch_gemm_simt<__bf16, __bf16>(out, lhs, rhs, bias, m, nn, k);
  }
  if (mfma_ok) return launch_gemm_mfma<F16Tag>(out, lhs, rhs, bias, m, nn, k, (int)stages);
  if (bias.present && bias.dtype == KG_DTYPE_F32) return launch_gemm_simt<_Float16, float>(out, lhs, rhs, bias, m, nn, k);
  return launch_gemm_simt<_Float16, _Float16>(out, lhs, rhs, bias, m, nn, k);
}

// ---------------------------------------------------------------------------------------
// conv2d
// ---------------------------------------------------------------------------------------

template <typename T, typename TB>
int launch_conv_direct(const Mem& out, const Mem& x, const Mem& w, const Mem& bias, const ConvShape& s) {
  const long long total = out.numel();
  hipLaunchKernelGGL((conv2d_direct_kernel<T, T, T, TB>), dim3(grid_1d(total, 256)), dim3(256), 0, g_stream,
                     static_cast<const T*>(x.data), static_cast<const T*>(w.data), static_cast<T*>(out.data),
                     static_cast<const TB*>(bias.present ? bias.data : nullptr), s);
  return finish_launch("conv2d(direct)");
}

int conv2d_impl(const KgArgSlot* args, unsigned long long n) {
  if (args == nullptr) return fail(kInvalid, "ordered_args is null");
  if (n != 12 && n != 17 && n != 18) return fail(kInvalid, "conv2d expects 12, 17 or 18 slots, got %llu", n);
  Mem out, x, w, bias;
  int rc;
  if ((rc = read_mem(args, 0, 4, false, "out", &out))) return rc;
  if ((rc = read_mem(args, 1, 4, false, "input", &x))) return rc;
  if ((rc = read_mem(args, 2, 4, false, "weight", &w))) return rc;
  if ((rc = read_mem(args, 3, 1, true, "bias", &bias))) return rc;
  long long p[8];
  const char* names[8] = {"stride_h", "stride_w", "dilation_h", "dilation_w", "pad_top", "pad_bottom", "pad_left", "pad_right"};
  for (int i = 0; i < 8; ++i)
    if ((rc = read_int(args, 4 + i, names[i], &p[i]))) return rc;
  for (int i = 0; i < 4; ++i)
    if (p[i] <= 0) return fail(kInvalid, "conv2d: %s must be positive, got %lld", names[i], p[i]);
  for (int i = 4; i < 8; ++i)
    if (p[i] < 0) return fail(kInvalid, "conv2d: %s must be non-negative, got %lld", names[i], p[i]);
  if (n >= 17) {
    const char* tnames[5] = {"tile_f", "tile_c", "tile_n", "tile_ho", "tile_wo"};
    for (int i = 0; i < 5; ++i) {
      long long t;
      if ((rc = read_int(args, 12 + i, tnames[i], &t))) return rc;
      if (t <= 0) return fail(kInvalid, "conv2d: %s must be positive, got %lld", tnames[i], t);
    }
  }
  // slot 17: memory_stage, the LDS stage count of the row-piece and implicit-GEMM kernels
  long long stages = 2;
  const bool staged = n == 18;
  if (staged) {
    if ((rc = read_int(args, 17, "memory_stage", &stages))) return rc;
    if (stages < 2 || stages > 4) return fail(kInvalid, "conv2d: memory_stage must be 2, 3 or 4, got %lld", stages);
  }
  if (!x.contiguous() || !w.contiguous() || !out.contiguous() || (bias.present && bias.stride[0] != 1))
    return fail(kInvalid, "conv2d: memory args must be contiguous");
  if (x.dtype != out.dtype || w.dtype != out.dtype) return fail(kInvalid, "conv2d: input/weight/out dtypes must match");
  if (bias.present && bias.dtype != out.dtype && bias.dtype != KG_DTYPE_F32)
    return fail(kInvalid, "conv2d: bias dtype must be f32 or match out");
  ConvShape s;
  s.n = (int)x.shape[0];
  s.c = (int)x.shape[1];
  s.h = (int)x.shape[2];
  s.w = (int)x.shape[3];
  s.f = (int)w.shape[0];
  s.kh = (int)w.shape[2];
  s.kw = (int)w.shape[3];
  s.sh = (int)p[0];
  s.sw = (int)p[1];
  s.dh = (int)p[2];
  s.dw = (int)p[3];
  s.pt = (int)p[4];
  s.pl = (int)p[6];
  if (w.shape[1] != x.shape[1]) return fail(kInvalid, "conv2d: weight C=%lld != input C=%lld", w.shape[1], x.shape[1]);
  // Ho/Wo with floor division, as the demos compute them (kernel/conv2d/inputs_static_tile_static.py:
  // 155-156, Python //): a window larger than the padded input gives an empty output
  // (Ho or Wo = 0), never a row built from outside the input.
  auto floor_div = [](long long a, long long b) { return a >= 0 ? a / b : -((-a + b - 1) / b); };
  const long long ho = std::max(0LL, floor_div(x.shape[2] + p[4] + p[5] - p[2] * (w.shape[2] - 1) - 1, p[0]) + 1);
  const long long wo = std::max(0LL, floor_div(x.shape[3] + p[6] + p[7] - p[3] * (w.shape[3] - 1) - 1, p[1]) + 1);
  s.ho = (int)ho;
  s.wo = (int)wo;
  if (out.shape[0] != x.shape[0] || out.shape[1] != w.shape[0] || out.shape[2] != ho || out.shape[3] != wo)
    return fail(kInvalid, "conv2d: out shape [%lld,%lld,%lld,%lld] != [%lld,%lld,%lld,%lld]", out.shape[0], out.shape[1],
                out.shape[2], out.shape[3], x.shape[0], w.shape[0], ho, wo);
  if (bias.present && bias.shape[0] != w.shape[0]) return fail(kInvalid, "conv2d: bias extent != F");
  if (g_cost) {
    long long mfma = 0;
    if (!staged && out.dtype != KG_DTYPE_F32 && conv_mfma_supported(s)) {  // live waves x 252 MFMAs per 7-row block
      mfma = (long long)s.n * ((s.h + convk::kRows - 1) / convk::kRows) * (s.w > 32 ? 4 : 2) * 252;
    } else if (conv_rowvec_supported(s, out.dtype == KG_DTYPE_F32)) {
      mfma = conv_rowvec_mfma(s, out.dtype == KG_DTYPE_F32);
    } else if (conv_igemm_supported(s)) {
      // implicit GEMM: per tile and 64-byte k slice, 4 waves x MI x 2 blocks x (2 MFMAs of
      // 32x32x16, or 8 of 32x32x2 for fp32)
      const long long mi = conv_igemm_mi(s), K = (long long)s.c * s.kh * s.kw;
      const long long per = out.dtype == KG_DTYPE_F32 ? 8 : 2, bk = out.dtype == KG_DTYPE_F32 ? 16 : 32;
      const long long tiles = cdiv(s.f, 64 * mi) * cdiv((long long)s.n * s.ho * s.wo, convg::kBN);
      mfma = tiles * cdiv(K, bk) * 4 * mi * 2 * per;
    }
    const long long es = esize(out.dtype);
    return record_cost(out.numel() * w.shape[1] * w.shape[2] * w.shape[3], mfma, out.dtype == KG_DTYPE_F32 ? 64 : 32,
                       (x.numel() + w.numel()) * es + (bias.present ? bias.shape[0] * esize(bias.dtype) : 0),
                       out.numel() * es);
  }
  if (out.numel() == 0) return finish_launch("conv2d(empty)");

  // The row-phase kernel stages its input rows in two fixed parts: a call that sets the
  // stage count takes the row-piece kernel (which supports every shape the row-phase one does)
  if (!staged && out.dtype == KG_DTYPE_F16 && conv_mfma_supported(s) && aligned16(x.data) && aligned16(w.data) && aligned16(out.data)) {
    const int bias_kind = !bias.present ? 0 : (bias.dtype == KG_DTYPE_F32 ? 1 : 2);
    hipError_t e = launch_conv2d_mfma<F16Tag>(static_cast<const uint16_t*>(x.data), static_cast<const uint16_t*>(w.data),
                                              static_cast<uint16_t*>(out.data), bias.present ? bias.data : nullptr,
                                              bias_kind, s, g_stream);
    if (e != hipSuccess) return fail(kHipFailure, "conv2d(mfma): %s", hipGetErrorString(e));
    return finish_launch("conv2d(mfma)");
  }
  if (!staged && out.dtype == KG_DTYPE_BF16 && conv_mfma_supported(s) && aligned16(x.data) && aligned16(w.data) && aligned16(out.data)) {
    const int bias_kind = !bias.present ? 0 : (bias.dtype == KG_DTYPE_F32 ? 1 : 2);
    hipError_t e = launch_conv2d_mfma<Bf16Tag>(static_cast<const uint16_t*>(x.data), static_cast<const uint16_t*>(w.data),
                                               static_cast<uint16_t*>(out.data), bias.present ? bias.data : nullptr,
                                               bias_kind, s, g_stream);
    if (e != hipSuccess) return fail(kHipFailure, "conv2d(mfma): %s", hipGetErrorString(e));
    return finish_launch("conv2d(mfma)");
  }
  // split-K for conv grids of fewer than two workgroups per CU: fp32 partials in the
  // matmul's per-stream split-K workspace (no workspace: the whole K range in one pass)
  SplitLease lease;  // held until both kernels of a split call are enqueued (this function's return)
  auto conv_partials = [&](int& splits) -> float* {
    if (splits <= 1) return nullptr;
    lease = split_workspace((size_t)splits * out.numel() * sizeof(float), g_stream);
    float* ws = static_cast<float*>(lease.ptr);
    if (ws == nullptr) splits = 1;
    return ws;
  };
  if (out.dtype == KG_DTYPE_F32 && conv_rowvec_supported(s, true) && aligned16(x.data) && aligned16(w.data) &&
      aligned16(out.data)) {
    int kcs = 0;
    int splits = conv_rowvec_splits(s, true, kSplitMaxWorkspace, &kcs);
    float* partial = conv_partials(splits);
    hipError_t e = launch_conv2d_rowvec_f32(static_cast<const float*>(x.data), static_cast<const float*>(w.data),
                                            static_cast<float*>(out.data),
                                            bias.present ? static_cast<const float*>(bias.data) : nullptr,
                                            bias.present ? 1 : 0, s, g_stream, partial, splits, kcs, (int)stages);
    if (e != hipSuccess) return fail(kHipFailure, "conv2d(rowvec f32): %s", hipGetErrorString(e));
    return finish_launch("conv2d(rowvec f32)");
  }
  if (out.dtype != KG_DTYPE_F32 && conv_rowvec_supported(s) && aligned16(x.data) && aligned16(w.data) &&
      aligned16(out.data)) {
    const int bias_kind = !bias.present ? 0 : (bias.dtype == KG_DTYPE_F32 ? 1 : 2);
    const uint16_t* xp = static_cast<const uint16_t*>(x.data);
    const uint16_t* wp = static_cast<const uint16_t*>(w.data);
    uint16_t* yp = static_cast<uint16_t*>(out.data);
    const void* bp = bias.present ? bias.data : nullptr;
    int kcs = 0;
    int splits = conv_rowvec_splits(s, false, kSplitMaxWorkspace, &kcs);
    float* partial = conv_partials(splits);
    hipError_t e = out.dtype == KG_DTYPE_BF16
                       ? launch_conv2d_rowvec<Bf16Tag>(xp, wp, yp, bp, bias_kind, s, g_stream, partial, splits, kcs,
                                                       (int)stages)
                       : launch_conv2d_rowvec<F16Tag>(xp, wp, yp, bp, bias_kind, s, g_stream, partial, splits, kcs,
                                                      (int)stages);
    if (e != hipSuccess) return fail(kHipFailure, "conv2d(rowvec): %s", hipGetErrorString(e));
    return finish_launch("conv2d(rowvec)");
  }
  if (conv_igemm_supported(s) && aligned16(out.data)) {
    const int bias_kind = !bias.present ? 0 : (bias.dtype == KG_DTYPE_F32 ? 1 : 2);
    const long long K = (long long)s.c * s.kh * s.kw;
    // Contraction order (measured on MI355X): 16-bit convs are bound by their load count,
    // so they keep the weight's own order and read weights as 16-byte chunks; fp32 and 1x1
    // convs gain more from the tap-major gather (one bounds check and address per chunk).
    const int per_chunk = out.dtype == KG_DTYPE_F32 ? 4 : 8;
    const bool tap_ok = s.c % per_chunk == 0;
    const bool vec_ok = aligned16(w.data) && K % per_chunk == 0;
    const bool one_tap = s.kh * s.kw == 1;
    const int order = tap_ok && (out.dtype == KG_DTYPE_F32 || one_tap || !vec_ok) ? kTapMajor
                      : vec_ok                                                       ? kChannelMajorVecW
                                                                                     : kChannelMajor;
    const bool w_vec = order == kTapMajor && one_tap && vec_ok;
    const void* bp = bias.present ? bias.data : nullptr;
    int kcs = 0;
    int splits = conv_igemm_splits(s, out.dtype == KG_DTYPE_F32, kSplitMaxWorkspace, &kcs);
    float* partial = conv_partials(splits);
    hipError_t e =
        out.dtype == KG_DTYPE_F32
            ? launch_conv2d_igemm<F32Tag>(x.data, w.data, out.data, bp, bias_kind, order, w_vec, s, g_stream, partial,
                                          splits, kcs, (int)stages)
        : out.dtype == KG_DTYPE_BF16
            ? launch_conv2d_igemm<Bf16Tag>(x.data, w.data, out.data, bp, bias_kind, order, w_vec, s, g_stream, partial,
                                           splits, kcs, (int)stages)
            : launch_conv2d_igemm<F16Tag>(x.data, w.data, out.data, bp, bias_kind, order, w_vec, s, g_stream, partial,
                                          splits, kcs, (int)stages);
    if (e != hipSuccess) return fail(kHipFailure, "conv2d(igemm): %s", hipGetErrorString(e));
    return finish_launch("conv2d(igemm)");
  }
  if (staged)
    return fail(kUnsupported, "conv2d: memory_stage sets the LDS stage count of the row-piece and implicit-GEMM kernels; "
                              "this shape takes the direct kernel, which stages nothing through LDS");
  const bool f32_bias = bias.present && bias.dtype == KG_DTYPE_F32;
  switch (out.dtype) {
    case KG_DTYPE_F32: return launch_conv_direct<float, float>(out, x, w, bias, s);
    case KG_DTYPE_BF16:
      return f32_bias ? launch_conv_direct<__bf16, float>(out, x, w, bias, s) : launch_conv_direct<__bf16, __bf16>(out, x, w, bias, s);
    default:
      return f32_bias ? launch_conv_direct<_Float16, float>(out, x, w, bias, s)
                      : launch_conv_direct<_Float16, _Float16>(out, x, w, bias, s);
  }
}

// ---------------------------------------------------------------------------------------
// flash attention
// ---------------------------------------------------------------------------------------

template <typename T>
int launch_fa_simt(const Mem& out, const Mem& q, const Mem& k, const Mem& v, const FaShape& s) {
  // one block per (b*h, query row) on a one-dimensional grid (gridDim.y is limited to 65535)
  const long long blocks = (long long)s.s_q * s.bh;
  if (blocks > 0x7fffffffLL) return fail(kUnsupported, "flash_attention(simt): %lld query rows exceed the grid limit", blocks);
  hipLaunchKernelGGL((fa_fwd_simt_kernel<T>), dim3((unsigned)blocks), dim3(128), 0, g_stream, static_cast<const T*>(q.data),
                     static_cast<const T*>(k.data), static_cast<const T*>(v.data), static_cast<T*>(out.data), s);
  return finish_launch("flash_attention(simt)");
}

int flash_attention_impl(const KgArgSlot* args, unsigned long long n) {
  if (args == nullptr) return fail(kInvalid, "ordered_args is null");
  if (n != 4 && n != 6 && n != 8 && n != 9)
    return fail(kInvalid, "flash_attention expects 4, 6, 8 or 9 slots, got %llu", n);
  Mem out, q, k, v;
  int rc;
  if ((rc = read_mem(args, 0, 4, false, "out", &out))) return rc;
  if ((rc = read_mem(args, 1, 4, false, "q", &q))) return rc;
  if ((rc = read_mem(args, 2, 4, false, "k", &k))) return rc;
  if ((rc = read_mem(args, 3, 4, false, "v", &v))) return rc;
  double scale = 1.0;
  long long causal = 0;
  if (n >= 6) {
    long long br, bc;
    if ((rc = read_int(args, 4, "br", &br))) return rc;
    if ((rc = read_int(args, 5, "bc", &bc))) return rc;
    if (br <= 0 || bc <= 0) return fail(kInvalid, "flash_attention: br/bc must be positive");
  }
  // slot 8: memory_stage, the K/V ring depth of the 16-bit MFMA kernel
  long long stages = fa::kDefaultStages;
  const bool staged = n == 9;
  if (staged) {
    if ((rc = read_int(args, 8, "memory_stage", &stages))) return rc;
    if (stages < 2 || stages > 4) return fail(kInvalid, "flash_attention: memory_stage must be 2, 3 or 4, got %lld", stages);
  }
  if (n >= 8) {
    if ((rc = read_float(args, 6, "scale", &scale))) return rc;
    if ((rc = read_int(args, 7, "causal", &causal))) return rc;
    if (causal != 0 && causal != 1) return fail(kInvalid, "flash_attention: causal must be 0 or 1");
    if (!std::isfinite(scale)) return fail(kInvalid, "flash_attention: scale must be finite");
  }
  for (int i = 0; i < 4; ++i) {
    if (q.shape[i] != out.shape[i]) return fail(kInvalid, "flash_attention: q/out shape mismatch at dim %d", i);
    if (k.shape[i] != v.shape[i]) return fail(kInvalid, "flash_attention: k/v shape mismatch at dim %d", i);
  }
  if (k.shape[0] != q.shape[0] || k.shape[1] != q.shape[1] || k.shape[3] != q.shape[3])
    return fail(kInvalid, "flash_attention: k batch/head/dim must match q");
  if (!out.contiguous() || !q.contiguous() || !k.contiguous() || !v.contiguous())
    return fail(kInvalid, "flash_attention: memory args must be contiguous");
  if (q.dtype != out.dtype || k.dtype != out.dtype || v.dtype != out.dtype)
    return fail(kInvalid, "flash_attention: q/k/v/out dtypes must match");
  FaShape s;
  s.bh = (int)(q.shape[0] * q.shape[1]);
  s.s_q = (int)q.shape[2];
  s.s_kv = (int)k.shape[2];
  s.d = (int)q.shape[3];
  s.scale = (float)scale;
  s.causal = (int)causal;
  if (s.s_kv == 0 && out.numel() > 0) return fail(kInvalid, "flash_attention: no keys (S_kv == 0) for a non-empty output");
  if (g_cost == nullptr && out.numel() == 0) return finish_launch("flash_attention(empty)");
  if (s.d > 512) return fail(kUnsupported, "flash_attention: head dim %d > 512", s.d);
  if (s.causal && s.s_kv != s.s_q) return fail(kUnsupported, "flash_attention: causal mask needs S_q == S_kv");
  if (g_cost) {
    const long long B_H = (long long)s.bh, D = s.d;
    // products Q.K^T and P.V that the mask keeps: causal row i sees keys 0..i
    const long long pairs = s.causal ? (long long)s.s_q * (s.s_q + 1) / 2 : (long long)s.s_q * s.s_kv;
    long long mfma = 0;
    if ((out.dtype == KG_DTYPE_BF16 || out.dtype == KG_DTYPE_F16) && fa_mfma_supported(s) && out.numel() > 0) {
      // per workgroup: waves x key tiles x (D/4 16x16x32 MFMAs for S^T + D/4 for PV + 4 row sums)
      const int waves = fa_mfma_waves(s);
      const int bm = 32 * waves;
      const int nmb = (s.s_q + bm - 1) / bm;
      long long tiles = 0;
      for (int mb = 0; mb < nmb; ++mb) {
        const int n_end = s.causal ? std::min(s.s_kv, (mb + 1) * bm) : s.s_kv;
        tiles += (n_end + fa::kBC - 1) / fa::kBC;
      }
      mfma = B_H * tiles * waves * (s.d / 2 + 4);
    }
    if (out.dtype == KG_DTYPE_F32 && fa_f32_mfma_supported(s) && out.numel() > 0) {
      // per workgroup and key tile: D MFMAs (32x32x2: D/2 for S^T, D/2 for PV) per wave that
      // has a query and (causal) a visible key in the tile
      const int nqb = (s.s_q + faf::kBM - 1) / faf::kBM;
      long long waves_tiles = 0;
      for (int qb = 0; qb < nqb; ++qb) {
        const int q_wg = qb * faf::kBM;
        const int n_tiles_all = (s.s_kv + faf::kBC - 1) / faf::kBC;
        const int n_tiles =
            s.causal ? std::min(n_tiles_all, (std::min(q_wg + faf::kBM, s.s_q) + faf::kBC - 1) / faf::kBC) : n_tiles_all;
        for (int w = 0; w < faf::kWaves; ++w) {
          const int q0 = q_wg + 32 * w;
          if (q0 >= s.s_q) continue;
          waves_tiles += s.causal ? std::min(n_tiles, q0 / faf::kBC + 1) : n_tiles;
        }
      }
      mfma = B_H * waves_tiles * s.d;
    }
    const long long es = esize(out.dtype);
    return record_cost(2 * B_H * pairs * D, mfma, out.dtype == KG_DTYPE_F32 ? 64 : 16,
                       (q.numel() + k.numel() + v.numel()) * es, out.numel() * es);
  }

  if ((out.dtype == KG_DTYPE_BF16 || out.dtype == KG_DTYPE_F16) && fa_mfma_supported(s) && aligned16(q.data) &&
      aligned16(k.data) && aligned16(v.data) && aligned16(out.data)) {
    hipError_t e = out.dtype == KG_DTYPE_BF16
                       ? launch_fa_fwd_mfma<Bf16Tag>(static_cast<const uint16_t*>(q.data), static_cast<const uint16_t*>(k.data),
                                                     static_cast<const uint16_t*>(v.data), static_cast<uint16_t*>(out.data), s,
                                                     g_stream, (int)stages)
                       : launch_fa_fwd_mfma<F16Tag>(static_cast<const uint16_t*>(q.data), static_cast<const uint16_t*>(k.data),
                                                    static_cast<const uint16_t*>(v.data), static_cast<uint16_t*>(out.data), s,
                                                    g_stream, (int)stages);
    if (e != hipSuccess) return fail(kHipFailure, "flash_attention(mfma): %s", hipGetErrorString(e));
    return finish_launch("flash_attention(mfma)");
  }
  if (out.dtype == KG_DTYPE_F32 && fa_f32_mfma_supported(s) && aligned16(q.data) && aligned16(k.data) &&
      aligned16(v.data) && aligned16(out.data)) {
    if (staged && stages != 2)
      return fail(kUnsupported, "flash_attention: the fp32 MFMA kernel keeps two K and two V buffers, so memory_stage "
                                "must be 2 for it, got %lld", stages);
    hipError_t e = launch_fa_fwd_f32_mfma(static_cast<const float*>(q.data), static_cast<const float*>(k.data),
                                          static_cast<const float*>(v.data), static_cast<float*>(out.data), s, g_stream);
    if (e != hipSuccess) return fail(kHipFailure, "flash_attention(f32-mfma): %s", hipGetErrorString(e));
    return finish_launch("flash_attention(f32-mfma)");
  }
  if (staged)
    return fail(kUnsupported, "flash_attention: memory_stage sets the K/V ring depth of the MFMA kernels; this call "
                              "takes the SIMT kernel, which stages nothing through LDS");
  switch (out.dtype) {
    case KG_DTYPE_F32: return launch_fa_simt<float>(out, q, k, v, s);
    case KG_DTYPE_BF16: return launch_fa_simt<__bf16>(out, q, k, v, s);
    default: return launch_fa_simt<_Float16>(out, q, k, v, s);
  }
}

}  // namespace

extern "C" {

int kg_gfx950_matmul_entry(const KgArgSlot* ordered_args, unsigned long long arg_count) {
  return matmul_impl(ordered_args, arg_count);
}

int kg_gfx950_conv2d_entry(const KgArgSlot* ordered_args, unsigned long long arg_count) {
  return conv2d_impl(ordered_args, arg_count);
}

int kg_gfx950_flash_attention_entry(const KgArgSlot* ordered_args, unsigned long long arg_count) {
  return flash_attention_impl(ordered_args, arg_count);
}

int kg_gfx950_fail(int code, const char* message) { return fail(code, "%s", message ? message : ""); }

int kg_gfx950_check_memory_slot(const KgArgSlot* slots, int index, int rank, int allow_absent, int dtype_code,
                                const char* name) {
  if (slots == nullptr) return fail(kInvalid, "ordered_args is null");
  Mem m;
  int rc = read_mem(slots, index, rank, allow_absent != 0, name ? name : "memory", &m);
  if (rc != kOk) return rc;
  if (m.present && dtype_code != 0 && m.dtype != dtype_code)
    return fail(kInvalid, "slot %d (%s): dtype %s, the kernel was generated for %s", index, name ? name : "memory",
                dtype_name(m.dtype), dtype_name(dtype_code));
  return kOk;
}

void* kg_gfx950_launch_stream(void) { return g_stream; }

int kg_gfx950_launch_synchronous(void) { return g_synchronous ? 1 : 0; }

int kg_gfx950_finish_launch(const char* what) { return finish_launch(what ? what : "kernel"); }

int kg_gfx950_set_launch_mode(int synchronous, void* stream) {
  g_synchronous = synchronous != 0;
  g_stream = static_cast<hipStream_t>(stream);
  return kOk;
}

const char* kg_gfx950_last_error(void) { return g_last_error; }

int kg_gfx950_cost(int op, const KgArgSlot* ordered_args, unsigned long long arg_count, long long* costs) {
  if (costs == nullptr) return fail(kInvalid, "cost: output array is null");
  CostOut out{};
  g_cost = &out;
  int rc;
  switch (op) {
    case KG_OP_MATMUL: rc = matmul_impl(ordered_args, arg_count); break;
    case KG_OP_CONV2D: rc = conv2d_impl(ordered_args, arg_count); break;
    case KG_OP_FLASH_ATTENTION: rc = flash_attention_impl(ordered_args, arg_count); break;
    default: rc = fail(kInvalid, "cost: unknown op %d", op);
  }
  g_cost = nullptr;
  if (rc == kOk) {
    for (int i = 0; i < KG_COST_KINDS; ++i) costs[i] = out.v[i];
    g_last_error[0] = '\0';
  }
  return rc;
}

int kg_gfx950_abi_version(void) { return 3; }


}  // extern "C"
