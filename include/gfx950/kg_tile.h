/*
 * gfx950/kg_tile.h - device runtime of the per-operation gfx950 emitter.
 *
 * The reference renders every operation of a final IR as a call into its target's
 * runtime headers (include/npu_demo/{Kernel,Dma}.h for the host, the include/cuda_sm89 headers
 * for its GPU sibling, where one thread of one block runs the whole body:
 * kernel_gen/dsl/gen_kernel/emit/cuda_sm89/source_bundle.py:615-620). This header is the
 * gfx950 counterpart used by kernels that the pattern pass does not map onto a
 * hand-written kernel: each workgroup runs one iteration of the kernel's parallel outer
 * loops at a time, and every operation is executed cooperatively by the workgroup's
 * threads on strided views of global memory (arguments and the workgroup's slice of a
 * scratch workspace), followed by a workgroup barrier.
 *
 * Arithmetic follows the reference's npu_demo primitives, so results match the host
 * execution bit for bit where the reference's own arithmetic is deterministic:
 *   matmul    sequential k, each product rounded to float before it is added
 *             (include/npu_demo/Kernel.h:900-948), acc = keep the output's value;
 *   exp       (float)exp((double)x)                               (Kernel.h:621-641);
 *   reduce    max from element 0 with `v > cur`, sum from 0 ascending (Kernel.h:701-881);
 *   truediv   (float)((double)a / (double)b); max `a > b ? a : b` (Kernel.h:348-443);
 *   img2col2d out[n,c,kh,kw,ho,wo] = in[n,c,ho*sh+kh*dh-ph, wo*sw+kw*dw-pl] or 0
 *             (Kernel.h:1041-1123; ph/pw are the top/bottom pads, pl/pr left/right).
 *
 * Every view an operation touches is checked against the memory it belongs to; a
 * violation sets the error word (and the operation is skipped), which the generated
 * entry reports as a failed call instead of reading or writing out of bounds.
 */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// Every sum and product below is rounded on its own, in program order, as the reference's
// host code computes it (no fused multiply-add).
#pragma clang fp contract(off)

namespace kg_tile {

constexpr int kThreads = 1024;

// ---- elements -------------------------------------------------------------------------
struct Bf16 {
  uint16_t bits;
};

__device__ __forceinline__ float ld(const float* p) { return *p; }
__device__ __forceinline__ float ld(const _Float16* p) { return (float)*p; }
__device__ __forceinline__ float ld(const Bf16* p) { return __builtin_bit_cast(float, (uint32_t)p->bits << 16); }
__device__ __forceinline__ void st(float* p, float v) { *p = v; }
__device__ __forceinline__ void st(_Float16* p, float v) { *p = (_Float16)v; }
__device__ __forceinline__ void st(Bf16* p, float v) {
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    p->bits = (uint16_t)((u >> 16) | 0x40u);  // NaN stays NaN
    return;
  }
  u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even
  p->bits = (uint16_t)(u >> 16);
}

// ---- integer helpers (Python semantics for // and %) ------------------------------------
__host__ __device__ __forceinline__ long long kg_min(long long a, long long b) { return a < b ? a : b; }
__host__ __device__ __forceinline__ long long kg_max(long long a, long long b) { return a > b ? a : b; }
__host__ __device__ __forceinline__ long long kg_floordiv(long long a, long long b) {
  if (b == 0) return 0;  // never reached: divisors are checked positive before launch
  long long q = a / b;
  if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
  return q;
}
__host__ __device__ __forceinline__ long long kg_mod(long long a, long long b) {
  if (b == 0) return 0;
  return a - kg_floordiv(a, b) * b;
}
__host__ __device__ __forceinline__ long long kg_trips(long long start, long long end, long long step) {
  return (step <= 0 || end <= start) ? 0 : (end - start + step - 1) / step;
}

// ---- views ------------------------------------------------------------------------------
template <typename T, int R>
struct View {
  T* p;
  long long shape[R];
  long long stride[R];
};

template <typename T, int R>
__device__ __forceinline__ long long numel(const View<T, R>& v) {
  long long n = 1;
#pragma unroll
  for (int d = 0; d < R; ++d) n *= v.shape[d] > 0 ? v.shape[d] : 0;
  return n;
}

// Row-major multi-index of element i over R extents (none of them 0), with 32-bit divisions
// where the index and the extents fit: a 64-bit division is a long instruction sequence on
// the GPU, and this runs once per element of every operation.
template <int R>
__device__ __forceinline__ void unravel(long long i, const long long (&shape)[R], long long (&idx)[R]) {
  bool narrow = i <= 0x7fffffffll;
#pragma unroll
  for (int d = 0; d < R; ++d) narrow = narrow && shape[d] <= 0x7fffffffll;
  if (narrow) {
    uint32_t u = (uint32_t)i;
#pragma unroll
    for (int d = R - 1; d >= 0; --d) {
      const uint32_t e = (uint32_t)shape[d];
      idx[d] = u % e;
      u /= e;
    }
    return;
  }
#pragma unroll
  for (int d = R - 1; d >= 0; --d) {
    idx[d] = i % shape[d];
    i /= shape[d];
  }
}

// element offset of the i-th element (row-major order over the view's shape)
template <typename T, int R>
__device__ __forceinline__ long long offset_of(const View<T, R>& v, long long i) {
  long long idx[R];
  unravel(i, v.shape, idx);
  long long off = 0;
#pragma unroll
  for (int d = 0; d < R; ++d) off += idx[d] * v.stride[d];
  return off;
}

// A tile of the workspace: contiguous row-major.
template <typename T, int R>
__device__ __forceinline__ View<T, R> tile(char* base, const long long (&shape)[R]) {
  View<T, R> v;
  v.p = reinterpret_cast<T*>(base);
  long long s = 1;
#pragma unroll
  for (int d = R - 1; d >= 0; --d) {
    v.shape[d] = shape[d] > 0 ? shape[d] : 0;
    v.stride[d] = s;
    s *= v.shape[d] > 0 ? v.shape[d] : 1;
  }
  return v;
}

// Sub-view at offsets / sizes / steps; sets the error word (and returns an empty view)
// when the region leaves the source.
template <typename T, int R>
__device__ __forceinline__ View<T, R> subview(const View<T, R>& src, const long long (&off)[R],
                                              const long long (&size)[R], const long long (&step)[R], int* err) {
  View<T, R> v;
  bool ok = true, empty = false;
  long long base = 0;
#pragma unroll
  for (int d = 0; d < R; ++d) {
    if (size[d] < 0 || step[d] <= 0) ok = false;
    if (size[d] == 0) empty = true;
  }
#pragma unroll
  for (int d = 0; d < R; ++d) {
    if (!empty && (off[d] < 0 || off[d] + (size[d] - 1) * step[d] >= src.shape[d])) ok = false;
    base += off[d] * src.stride[d];
    v.shape[d] = size[d] > 0 ? size[d] : 0;
    v.stride[d] = src.stride[d] * step[d];
  }
  if (!ok) {
    if (threadIdx.x == 0) atomicOr(err, 1);
#pragma unroll
    for (int d = 0; d < R; ++d) v.shape[d] = 0;
    base = 0;
  }
  v.p = src.p + (empty ? 0 : base);
  return v;
}

// Reshape of a row-major contiguous view (the error word is set otherwise, or when the
// element counts differ).
template <int RO, typename T, int R>
__device__ __forceinline__ View<T, RO> reshape(const View<T, R>& src, const long long (&shape)[RO], int* err) {
  bool ok = true;
  long long s = 1;
#pragma unroll
  for (int d = R - 1; d >= 0; --d) {
    if (src.shape[d] != 1 && src.stride[d] != s) ok = false;
    s *= src.shape[d];
  }
  long long n = 1;
#pragma unroll
  for (int d = 0; d < RO; ++d) n *= shape[d] > 0 ? shape[d] : 0;
  if (n != numel(src)) ok = false;
  View<T, RO> v = tile<T, RO>(reinterpret_cast<char*>(src.p), shape);
  if (!ok) {
    if (threadIdx.x == 0) atomicOr(err, 2);
#pragma unroll
    for (int d = 0; d < RO; ++d) v.shape[d] = 0;
  }
  return v;
}

__device__ __forceinline__ void sync() { __syncthreads(); }

// Element loop of the element-wise operations: each thread takes i = threadIdx.x,
// threadIdx.x + kThreads, ... < n, and evaluates kU of its elements (value(i)) before it
// stores them (store(i, v)), so that their loads are in flight together. Each element is
// still read before it is written; elements of different threads were never ordered.
template <typename Value, typename Store>
__device__ __forceinline__ void each_element(long long n, Value value, Store store) {
  constexpr int kU = 4;
  long long i = threadIdx.x;
  for (; i + (kU - 1) * kThreads < n; i += kU * kThreads) {
    float v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) v[u] = value(i + u * kThreads);
#pragma unroll
    for (int u = 0; u < kU; ++u) store(i + u * kThreads, v[u]);
  }
  for (; i < n; i += kThreads) store(i, value(i));
}

// Multi-index of a thread's elements over one shape: the thread's first element, then the
// next one kThreads further on, stepped digit by digit with carries (no division per element).
template <int R>
struct Walk {
  long long idx[R], step[R];
  __device__ __forceinline__ explicit Walk(const long long (&shape)[R]) {
    unravel(threadIdx.x, shape, idx);
    long long t = kThreads;
#pragma unroll
    for (int d = R - 1; d > 0; --d) {
      step[d] = t % shape[d];
      t /= shape[d];
    }
    step[0] = t;
  }
  // every digit below the first stays under its extent: idx + step + carry < 2 * extent
  __device__ __forceinline__ void next(const long long (&shape)[R]) {
    long long c = 0;
#pragma unroll
    for (int d = R - 1; d > 0; --d) {
      idx[d] += step[d] + c;
      c = idx[d] >= shape[d];
      if (c) idx[d] -= shape[d];
    }
    idx[0] += step[0] + c;
  }
  __device__ __forceinline__ long long offset(const long long (&stride)[R]) const {
    long long off = 0;
#pragma unroll
    for (int d = 0; d < R; ++d) off += idx[d] * stride[d];
    return off;
  }
};

// each_element over the n > 0 elements of one shape with a Walk: value(idx) and where(idx)
// (the element's destination) for kU elements, then store(where, v) for them.
template <int R, typename Value, typename Where, typename Store>
__device__ __forceinline__ void each_index(long long n, const long long (&shape)[R], Value value, Where where,
                                           Store store) {
  constexpr int kU = 4;
  Walk<R> w(shape);
  long long i = threadIdx.x;
  for (; i + (kU - 1) * kThreads < n; i += kU * kThreads) {
    float v[kU];
    long long o[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      v[u] = value(w.idx);
      o[u] = where(w.idx);
      w.next(shape);
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) store(o[u], v[u]);
  }
  for (; i < n; i += kThreads) {
    store(where(w.idx), value(w.idx));
    w.next(shape);
  }
}

// ---- dma ----------------------------------------------------------------------------------
template <typename T, int R>
__device__ void fill(const View<T, R>& t, float value) {
  const long long n = numel(t);
  if (n > 0)
    each_index<R>(
        n, t.shape, [&](const long long (&)[R]) { return value; },
        [&](const long long (&idx)[R]) {
          long long off = 0;
#pragma unroll
          for (int d = 0; d < R; ++d) off += idx[d] * t.stride[d];
          return off;
        },
        [&](long long off, float v) { st(t.p + off, v); });
  sync();
}

// dst <- src element by element in row-major order (deslice / slice after their region
// views are formed); the element counts must agree.
template <typename TD, int RD, typename TS, int RS>
__device__ void copy(const View<TD, RD>& dst, const View<TS, RS>& src, int* err) {
  const long long n = numel(dst);
  if (n != numel(src)) {
    if (threadIdx.x == 0 && n > 0) atomicOr(err, 4);
    sync();
    return;
  }
  if constexpr (RD == RS) {
    bool same = n > 0;
#pragma unroll
    for (int d = 0; d < RD; ++d) same = same && dst.shape[d] == src.shape[d];
    if (same) {  // one walk serves both views
      each_index<RD>(
          n, dst.shape, [&](const long long (&idx)[RD]) {
            long long off = 0;
#pragma unroll
            for (int d = 0; d < RD; ++d) off += idx[d] * src.stride[d];
            return ld(src.p + off);
          },
          [&](const long long (&idx)[RD]) {
            long long off = 0;
#pragma unroll
            for (int d = 0; d < RD; ++d) off += idx[d] * dst.stride[d];
            return off;
          },
          [&](long long off, float v) { st(dst.p + off, v); });
      sync();
      return;
    }
  }
  each_element(
      n, [&](long long i) { return ld(src.p + offset_of(src, i)); },
      [&](long long i, float v) { st(dst.p + offset_of(dst, i), v); });
  sync();
}

// dst <- src expanded along its size-1 axes (trailing axes aligned, numpy rules).
template <typename TD, int RD, typename TS, int RS>
__device__ void broadcast(const View<TD, RD>& dst, const View<TS, RS>& src, int* err) {
  static_assert(RS <= RD, "broadcast source rank");
  bool ok = true;
#pragma unroll
  for (int d = 0; d < RS; ++d) {
    const long long sd = src.shape[d], dd = dst.shape[RD - RS + d];
    if (sd != 1 && sd != dd) ok = false;
  }
  if (!ok) {
    if (threadIdx.x == 0) atomicOr(err, 8);
    sync();
    return;
  }
  each_element(
      numel(dst),
      [&](long long i) {
        long long idx[RD], so = 0;
        unravel(i, dst.shape, idx);
#pragma unroll
        for (int d = RD - 1; d >= 0; --d) {
          const int s = d - (RD - RS);
          if (s >= 0 && src.shape[s] != 1) so += idx[d] * src.stride[s];
        }
        return ld(src.p + so);
      },
      [&](long long i, float v) { st(dst.p + offset_of(dst, i), v); });
  sync();
}

// dst[i_0..i_{R-1}] = src[j] with j[perm[d]] = i_d.
template <typename TD, typename TS, int R>
__device__ void transpose(const View<TD, R>& dst, const View<TS, R>& src, const int (&perm)[R], int* err) {
  bool ok = true;
#pragma unroll
  for (int d = 0; d < R; ++d)
    if (dst.shape[d] != src.shape[perm[d]]) ok = false;
  if (!ok) {
    if (threadIdx.x == 0) atomicOr(err, 16);
    sync();
    return;
  }
  each_element(
      numel(dst),
      [&](long long i) {
        long long idx[R], so = 0;
        unravel(i, dst.shape, idx);
#pragma unroll
        for (int d = R - 1; d >= 0; --d) so += idx[d] * src.stride[perm[d]];
        return ld(src.p + so);
      },
      [&](long long i, float v) { st(dst.p + offset_of(dst, i), v); });
  sync();
}

// ---- kernel -------------------------------------------------------------------------------
// Operand staging of matmul: lhs[:, k0:k0+KC] and rhs[k0:k0+KC, :] as fp32 in LDS.
constexpr int kMatmulStage = 4096;  // floats per operand (16 KiB each)

// out (+)= lhs @ rhs. Each output sums its products in k order, one product and one add
// at a time (the reference's arithmetic). Each thread owns a block of up to kB x kB outputs,
// so every operand element it reads feeds kB products (rows and columns past the output are
// computed on clamped indices and not stored). When max(M, N) <= kMatmulStage the operands
// are staged through LDS in k chunks (a workspace tile lives in global memory, and with one
// workgroup per CU its load latency is what the loop waits on); otherwise they are read in
// place.
template <typename TO, typename TL, typename TR>
__device__ void matmul(const View<TO, 2>& out, const View<TL, 2>& lhs, const View<TR, 2>& rhs, bool acc, int* err) {
  const long long M = out.shape[0], N = out.shape[1], K = lhs.shape[1];
  if (lhs.shape[0] != M || rhs.shape[0] != K || rhs.shape[1] != N) {
    if (threadIdx.x == 0) atomicOr(err, 32);
    sync();
    return;
  }
  constexpr int kB = 4;
  const long long mb = (M + kB - 1) / kB, nb = (N + kB - 1) / kB, blocks = mb * nb;
  const bool staged = M <= kMatmulStage && N <= kMatmulStage;
  // kB - 1 floats past each stage: the last k step's block may read (and discard) elements
  // past the chunk's last row or column
  __shared__ float s_l[kMatmulStage + kB], s_r[kMatmulStage + kB];
  // k chunk: M x KC and KC x N floats fit the stages (KC >= 1 when staged)
  const long long mn = M > N ? M : N;
  const long long KC = staged && mn > 0 ? (kMatmulStage / mn < K ? kMatmulStage / mn : K) : K;
  const uint32_t um = (uint32_t)M, un = (uint32_t)N;
  // rounds of kThreads blocks, the same count on every thread (the staging is cooperative)
  for (long long blk0 = 0; blk0 < blocks; blk0 += kThreads) {
    const long long blk = blk0 + threadIdx.x;
    const bool active = blk < blocks;
    const long long m0 = active ? (blk / nb) * kB : 0, n0 = active ? (blk % nb) * kB : 0;
    long long mi[kB], nj[kB];
#pragma unroll
    for (int i = 0; i < kB; ++i) mi[i] = m0 + i < M ? m0 + i : M - 1;
#pragma unroll
    for (int j = 0; j < kB; ++j) nj[j] = n0 + j < N ? n0 + j : N - 1;
    float a[kB][kB];
#pragma unroll
    for (int i = 0; i < kB; ++i)
#pragma unroll
      for (int j = 0; j < kB; ++j)
        a[i][j] = active && acc && m0 + i < M && n0 + j < N
                      ? ld(out.p + (m0 + i) * out.stride[0] + (n0 + j) * out.stride[1])
                      : 0.0f;
    if (staged) {
      for (long long k0 = 0; k0 < K; k0 += KC) {
        const int kc = (int)(K - k0 < KC ? K - k0 : KC);
        // lhs chunk k-major (s_l[k * M + m]: a thread's kB rows are adjacent), rhs row-major;
        // element e of a chunk is read in the operand's row-major order
        const long long lsh[2] = {M, kc}, rsh[2] = {kc, N};
        each_index<2>(
            M * kc, lsh, [&](const long long (&x)[2]) { return ld(lhs.p + x[0] * lhs.stride[0] + (k0 + x[1]) * lhs.stride[1]); },
            [&](const long long (&x)[2]) { return x[1] * M + x[0]; }, [&](long long o, float v) { s_l[(uint32_t)o] = v; });
        each_index<2>(
            (long long)kc * N, rsh,
            [&](const long long (&x)[2]) { return ld(rhs.p + (k0 + x[0]) * rhs.stride[0] + x[1] * rhs.stride[1]); },
            [&](const long long (&x)[2]) { return x[0] * N + x[1]; }, [&](long long o, float v) { s_r[(uint32_t)o] = v; });
        sync();
        if (active) {
          // 32-bit LDS indexes with the block's rows and columns as immediate offsets: rows
          // and columns past the output read neighbouring stage elements, whose products go
          // to accumulators that are not stored
          const uint32_t um0 = (uint32_t)m0, un0 = (uint32_t)n0;
#pragma unroll 4
          for (int k = 0; k < kc; ++k) {
            const uint32_t lo = (uint32_t)k * um + um0, ro = (uint32_t)k * un + un0;
            float lv[kB], rv[kB];
#pragma unroll
            for (int i = 0; i < kB; ++i) lv[i] = s_l[lo + i];
#pragma unroll
            for (int j = 0; j < kB; ++j) rv[j] = s_r[ro + j];
#pragma unroll
            for (int i = 0; i < kB; ++i)
#pragma unroll
              for (int j = 0; j < kB; ++j) {
                const float prod = lv[i] * rv[j];
                a[i][j] = a[i][j] + prod;
              }
          }
        }
        sync();
      }
    } else if (active) {
      const TL* l[kB];
      const TR* r[kB];
#pragma unroll
      for (int i = 0; i < kB; ++i) l[i] = lhs.p + mi[i] * lhs.stride[0];
#pragma unroll
      for (int j = 0; j < kB; ++j) r[j] = rhs.p + nj[j] * rhs.stride[1];
      // unrolled so that the loads of several k steps are in flight together
#pragma unroll 4
      for (long long k = 0; k < K; ++k) {
        float lv[kB], rv[kB];
#pragma unroll
        for (int i = 0; i < kB; ++i) lv[i] = ld(l[i] + k * lhs.stride[1]);
#pragma unroll
        for (int j = 0; j < kB; ++j) rv[j] = ld(r[j] + k * rhs.stride[0]);
#pragma unroll
        for (int i = 0; i < kB; ++i)
#pragma unroll
          for (int j = 0; j < kB; ++j) {
            const float prod = lv[i] * rv[j];
            a[i][j] = a[i][j] + prod;
          }
      }
    }
    if (active) {
#pragma unroll
      for (int i = 0; i < kB; ++i)
#pragma unroll
        for (int j = 0; j < kB; ++j)
          if (m0 + i < M && n0 + j < N) st(out.p + (m0 + i) * out.stride[0] + (n0 + j) * out.stride[1], a[i][j]);
    }
  }
  sync();
}

template <typename TO, typename TI>
__device__ void img2col2d(const View<TO, 6>& out, const View<TI, 4>& in, long long kh, long long kw, long long sh,
                          long long sw, long long dh, long long dw, long long ph, long long pw, long long pl,
                          long long pr, int* err) {
  const long long H = in.shape[2], W = in.shape[3];
  const long long ho = kg_floordiv(H + ph + pw - dh * (kh - 1) - 1, sh) + 1;
  const long long wo = kg_floordiv(W + pl + pr - dw * (kw - 1) - 1, sw) + 1;
  if (out.shape[0] != in.shape[0] || out.shape[1] != in.shape[1] || out.shape[2] != kh || out.shape[3] != kw ||
      out.shape[4] != (ho > 0 ? ho : 0) || out.shape[5] != (wo > 0 ? wo : 0) || sh <= 0 || sw <= 0) {
    if (threadIdx.x == 0) atomicOr(err, 64);
    sync();
    return;
  }
  each_element(
      numel(out),
      [&](long long i) {
        long long idx[6];  // b, c, r (kh), q (kw), y, x: out.shape[2] == kh and out.shape[3] == kw
        unravel(i, out.shape, idx);
        const long long b = idx[0], c = idx[1], r = idx[2], q = idx[3], y = idx[4], x = idx[5];
        const long long sy = y * sh + r * dh - ph, sx = x * sw + q * dw - pl;
        float v = 0.0f;
        if (sy >= 0 && sy < H && sx >= 0 && sx < W)
          v = ld(in.p + b * in.stride[0] + c * in.stride[1] + sy * in.stride[2] + sx * in.stride[3]);
        return v;
      },
      [&](long long i, float v) { st(out.p + offset_of(out, i), v); });
  sync();
}

template <typename TO, int R, typename TI>
__device__ void exp(const View<TO, R>& out, const View<TI, R>& in, int* err) {
  const long long n = numel(out);
  if (n != numel(in)) {
    if (threadIdx.x == 0 && n > 0) atomicOr(err, 128);
    sync();
    return;
  }
  each_element(
      n, [&](long long i) { return ld(in.p + offset_of(in, i)); },
      [&](long long i, float v) { st(out.p + offset_of(out, i), (float)::exp((double)v)); });
  sync();
}

// kind 0 = max, 1 = sum; rows of a rank-2 input into out[rows, 1]
template <typename TO, typename TI>
__device__ void reduce_rows(const View<TO, 2>& out, const View<TI, 2>& in, int kind, int* err) {
  const long long rows = in.shape[0], cols = in.shape[1];
  if (out.shape[0] != rows || out.shape[1] != 1) {
    if (threadIdx.x == 0) atomicOr(err, 256);
    sync();
    return;
  }
  for (long long i = threadIdx.x; i < rows; i += kThreads) {
    const TI* row = in.p + i * in.stride[0];
    float a;
    if (kind == 0) {
      a = cols > 0 ? ld(row) : -__builtin_inff();
      for (long long j = 1; j < cols; ++j) {
        const float v = ld(row + j * in.stride[1]);
        a = v > a ? v : a;
      }
    } else {
      a = 0.0f;
      for (long long j = 0; j < cols; ++j) a = a + ld(row + j * in.stride[1]);
    }
    st(out.p + i * out.stride[0], a);
  }
  sync();
}

// kind 0 add, 1 sub, 2 mul, 3 truediv, 4 max; same shapes
template <typename TO, typename TL, typename TR, int R>
__device__ void binary(const View<TO, R>& out, const View<TL, R>& lhs, const View<TR, R>& rhs, int kind, int* err) {
  bool ok = true;
#pragma unroll
  for (int d = 0; d < R; ++d)
    if (lhs.shape[d] != out.shape[d] || rhs.shape[d] != out.shape[d]) ok = false;
  if (!ok) {
    if (threadIdx.x == 0) atomicOr(err, 512);
    sync();
    return;
  }
  // every element is read before it is written (out may alias an operand); the three views
  // have one shape, so one walk over it serves them all
  const long long n = numel(out);
  if (n > 0)
    each_index<R>(
      n, out.shape,
      [&](const long long (&idx)[R]) {
        long long lo = 0, ro = 0;
#pragma unroll
        for (int d = 0; d < R; ++d) {
          lo += idx[d] * lhs.stride[d];
          ro += idx[d] * rhs.stride[d];
        }
        const float a = ld(lhs.p + lo);
        const float b = ld(rhs.p + ro);
        switch (kind) {
          case 0: return a + b;
          case 1: return a - b;
          case 2: return a * b;
          case 3: return (float)((double)a / (double)b);
          default: return a > b ? a : b;
        }
      },
      [&](const long long (&idx)[R]) {
        long long off = 0;
#pragma unroll
        for (int d = 0; d < R; ++d) off += idx[d] * out.stride[d];
        return off;
      },
      [&](long long off, float v) { st(out.p + off, v); });
  sync();
}

}  // namespace kg_tile
