// TEST INFRASTRUCTURE ONLY: C-callable wrappers around the reference's own npu_demo
// primitives, compiled from the header files where they lie under the reference tree
// (include/npu_demo/npu_demo.h), with the reference's flags (g++ -std=c++17 -shared
// -fPIC, no -O: kernel_gen/execute_engine/builtin_strategy/common.py:308-339). Used by
// tests to check the C restatement in kg_oracle.c element for element.
#include "include/npu_demo/npu_demo.h"

#define KGR_EXPORT extern "C" __attribute__((visibility("default")))

namespace {
long long contiguous_strides(const long long* shape, int rank, long long* stride) {
  long long n = 1;
  for (int i = rank - 1; i >= 0; --i) {
    stride[i] = n;
    n *= shape[i];
  }
  return n;
}
}  // namespace

// npu_demo::matmul (include/npu_demo/Kernel.h:900-948) on contiguous [m,k] x [k,n] -> [m,n].
KGR_EXPORT int kgr_matmul(float* out, const float* lhs, const float* rhs, long long m, long long n, long long k, int acc) {
  int ctx = 0;
  long long ls[2] = {m, k}, rs[2] = {k, n}, os[2] = {m, n};
  long long lst[2], rst[2], ost[2];
  contiguous_strides(ls, 2, lst);
  contiguous_strides(rs, 2, rst);
  contiguous_strides(os, 2, ost);
  Memory<TSM, float> L(const_cast<float*>(lhs), ls, lst, 2, MemoryFormat::Norm);
  Memory<TSM, float> R(const_cast<float*>(rhs), rs, rst, 2, MemoryFormat::Norm);
  Memory<TLM1, float> O(out, os, ost, 2, MemoryFormat::Norm);
  return npu_demo::matmul<TSM, TSM, TLM1, float, float, float>(ctx, O, L, R, acc != 0) == StatusCode::kOk ? 0 : -1;
}

// npu_demo::img2col2d (Kernel.h:1041-1123): [n,c,h,w] -> [n,c,kh,kw,ho,wo].
KGR_EXPORT int kgr_img2col2d(float* out, const float* in, long long n, long long c, long long h, long long w, long long kh,
                             long long kw, long long sh, long long sw, long long dh, long long dw, long long ph, long long pw,
                             long long pl, long long pr) {
  int ctx = 0;
  const long long ho = ((h + ph + pw - dh * (kh - 1) - 1) / sh) + 1;
  const long long wo = ((w + pl + pr - dw * (kw - 1) - 1) / sw) + 1;
  long long is[4] = {n, c, h, w}, ist[4];
  long long os[6] = {n, c, kh, kw, ho, wo}, ost[6];
  contiguous_strides(is, 4, ist);
  contiguous_strides(os, 6, ost);
  Memory<GM, float> I(const_cast<float*>(in), is, ist, 4, MemoryFormat::Norm);
  Memory<TSM, float> O(out, os, ost, 6, MemoryFormat::Norm);
  return npu_demo::img2col2d<GM, TSM, float, float>(ctx, O, I, kh, kw, sh, sw, dh, dw, ph, pw, pl, pr) == StatusCode::kOk ? 0 : -1;
}

// npu_demo::exp (Kernel.h:621-641) on a contiguous [rows, cols] tile.
KGR_EXPORT int kgr_exp(float* out, const float* in, long long rows, long long cols) {
  int ctx = 0;
  long long s[2] = {rows, cols}, st[2];
  contiguous_strides(s, 2, st);
  Memory<TSM, float> I(const_cast<float*>(in), s, st, 2, MemoryFormat::Norm);
  Memory<TSM, float> O(out, s, st, 2, MemoryFormat::Norm);
  return npu_demo::exp<TSM, float, float>(ctx, O, I) == StatusCode::kOk ? 0 : -1;
}

// npu_demo::reduce_max / reduce_sum, axis = 1 (Kernel.h:701-750, :831-881).
KGR_EXPORT int kgr_reduce_rows(float* out, const float* in, long long rows, long long cols, int is_max) {
  int ctx = 0;
  long long s[2] = {rows, cols}, st[2];
  long long os[2] = {rows, 1}, ost[2] = {1, 1};
  contiguous_strides(s, 2, st);
  Memory<TSM, float> I(const_cast<float*>(in), s, st, 2, MemoryFormat::Norm);
  Memory<TSM, float> O(out, os, ost, 2, MemoryFormat::Norm);
  const Status r = is_max ? npu_demo::reduce_max<TSM, float, float>(ctx, O, I, 1)
                          : npu_demo::reduce_sum<TSM, float, float>(ctx, O, I, 1);
  return r == StatusCode::kOk ? 0 : -1;
}

// npu_demo::max / truediv (Kernel.h:424-443, :348-371) on contiguous [rows, cols].
KGR_EXPORT int kgr_binary(float* out, const float* lhs, const float* rhs, long long rows, long long cols, int op) {
  int ctx = 0;
  long long s[2] = {rows, cols}, st[2];
  contiguous_strides(s, 2, st);
  Memory<TSM, float> L(const_cast<float*>(lhs), s, st, 2, MemoryFormat::Norm);
  Memory<TSM, float> R(const_cast<float*>(rhs), s, st, 2, MemoryFormat::Norm);
  Memory<TSM, float> O(out, s, st, 2, MemoryFormat::Norm);
  Status r = StatusCode::kError;
  if (op == 0) r = npu_demo::max<TSM, float, float>(ctx, O, L, R);
  else if (op == 1) r = npu_demo::truediv<TSM, float, float>(ctx, O, L, R);
  else if (op == 2) r = npu_demo::sub<TSM, float, float>(ctx, O, L, R);
  else if (op == 3) r = npu_demo::mul<TSM, float, float>(ctx, O, L, R);
  else if (op == 4) r = npu_demo::add<TSM, float, float>(ctx, O, L, R);
  return r == StatusCode::kOk ? 0 : -1;
}
