/*
 * kg_oracle.c - TEST INFRASTRUCTURE ONLY.
 *
 * A CPU restatement, written from scratch in C, of what the reference executes on the
 * host when it runs its matmul / conv2d / flash-attention demos through the npu_demo
 * target (the "cpu-target" path of kernelcode_generate):
 *   - the primitives of include/npu_demo/Kernel.h (matmul :900-948, img2col2d :1041-1123,
 *     exp :621-641, reduce_sum :701-750, reduce_max :831-881, max :424-443,
 *     truediv :348-371) and include/npu_demo/Dma.h (fill/slice/deslice/broadcast),
 *   - the demo loop nests of kernel/matmul/inputs_static_tile_static.py:56-110,
 *     kernel/conv2d/inputs_static_tile_static.py:115-215 and
 *     kernel/flash_attention/inputs_static_tile_static.py:90-190,
 *   - the block-strided top-level loop of kernel_gen/passes/arch/arch_parallelize.py:637-680
 *     run on `threads` host threads (npu_demo::launch, include/npu_demo/Arch.h:809-908).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * code, and only as the checker or the timed CPU baseline. The product path never does.
 *
 * Arithmetic is plain fp32 in the reference's order (build with -ffp-contract=off so no
 * multiply-add is fused), exp is (float)exp((double)x) and division goes through double,
 * as in the reference.
 */
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define KGO_EXPORT __attribute__((visibility("default")))

/* ---------------------------------------------------------------------------------- */
/* Primitives                                                                          */
/* ---------------------------------------------------------------------------------- */

/* npu_demo::matmul (Kernel.h:900-948): out[m,n] (=|+=) sum_k lhs[m,k]*rhs[k,n], k ascending,
 * every step rounded to float. Row strides in elements. */
KGO_EXPORT void kgo_matmul(float* out, long ldo, const float* lhs, long ldl, const float* rhs, long ldr, long m,
                           long n, long k, int acc) {
  for (long mi = 0; mi < m; ++mi) {
    for (long ni = 0; ni < n; ++ni) {
      float a = acc ? out[mi * ldo + ni] : 0.0f;
      for (long ki = 0; ki < k; ++ki) {
        const float prod = lhs[mi * ldl + ki] * rhs[ki * ldr + ni];
        a = a + prod;
      }
      out[mi * ldo + ni] = a;
    }
  }
}

/* npu_demo::img2col2d (Kernel.h:1041-1123): [N,C,H,W] -> [N,C,KH,KW,Ho,Wo]; ph/pw are the
 * top/bottom pads and pl/pr left/right (Kernel.h:1077-1078). Returns 0, or -1 like kError. */
KGO_EXPORT int kgo_img2col2d(float* out, const float* in, long n, long c, long h, long w, long kh, long kw, long sh,
                             long sw, long dh, long dw, long ph, long pw, long pl, long pr) {
  if (kh <= 0 || kw <= 0 || sh <= 0 || sw <= 0 || dh <= 0 || dw <= 0) return -1;
  if (ph < 0 || pw < 0 || pl < 0 || pr < 0) return -1;
  const long ho = ((h + ph + pw - dh * (kh - 1) - 1) / sh) + 1;
  const long wo = ((w + pl + pr - dw * (kw - 1) - 1) / sw) + 1;
  if (n <= 0 || c <= 0 || h <= 0 || w <= 0 || ho <= 0 || wo <= 0) return -1;
  long o = 0;
  for (long ni = 0; ni < n; ++ni)
    for (long ci = 0; ci < c; ++ci) {
      const float* plane = in + (ni * c + ci) * h * w;
      for (long r = 0; r < kh; ++r)
        for (long q = 0; q < kw; ++q)
          for (long y = 0; y < ho; ++y) {
            const long sy = y * sh + r * dh - ph;
            for (long x = 0; x < wo; ++x) {
              const long sx = x * sw + q * dw - pl;
              out[o++] = (sy < 0 || sy >= h || sx < 0 || sx >= w) ? 0.0f : plane[sy * w + sx];
            }
          }
    }
  return 0;
}

/* npu_demo::exp (Kernel.h:621-641): computed in double, cast to float. */
KGO_EXPORT float kgo_exp(float x) { return (float)exp((double)x); }

/* npu_demo::reduce_max axis=1 (Kernel.h:831-881): starts from element 0, keeps a when
 * value > current is false. */
KGO_EXPORT void kgo_reduce_max_rows(float* out, const float* in, long rows, long cols, long ld) {
  for (long i = 0; i < rows; ++i) {
    float cur = in[i * ld];
    for (long j = 1; j < cols; ++j) {
      const float v = in[i * ld + j];
      cur = v > cur ? v : cur;
    }
    out[i] = cur;
  }
}

/* npu_demo::reduce_sum axis=1 (Kernel.h:701-750): starts from 0, ascending. */
KGO_EXPORT void kgo_reduce_sum_rows(float* out, const float* in, long rows, long cols, long ld) {
  for (long i = 0; i < rows; ++i) {
    float acc = 0.0f;
    for (long j = 0; j < cols; ++j) acc = acc + in[i * ld + j];
    out[i] = acc;
  }
}

static inline float kgo_max2(float a, float b) { return a > b ? a : b; } /* Kernel.h:431 */
static inline float kgo_div(float a, float b) { return (float)((double)a / (double)b); } /* Kernel.h:365-370 */

/* ---------------------------------------------------------------------------------- */
/* Block-strided top-level loop on host threads                                        */
/* ---------------------------------------------------------------------------------- */

typedef void (*kgo_body_fn)(void* ctx, long iter);

typedef struct {
  kgo_body_fn body;
  void* ctx;
  long start, end, step, bid, nblocks;
} kgo_worker;

static void* kgo_worker_main(void* arg) {
  kgo_worker* w = (kgo_worker*)arg;
  /* arch_parallelize.py:637-680: start + bid*step, step*block_num */
  for (long i = w->start + w->bid * w->step; i < w->end; i += w->step * w->nblocks) w->body(w->ctx, i);
  return NULL;
}

static void kgo_launch(kgo_body_fn body, void* ctx, long start, long end, long step, int threads) {
  if (threads <= 1) {
    for (long i = start; i < end; i += step) body(ctx, i);
    return;
  }
  pthread_t tids[64];
  kgo_worker ws[64];
  if (threads > 64) threads = 64;
  for (int b = 0; b < threads; ++b) {
    ws[b].body = body;
    ws[b].ctx = ctx;
    ws[b].start = start;
    ws[b].end = end;
    ws[b].step = step;
    ws[b].bid = b;
    ws[b].nblocks = threads;
    pthread_create(&tids[b], NULL, kgo_worker_main, &ws[b]);
  }
  for (int b = 0; b < threads; ++b) pthread_join(tids[b], NULL);
}

static long kgo_min(long a, long b) { return a < b ? a : b; }
static long kgo_maxl(long a, long b) { return a > b ? a : b; }

/* ---------------------------------------------------------------------------------- */
/* Matmul demo (kernel/matmul/inputs_static_tile_static.py:56-110)                      */
/* ---------------------------------------------------------------------------------- */

typedef struct {
  float* out;
  const float *lhs, *rhs, *bias;
  long M, N, K, tm, tn, tk;
  int fused;
} kgo_mm_ctx;

static void kgo_mm_body(void* vctx, long m0) {
  const kgo_mm_ctx* c = (const kgo_mm_ctx*)vctx;
  const long cur_m = kgo_min(c->tm, c->M - m0);
  float* lt = (float*)malloc(sizeof(float) * (size_t)(c->tm * c->tk));
  float* rt = (float*)malloc(sizeof(float) * (size_t)(c->tk * c->tn));
  float* acc = (float*)malloc(sizeof(float) * (size_t)(c->tm * c->tn));
  float* part = (float*)malloc(sizeof(float) * (size_t)(c->tm * c->tn));
  for (long n0 = 0; n0 < c->N; n0 += c->tn) {
    const long cur_n = kgo_min(c->tn, c->N - n0);
    memset(acc, 0, sizeof(float) * (size_t)(cur_m * cur_n)); /* fill(acc, 0) */
    for (long k0 = 0; k0 < c->K; k0 += c->tk) {
      const long cur_k = kgo_min(c->tk, c->K - k0);
      for (long i = 0; i < cur_m; ++i) memcpy(lt + i * cur_k, c->lhs + (m0 + i) * c->K + k0, sizeof(float) * (size_t)cur_k);
      for (long i = 0; i < cur_k; ++i) memcpy(rt + i * cur_n, c->rhs + (k0 + i) * c->N + n0, sizeof(float) * (size_t)cur_n);
      if (c->fused) {
        /* KernelAggregatePass(matmul_acc=True) (kernel_gen/passes/kernel/kernel_aggregate.py:292,
         * npu_demo_lowering.py:134): matmul(acc, lhs, rhs, acc = k0 != k_start). */
        kgo_matmul(acc, cur_n, lt, cur_k, rt, cur_n, cur_m, cur_n, cur_k, k0 != 0);
      } else {
        kgo_matmul(part, cur_n, lt, cur_k, rt, cur_n, cur_m, cur_n, cur_k, 0);
        for (long e = 0; e < cur_m * cur_n; ++e) acc[e] = acc[e] + part[e]; /* kernel.add */
      }
    }
    if (c->bias != NULL)
      for (long i = 0; i < cur_m; ++i)
        for (long j = 0; j < cur_n; ++j) acc[i * cur_n + j] = acc[i * cur_n + j] + c->bias[n0 + j];
    for (long i = 0; i < cur_m; ++i) memcpy(c->out + (m0 + i) * c->N + n0, acc + i * cur_n, sizeof(float) * (size_t)cur_n);
  }
  free(lt);
  free(rt);
  free(acc);
  free(part);
}

/* out[M,N] = lhs[M,K] @ rhs[K,N] (+ bias[N]); tiles (tm, tn, tk); fused != 0 follows the
 * npu-demo-lowering pipeline (sequential k over the whole K), fused == 0 the unlowered
 * DSL text (per-k-tile partial sums added into acc). Optional row range [m_begin, m_end)
 * (in tile-aligned rows) lets the CPU baseline time a sample of outer tiles. */
KGO_EXPORT void kgo_matmul_demo(float* out, const float* lhs, const float* rhs, const float* bias, long M, long N,
                                long K, long tm, long tn, long tk, int fused, int threads, long m_begin, long m_end) {
  kgo_mm_ctx c = {out, lhs, rhs, bias, M, N, K, tm, tn, tk, fused};
  if (m_end <= 0 || m_end > M) m_end = M;
  kgo_launch(kgo_mm_body, &c, m_begin, m_end, tm, threads);
}

/* ---------------------------------------------------------------------------------- */
/* Conv2d demo (kernel/conv2d/inputs_static_tile_static.py:115-215)                     */
/* ---------------------------------------------------------------------------------- */

typedef struct {
  float* out;
  const float *x, *w, *bias;
  long N, C, H, W, F, KH, KW, sh, sw, dh, dw, pt, pb, pl, pr, Ho, Wo;
  long tf, tc, tn, tho, two;
} kgo_conv_ctx;

static void kgo_conv_body(void* vctx, long f0) {
  const kgo_conv_ctx* c = (const kgo_conv_ctx*)vctx;
  const long cur_f = kgo_min(c->tf, c->F - f0);
  const long kk_max = c->tc * c->KH * c->KW;
  const long sp_max = c->tho * c->two;
  float* col = (float*)malloc(sizeof(float) * (size_t)(kk_max * sp_max));
  float* wt = (float*)malloc(sizeof(float) * (size_t)(c->tf * kk_max));
  float* out2 = (float*)malloc(sizeof(float) * (size_t)(c->tf * sp_max));
  float* acc = (float*)malloc(sizeof(float) * (size_t)(c->tf * sp_max));
  float* win = NULL;
  size_t win_cap = 0;
  for (long n0 = 0; n0 < c->N; n0 += c->tn) {
    const long cur_n = kgo_min(c->tn, c->N - n0);
    for (long ho0 = 0; ho0 < c->Ho; ho0 += c->tho) {
      const long cur_ho = kgo_min(c->tho, c->Ho - ho0);
      for (long wo0 = 0; wo0 < c->Wo; wo0 += c->two) {
        const long cur_wo = kgo_min(c->two, c->Wo - wo0);
        const long sp = cur_ho * cur_wo;
        const long h_origin = ho0 * c->sh - c->pt;
        const long w_origin = wo0 * c->sw - c->pl;
        const long h_wend = (ho0 + cur_ho - 1) * c->sh - c->pt + (c->KH - 1) * c->dh + 1;
        const long w_wend = (wo0 + cur_wo - 1) * c->sw - c->pl + (c->KW - 1) * c->dw + 1;
        const long h_start = kgo_maxl(h_origin, 0), w_start = kgo_maxl(w_origin, 0);
        const long h_end = kgo_min(h_wend, c->H), w_end = kgo_min(w_wend, c->W);
        const long ih = h_end - h_start, iw = w_end - w_start;
        const long lpt = kgo_maxl(c->pt - ho0 * c->sh, 0), lpl = kgo_maxl(c->pl - wo0 * c->sw, 0);
        const long lpb = kgo_maxl(h_wend - c->H, 0), lpr = kgo_maxl(w_wend - c->W, 0);
        for (long ni = 0; ni < cur_n; ++ni) {
          const long b = n0 + ni;
          for (long e = 0; e < cur_f * sp; ++e) acc[e] = 0.0f; /* fill(acc, 0) */
          for (long c0 = 0; c0 < c->C; c0 += c->tc) {
            const long cur_c = kgo_min(c->tc, c->C - c0);
            const long kt = cur_c * c->KH * c->KW;
            /* weight tile [cur_f, cur_c, KH, KW] reshaped to [cur_f, kt] */
            for (long fi = 0; fi < cur_f; ++fi)
              for (long ci = 0; ci < cur_c; ++ci)
                memcpy(wt + fi * kt + ci * c->KH * c->KW, c->w + ((f0 + fi) * c->C + c0 + ci) * c->KH * c->KW,
                       sizeof(float) * (size_t)(c->KH * c->KW));
            if (ih <= 0 || iw <= 0) {
              /* The output tile's receptive field lies entirely in the zero padding (only
               * possible with tiny tiles and pads): every column entry is a padded zero. */
              memset(col, 0, sizeof(float) * (size_t)(kt * sp));
            } else {
              /* slice the clipped input window [1, cur_c, ih, iw] */
              const size_t need = (size_t)(cur_c * ih * iw);
              if (need > win_cap) {
                free(win);
                win = (float*)malloc(sizeof(float) * need);
                win_cap = need;
              }
              for (long ci = 0; ci < cur_c; ++ci)
                for (long y = 0; y < ih; ++y)
                  memcpy(win + (ci * ih + y) * iw, c->x + (((b * c->C) + c0 + ci) * c->H + h_start + y) * c->W + w_start,
                         sizeof(float) * (size_t)iw);
              if (kgo_img2col2d(col, win, 1, cur_c, ih, iw, c->KH, c->KW, c->sh, c->sw, c->dh, c->dw, lpt, lpb, lpl, lpr) != 0)
                memset(col, 0, sizeof(float) * (size_t)(kt * sp));
            }
            kgo_matmul(out2, sp, wt, kt, col, sp, cur_f, sp, kt, 0);
            for (long e = 0; e < cur_f * sp; ++e) acc[e] = acc[e] + out2[e]; /* transpose + add */
          }
          if (c->bias != NULL)
            for (long fi = 0; fi < cur_f; ++fi)
              for (long e = 0; e < sp; ++e) acc[fi * sp + e] = acc[fi * sp + e] + c->bias[f0 + fi];
          for (long fi = 0; fi < cur_f; ++fi)
            for (long y = 0; y < cur_ho; ++y)
              memcpy(c->out + ((b * c->F + f0 + fi) * c->Ho + ho0 + y) * c->Wo + wo0, acc + fi * sp + y * cur_wo,
                     sizeof(float) * (size_t)cur_wo);
        }
      }
    }
  }
  free(win);
  free(col);
  free(wt);
  free(out2);
  free(acc);
}

/* out[N,F,Ho,Wo] = conv2d(x[N,C,H,W], w[F,C,KH,KW]) (+ bias[F]) with stride (sh,sw),
 * dilation (dh,dw), pads top/bottom/left/right; tiles (tf, tc, tn, tho, two). The f0 range
 * [f_begin, f_end) selects a sample of outer tiles for timing (f_end <= 0: all). */
KGO_EXPORT int kgo_conv2d_demo(float* out, const float* x, const float* w, const float* bias, long N, long C, long H,
                               long W, long F, long KH, long KW, long sh, long sw, long dh, long dw, long pt, long pb,
                               long pl, long pr, long tf, long tc, long tn, long tho, long two, int threads,
                               long f_begin, long f_end) {
  kgo_conv_ctx c;
  c.out = out;
  c.x = x;
  c.w = w;
  c.bias = bias;
  c.N = N; c.C = C; c.H = H; c.W = W; c.F = F; c.KH = KH; c.KW = KW;
  c.sh = sh; c.sw = sw; c.dh = dh; c.dw = dw; c.pt = pt; c.pb = pb; c.pl = pl; c.pr = pr;
  c.Ho = (H + pt + pb - dh * (KH - 1) - 1) / sh + 1;
  c.Wo = (W + pl + pr - dw * (KW - 1) - 1) / sw + 1;
  c.tf = tf; c.tc = tc; c.tn = tn; c.tho = tho; c.two = two;
  if (c.Ho <= 0 || c.Wo <= 0) return -1;
  if (f_end <= 0 || f_end > F) f_end = F;
  kgo_launch(kgo_conv_body, &c, f_begin, f_end, tf, threads);
  return 0;
}

/* ---------------------------------------------------------------------------------- */
/* Flash-attention demo (kernel/flash_attention/inputs_static_tile_static.py:90-190)    */
/* ---------------------------------------------------------------------------------- */

typedef struct {
  float* out;
  const float *q, *k, *v;
  long B, H, S, D, br, bc;
  float scale;
  int causal;
  int apply_scale;
  long m_begin, m_end; /* query-block range per head (m_end <= 0: all) */
} kgo_fa_ctx;

static void kgo_fa_head(const kgo_fa_ctx* c, long b0, long h0) {
  const long S = c->S, D = c->D, br = c->br, bc = c->bc;
  float* qf = (float*)malloc(sizeof(float) * (size_t)(br * D));
  float* kf = (float*)malloc(sizeof(float) * (size_t)(bc * D));
  float* kt = (float*)malloc(sizeof(float) * (size_t)(D * bc));
  float* vf = (float*)malloc(sizeof(float) * (size_t)(bc * D));
  float* score = (float*)malloc(sizeof(float) * (size_t)(br * bc));
  float* st = (float*)malloc(sizeof(float) * (size_t)(br * bc));
  float* ex = (float*)malloc(sizeof(float) * (size_t)(br * bc));
  float* part = (float*)malloc(sizeof(float) * (size_t)(br * D));
  float* wgt = (float*)malloc(sizeof(float) * (size_t)(br * D));
  float* mst = (float*)malloc(sizeof(float) * (size_t)br);
  float* sst = (float*)malloc(sizeof(float) * (size_t)br);
  float* tmax = (float*)malloc(sizeof(float) * (size_t)br);
  float* tsum = (float*)malloc(sizeof(float) * (size_t)br);
  const long head = (b0 * c->H + h0) * S * D;
  const long m_end = (c->m_end <= 0 || c->m_end > S) ? S : c->m_end;
  for (long m0 = c->m_begin; m0 < m_end; m0 += br) {
    const long cur_br = kgo_min(br, S - m0);
    memset(qf, 0, sizeof(float) * (size_t)(br * D));
    memcpy(qf, c->q + head + m0 * D, sizeof(float) * (size_t)(cur_br * D));
    for (long i = 0; i < br; ++i) {
      mst[i] = -INFINITY;
      sst[i] = 0.0f;
    }
    memset(wgt, 0, sizeof(float) * (size_t)(br * D));
    /* causal extension: key blocks past the query block are skipped entirely */
    const long n_end = c->causal ? kgo_min(S, m0 + br) : S;
    for (long n0 = 0; n0 < n_end; n0 += bc) {
      const long cur_bc = kgo_min(bc, S - n0);
      memset(kf, 0, sizeof(float) * (size_t)(bc * D));
      memcpy(kf, c->k + head + n0 * D, sizeof(float) * (size_t)(cur_bc * D));
      for (long j = 0; j < bc; ++j)
        for (long d = 0; d < D; ++d) kt[d * bc + j] = kf[j * D + d]; /* nn.transpose */
      kgo_matmul(score, bc, qf, D, kt, bc, br, bc, D, 0);
      for (long e = 0; e < br * bc; ++e) st[e] = -INFINITY; /* fill(score_tile, "-inf") */
      for (long i = 0; i < cur_br; ++i)
        for (long j = 0; j < cur_bc; ++j) {
          float s = score[i * bc + j];
          if (c->apply_scale) s = s * c->scale; /* scale extension: kernel.mul by a 1/sqrt(D) tile */
          if (c->causal && n0 + j > m0 + i) s = -INFINITY; /* causal extension: 0/-inf mask add */
          st[i * bc + j] = s;
        }
      kgo_reduce_max_rows(tmax, st, br, bc, bc);
      for (long i = 0; i < br; ++i) tmax[i] = kgo_max2(mst[i], tmax[i]); /* m_next */
      for (long i = 0; i < br; ++i)
        for (long j = 0; j < bc; ++j) ex[i * bc + j] = kgo_exp(st[i * bc + j] - tmax[i]);
      kgo_reduce_sum_rows(tsum, ex, br, bc, bc);
      memset(vf, 0, sizeof(float) * (size_t)(bc * D));
      memcpy(vf, c->v + head + n0 * D, sizeof(float) * (size_t)(cur_bc * D));
      kgo_matmul(part, D, ex, bc, vf, D, br, D, bc, 0);
      for (long i = 0; i < br; ++i) {
        const float old_scale = kgo_exp(mst[i] - tmax[i]);
        sst[i] = sst[i] * old_scale + tsum[i];
        for (long d = 0; d < D; ++d) wgt[i * D + d] = wgt[i * D + d] * old_scale + part[i * D + d];
        mst[i] = tmax[i];
      }
    }
    for (long i = 0; i < cur_br; ++i)
      for (long d = 0; d < D; ++d) c->out[head + (m0 + i) * D + d] = kgo_div(wgt[i * D + d], sst[i]);
  }
  free(qf); free(kf); free(kt); free(vf); free(score); free(st); free(ex);
  free(part); free(wgt); free(mst); free(sst); free(tmax); free(tsum);
}

static void kgo_fa_body(void* vctx, long b0) {
  const kgo_fa_ctx* c = (const kgo_fa_ctx*)vctx;
  for (long h0 = 0; h0 < c->H; ++h0) kgo_fa_head(c, b0, h0);
}

/* out/q/k/v [B,H,S,D]; tiles (br, bc). The reference demo has no scale and no mask
 * (apply_scale = 0, causal = 0). The query range [m_begin, m_end) per head selects a
 * sample of query blocks for timing (m_end <= 0: all). */
KGO_EXPORT void kgo_flash_attention_demo(float* out, const float* q, const float* k, const float* v, long B, long H,
                                         long S, long D, long br, long bc, int apply_scale, float scale, int causal,
                                         int threads, long m_begin, long m_end) {
  kgo_fa_ctx c;
  c.out = out;
  c.q = q;
  c.k = k;
  c.v = v;
  c.B = B; c.H = H; c.S = S; c.D = D; c.br = br; c.bc = bc;
  c.scale = scale;
  c.causal = causal;
  c.apply_scale = apply_scale;
  c.m_begin = m_begin;
  c.m_end = m_end;
  kgo_launch(kgo_fa_body, &c, 0, B, 1, threads);
}
