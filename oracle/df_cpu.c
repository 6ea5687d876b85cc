/*
 * df_cpu.c -- C restatement (fp32, OpenMP) of the reference Depthformer decode
 * steps: Depthformer::temporal_step (depthformer/model.cpp:322-514) and
 * Depthformer::depth_step (model.cpp:516-659) with the layers of
 * depthformer/modules.cpp:72-455 and nn_ops.h:66-98.
 *
 * TEST INFRASTRUCTURE ONLY: a second, independent CPU restatement that the
 * numpy oracle is checked against (tests/test_oracle_c.py), and the CPU
 * baseline that bench.py times at 1 thread and at every core.  Nothing in the
 * product links or loads it.
 *
 * Layout (all fp32, row-major):
 *   stacked weights of one stack (temporal or depth), layer i at i * size:
 *     norm_sa (L, D), wq / wk / wv (L, HD, D), wo (L, D, HD), [norm_ca (L, D),
 *     cq (L, HD, D), co (L, D, HD)], norm_ff (L, D), wi0 / wi1 (L, F, D),
 *     wo2 (L, D, F) -- Linear weights stored (out, in) (modules.h:74-76);
 *   self K/V cache of layer i: k, v (L, 2, H, Lmax, 64), slot = position;
 *   cross K/V of layer i: ck, cv (L, 2, H, S, 64);
 *   bias table (buckets, H) and the bucket of each distance n (n < nb).
 */
#include <math.h>
#include <stddef.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef struct {
  int L, D, HD, H, F;
  int cross;                  /* temporal stack: cross attention after self attention */
  const float *norm_sa, *wq, *wk, *wv, *wo;
  const float *norm_ca, *cq, *co;
  const float *norm_ff, *wi0, *wi1, *wo2;
  const float* bias_tab;      /* (buckets, H) */
  const int* buckets;         /* bucket of distance n */
} df_stack;

void df_set_threads(int n) {
#ifdef _OPENMP
  omp_set_num_threads(n > 0 ? n : 1);
#else
  (void)n;
#endif
}

int df_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* x * rsqrt(mean(x^2) + 1e-6) rounded, times w (modules.cpp:72-84) */
static void rms_norm(const float* x, const float* w, int D, float* y) {
  float ss = 0.f;
  for (int i = 0; i < D; ++i) ss += x[i] * x[i];
  const float inv = 1.0f / sqrtf(ss / (float)D + 1e-6f);
  for (int i = 0; i < D; ++i) y[i] = (x[i] * inv) * w[i];
}

/* y_r = W x_r for both CFG rows, W (N, K); one pass over W */
static void gemv2(const float* W, const float* x0, const float* x1, int N, int K, float* y0, float* y1) {
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n) {
    const float* w = W + (size_t)n * K;
    float a0 = 0.f, a1 = 0.f;
#pragma omp simd reduction(+ : a0, a1)
    for (int k = 0; k < K; ++k) {
      a0 += w[k] * x0[k];
      a1 += w[k] * x1[k];
    }
    y0[n] = a0;
    y1[n] = a1;
  }
}

/* tanh GELU with float32 constants (nn_ops.h:66-98) */
static float gelu_t(float x) {
  const float c0 = 0.7978845608028654f, c1 = 0.044715f;
  return 0.5f * (x * (1.0f + tanhf(c0 * (x * (1.0f + c1 * (x * x))))));
}

/* softmax(q . k_j + bias_j) . v over n keys of one head; k/v rows of 64 */
static void attend(const float* q, const float* K, const float* V, int n, const float* bias, float* out) {
  float* s = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
  float mx = -INFINITY;
  for (int j = 0; j < n; ++j) {
    float a = 0.f;
#pragma omp simd reduction(+ : a)
    for (int d = 0; d < 64; ++d) a += q[d] * K[(size_t)j * 64 + d];
    s[j] = a + (bias ? bias[j] : 0.f);
    if (s[j] > mx) mx = s[j];
  }
  float z = 0.f;
  for (int j = 0; j < n; ++j) {
    s[j] = expf(s[j] - mx);
    z += s[j];
  }
  float o[64] = {0.f};
  for (int j = 0; j < n; ++j)
#pragma omp simd
    for (int d = 0; d < 64; ++d) o[d] += s[j] * V[(size_t)j * 64 + d];
  for (int d = 0; d < 64; ++d) out[d] = o[d] / z;
  free(s);
}

/*
 * One decoder stack at ring position `pos` for the two CFG rows (x: 2 x D,
 * updated in place): per layer pre-norm self attention over slots 0..pos
 * (bias table[bucket(pos - j), h], scale 1.0; modules.cpp:243-295), residual,
 * [pre-norm cross attention over S keys, residual], pre-norm gated GELU FFN,
 * residual (modules.cpp:384-408).  K/V of position pos are written to the
 * self cache.
 */
static void run_stack(const df_stack* st, float* x, int pos, float* kc, float* vc, int Lmax, const float* ck,
                      const float* cv, int S) {
  const int D = st->D, HD = st->HD, H = st->H, F = st->F;
  const int M = D > F ? D : F;
  float* xn = (float*)malloc(sizeof(float) * 2 * (size_t)M);
  float* q = (float*)malloc(sizeof(float) * 2 * (size_t)HD);
  float* k = (float*)malloc(sizeof(float) * 2 * (size_t)HD);
  float* v = (float*)malloc(sizeof(float) * 2 * (size_t)HD);
  float* at = (float*)malloc(sizeof(float) * 2 * (size_t)HD);
  float* y = (float*)malloc(sizeof(float) * 2 * (size_t)M);
  float* g = (float*)malloc(sizeof(float) * 2 * (size_t)F);
  float* u = (float*)malloc(sizeof(float) * 2 * (size_t)F);
  float* bias = (float*)malloc(sizeof(float) * 2 * (size_t)H * (size_t)(pos + 1));
  for (int li = 0; li < st->L; ++li) {
    const size_t dd = (size_t)li * D, qd = (size_t)li * HD * D, oq = (size_t)li * D * HD;
    const size_t fd = (size_t)li * F * D, df = (size_t)li * D * F;
    /* self attention */
    for (int r = 0; r < 2; ++r) rms_norm(x + r * D, st->norm_sa + dd, D, xn + r * M);
    gemv2(st->wq + qd, xn, xn + M, HD, D, q, q + HD);
    gemv2(st->wk + qd, xn, xn + M, HD, D, k, k + HD);
    gemv2(st->wv + qd, xn, xn + M, HD, D, v, v + HD);
    for (int r = 0; r < 2; ++r)
      for (int h = 0; h < H; ++h) {
        const size_t base = ((((size_t)li * 2 + r) * H + h) * Lmax) * 64;
        memcpy(kc + base + (size_t)pos * 64, k + r * HD + h * 64, 64 * sizeof(float));
        memcpy(vc + base + (size_t)pos * 64, v + r * HD + h * 64, 64 * sizeof(float));
      }
#pragma omp parallel for schedule(static)
    for (int rh = 0; rh < 2 * H; ++rh) {
      const int r = rh / H, h = rh % H;
      float* bh = bias + (size_t)rh * (pos + 1);
      for (int j = 0; j <= pos; ++j) bh[j] = st->bias_tab[st->buckets[pos - j] * H + h];
      const size_t base = ((((size_t)li * 2 + r) * H + h) * Lmax) * 64;
      attend(q + r * HD + h * 64, kc + base, vc + base, pos + 1, bh, at + r * HD + h * 64);
    }
    gemv2(st->wo + oq, at, at + HD, D, HD, y, y + M);
    for (int r = 0; r < 2; ++r)
      for (int i = 0; i < D; ++i) x[r * D + i] += y[r * M + i];
    /* cross attention over the encoder K/V */
    if (st->cross) {
      for (int r = 0; r < 2; ++r) rms_norm(x + r * D, st->norm_ca + dd, D, xn + r * M);
      gemv2(st->cq + qd, xn, xn + M, HD, D, q, q + HD);
#pragma omp parallel for schedule(static)
      for (int rh = 0; rh < 2 * H; ++rh) {
        const int r = rh / H, h = rh % H;
        const size_t base = ((((size_t)li * 2 + r) * H + h) * (size_t)S) * 64;
        attend(q + r * HD + h * 64, ck + base, cv + base, S, NULL, at + r * HD + h * 64);
      }
      gemv2(st->co + oq, at, at + HD, D, HD, y, y + M);
      for (int r = 0; r < 2; ++r)
        for (int i = 0; i < D; ++i) x[r * D + i] += y[r * M + i];
    }
    /* gated GELU feed-forward (modules.cpp:222-226) */
    for (int r = 0; r < 2; ++r) rms_norm(x + r * D, st->norm_ff + dd, D, xn + r * M);
    gemv2(st->wi0 + fd, xn, xn + M, F, D, g, g + F);
    gemv2(st->wi1 + fd, xn, xn + M, F, D, u, u + F);
    for (int i = 0; i < 2 * F; ++i) g[i] = gelu_t(g[i]) * u[i];
    gemv2(st->wo2 + df, g, g + F, D, F, y, y + M);
    for (int r = 0; r < 2; ++r)
      for (int i = 0; i < D; ++i) x[r * D + i] += y[r * M + i];
  }
  free(xn);
  free(q);
  free(k);
  free(v);
  free(at);
  free(y);
  free(g);
  free(u);
  free(bias);
}

/* temporal_step: in/out (2, D); caches as in the file comment; no final norm */
void df_temporal_step(const df_stack* st, const float* in, int frame_idx, float* kc, float* vc, int Lmax,
                      const float* ck, const float* cv, int S, float* out) {
  memcpy(out, in, sizeof(float) * 2 * (size_t)st->D);
  run_stack(st, out, frame_idx, kc, vc, Lmax, ck, cv, S);
}

/* depth_step: in (2, D); decoder_norm, then `head_rows` lm_head rows from
 * head_w (a level slice or the whole vocabulary) -> logits (2, head_rows) */
void df_depth_step(const df_stack* st, const float* in, int depth_idx, float* kc, float* vc, int Lmax,
                   const float* dec_norm, const float* head_w, int head_rows, float* logits) {
  const int D = st->D;
  float* x = (float*)malloc(sizeof(float) * 2 * (size_t)D);
  float* xn = (float*)malloc(sizeof(float) * 2 * (size_t)D);
  memcpy(x, in, sizeof(float) * 2 * (size_t)D);
  run_stack(st, x, depth_idx, kc, vc, Lmax, NULL, NULL, 0);
  for (int r = 0; r < 2; ++r) rms_norm(x + r * D, dec_norm, D, xn + r * D);
  gemv2(head_w, xn, xn + D, head_rows, D, logits, logits + head_rows);
  free(x);
  free(xn);
}
