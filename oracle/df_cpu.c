/*
 * df_cpu.c -- C restatement (OpenMP) of the reference Depthformer streaming
 * decode of one chunk: Depthformer::encode (depthformer/model.cpp:226-241)
 * with the encoder layers of modules.cpp:349-358, the cross K/V projection
 * (DecoderLayer::precompute_cross_kv, modules.cpp:448-455),
 * Depthformer::temporal_step (model.cpp:322-514), Depthformer::depth_step
 * (model.cpp:516-659) with the layers of modules.cpp:72-455 and nn_ops.h:66-98,
 * and the generate_tokens loop (depthformer/decode.cpp:239-573: CFG
 * decode.cpp:71-85, top-k decode.cpp:104-122, the draw decode.cpp:124-148,
 * the feedback and frame mean decode.cpp:263-273, 465-484).
 *
 * TEST INFRASTRUCTURE ONLY: a second, independent CPU restatement that the
 * numpy oracle is checked against (tests/test_oracle_c.py), the fast checker
 * of the chunk-level parity tests, and the CPU baseline that bench.py times.
 * Nothing in the product links or loads it.
 *
 * Precision (df_set_mode): 0 = float32 throughout; 1 = bf16-emulating, as the
 * numpy oracle's "bf16" mode: values held in float32, every op output the
 * reference materialises in the model dtype rounded to bf16 (nearest, ties
 * to even) -- Linear outputs, the normalised value and its weight product in
 * RMSNorm, the attention output, residual sums, each step of the tanh GELU
 * with bf16 constants, the embedding + position sum, the frame sum and mean;
 * dot products, norms' sums of squares and softmax accumulate in float32.
 * The caller passes weights already rounded to the model dtype.
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
#include <stdint.h>
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

/* The encoder (modules.cpp:349-358) and the embedding tables. */
typedef struct {
  int L, D, HD, H, F, V, max_len;
  const float *norm_attn, *wq, *wk, *wv, *wo, *norm_ff, *wi0, *wi1, *wo2; /* stacked as above */
  const float* enc_norm;      /* (D) */
  const float* emb;           /* (V, D) token_embedding */
  const float* pe;            /* (max_len, D) fp32 sinusoid table (model.cpp:54-80) */
} df_encoder;

static int g_mode = 0; /* 0: fp32, 1: bf16-emulating */

void df_set_mode(int mode) { g_mode = mode; }

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

/* The value materialised in the model dtype: bf16 round-to-nearest-even of
 * the float32 bits (NaN kept), or the float32 value itself. */
static inline float R(float x) {
  if (!g_mode) return x;
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return x;
  u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  memcpy(&x, &u, 4);
  return x;
}

/* x[i] <- bf16(x[i]) in place, whatever the mode (the weights' cast to the
 * model dtype, modules.cpp:47-54) */
void df_round_bf16(float* x, size_t n) {
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; ++i) {
    uint32_t u;
    memcpy(&u, &x[i], 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) continue;
    u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
    memcpy(&x[i], &u, 4);
  }
}

/* R(R(x * rsqrt(mean(x^2) + 1e-6)) * w) (modules.cpp:72-84) */
static void rms_norm(const float* x, const float* w, int D, float* y) {
  float ss = 0.f;
  for (int i = 0; i < D; ++i) ss += x[i] * x[i];
  const float inv = 1.0f / sqrtf(ss / (float)D + 1e-6f);
  for (int i = 0; i < D; ++i) y[i] = R(R(x[i] * inv) * w[i]);
}

/* y_r = R(W x_r) for both CFG rows, W (N, K); one pass over W */
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
    y0[n] = R(a0);
    y1[n] = R(a1);
  }
}

/* Y (M, N) = R(X (M, K) W (N, K)^T): blocks of 32 rows of X against tiles
 * of 4 rows of W, 4 x 4 dot products at a time. */
static void gemm(const float* X, int M, const float* W, int N, int K, float* Y) {
  const int MB = 32;
  const int nmb = (M + MB - 1) / MB, nnt = (N + 3) / 4;
#pragma omp parallel for schedule(dynamic, 1) collapse(2)
  for (int mb = 0; mb < nmb; ++mb) {
    for (int nt = 0; nt < nnt; ++nt) {
      const int m1 = mb * MB + MB < M ? mb * MB + MB : M;
      const int n0 = nt * 4;
      const float* w[4];
      for (int j = 0; j < 4; ++j) w[j] = W + (size_t)(n0 + j < N ? n0 + j : N - 1) * K;
      for (int m0 = mb * MB; m0 < m1; m0 += 4) {
        const float* x[4];
        for (int i = 0; i < 4; ++i) x[i] = X + (size_t)(m0 + i < M ? m0 + i : M - 1) * K;
        float a00 = 0, a01 = 0, a02 = 0, a03 = 0, a10 = 0, a11 = 0, a12 = 0, a13 = 0;
        float a20 = 0, a21 = 0, a22 = 0, a23 = 0, a30 = 0, a31 = 0, a32 = 0, a33 = 0;
#pragma omp simd reduction(+ : a00, a01, a02, a03, a10, a11, a12, a13, a20, a21, a22, a23, a30, a31, a32, a33)
        for (int k = 0; k < K; ++k) {
          const float w0 = w[0][k], w1 = w[1][k], w2 = w[2][k], w3 = w[3][k];
          const float x0 = x[0][k], x1 = x[1][k], x2 = x[2][k], x3 = x[3][k];
          a00 += x0 * w0; a01 += x0 * w1; a02 += x0 * w2; a03 += x0 * w3;
          a10 += x1 * w0; a11 += x1 * w1; a12 += x1 * w2; a13 += x1 * w3;
          a20 += x2 * w0; a21 += x2 * w1; a22 += x2 * w2; a23 += x2 * w3;
          a30 += x3 * w0; a31 += x3 * w1; a32 += x3 * w2; a33 += x3 * w3;
        }
        const float a[4][4] = {{a00, a01, a02, a03}, {a10, a11, a12, a13}, {a20, a21, a22, a23},
                               {a30, a31, a32, a33}};
        for (int i = 0; i < 4 && m0 + i < M; ++i)
          for (int j = 0; j < 4 && n0 + j < N; ++j) Y[(size_t)(m0 + i) * N + n0 + j] = R(a[i][j]);
      }
    }
  }
}

/* tanh GELU with per-op rounding and model-dtype constants (nn_ops.h:66-98) */
static float gelu_t(float x) {
  const float half = R(0.5f), one = R(1.0f), c0 = R(0.7978845608028654f), c1 = R(0.044715f);
  float t = R(x * x);
  t = R(c1 * t);
  t = R(one + t);
  t = R(x * t);
  t = R(c0 * t);
  t = R(tanhf(t));
  t = R(one + t);
  t = R(x * t);
  return R(half * t);
}

/* R(softmax(q . k_j + bias_j) . v) over n keys of one head; k/v rows of 64
 * (scale 1.0, modules.cpp:289-290); s is scratch of n floats */
static void attend(const float* q, const float* K, const float* V, int n, const float* bias, float* out, float* s) {
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
  for (int d = 0; d < 64; ++d) out[d] = R(o[d] / z);
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
  const int NS = (S > pos + 1 ? S : pos + 1);
  float* xn = (float*)malloc(sizeof(float) * 2 * (size_t)M);
  float* q = (float*)malloc(sizeof(float) * 2 * (size_t)HD);
  float* k = (float*)malloc(sizeof(float) * 2 * (size_t)HD);
  float* v = (float*)malloc(sizeof(float) * 2 * (size_t)HD);
  float* at = (float*)malloc(sizeof(float) * 2 * (size_t)HD);
  float* y = (float*)malloc(sizeof(float) * 2 * (size_t)M);
  float* g = (float*)malloc(sizeof(float) * 2 * (size_t)F);
  float* u = (float*)malloc(sizeof(float) * 2 * (size_t)F);
  float* bias = (float*)malloc(sizeof(float) * 2 * (size_t)H * (size_t)(pos + 1));
  float* sc = (float*)malloc(sizeof(float) * 2 * (size_t)H * (size_t)NS);
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
      attend(q + r * HD + h * 64, kc + base, vc + base, pos + 1, bh, at + r * HD + h * 64, sc + (size_t)rh * NS);
    }
    gemv2(st->wo + oq, at, at + HD, D, HD, y, y + M);
    for (int r = 0; r < 2; ++r)
      for (int i = 0; i < D; ++i) x[r * D + i] = R(x[r * D + i] + y[r * M + i]);
    /* cross attention over the encoder K/V */
    if (st->cross) {
      for (int r = 0; r < 2; ++r) rms_norm(x + r * D, st->norm_ca + dd, D, xn + r * M);
      gemv2(st->cq + qd, xn, xn + M, HD, D, q, q + HD);
#pragma omp parallel for schedule(static)
      for (int rh = 0; rh < 2 * H; ++rh) {
        const int r = rh / H, h = rh % H;
        const size_t base = ((((size_t)li * 2 + r) * H + h) * (size_t)S) * 64;
        attend(q + r * HD + h * 64, ck + base, cv + base, S, NULL, at + r * HD + h * 64, sc + (size_t)rh * NS);
      }
      gemv2(st->co + oq, at, at + HD, D, HD, y, y + M);
      for (int r = 0; r < 2; ++r)
        for (int i = 0; i < D; ++i) x[r * D + i] = R(x[r * D + i] + y[r * M + i]);
    }
    /* gated GELU feed-forward (modules.cpp:222-226) */
    for (int r = 0; r < 2; ++r) rms_norm(x + r * D, st->norm_ff + dd, D, xn + r * M);
    gemv2(st->wi0 + fd, xn, xn + M, F, D, g, g + F);
    gemv2(st->wi1 + fd, xn, xn + M, F, D, u, u + F);
    for (int i = 0; i < 2 * F; ++i) g[i] = R(gelu_t(g[i]) * u[i]);
    gemv2(st->wo2 + df, g, g + F, D, F, y, y + M);
    for (int r = 0; r < 2; ++r)
      for (int i = 0; i < D; ++i) x[r * D + i] = R(x[r * D + i] + y[r * M + i]);
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
  free(sc);
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

/* Depthformer::encode (model.cpp:226-241): tokens (rows, S) -> out (rows, S, D):
 * R(emb + R(pe)), then per layer x = R(x + O(attn(norm(x)))), x = R(x +
 * FFN(norm(x))) with bidirectional attention and no bias (modules.cpp:349-358),
 * then encoder_norm. */
void df_encode(const df_encoder* e, const int* tokens, int rows, int S, float* out) {
  const int D = e->D, HD = e->HD, H = e->H, F = e->F;
  const size_t M = (size_t)rows * S;
  float* x = out;
  float* xn = (float*)malloc(sizeof(float) * M * (size_t)D);
  float* q = (float*)malloc(sizeof(float) * M * (size_t)HD);
  float* k = (float*)malloc(sizeof(float) * M * (size_t)HD);
  float* v = (float*)malloc(sizeof(float) * M * (size_t)HD);
  float* at = (float*)malloc(sizeof(float) * M * (size_t)HD);
  float* y = (float*)malloc(sizeof(float) * M * (size_t)D);
  float* g = (float*)malloc(sizeof(float) * M * (size_t)F);
  float* u = (float*)malloc(sizeof(float) * M * (size_t)F);
  for (size_t m = 0; m < M; ++m) {
    const float* er = e->emb + (size_t)tokens[m] * D;
    const float* pr = e->pe + (size_t)(m % S) * D;
    for (int i = 0; i < D; ++i) x[m * D + i] = R(er[i] + R(pr[i]));
  }
  for (int li = 0; li < e->L; ++li) {
    const size_t dd = (size_t)li * D, qd = (size_t)li * HD * D, oq = (size_t)li * D * HD;
    const size_t fd = (size_t)li * F * D, df = (size_t)li * D * F;
#pragma omp parallel for schedule(static)
    for (size_t m = 0; m < M; ++m) rms_norm(x + m * D, e->norm_attn + dd, D, xn + m * D);
    gemm(xn, (int)M, e->wq + qd, HD, D, q);
    gemm(xn, (int)M, e->wk + qd, HD, D, k);
    gemm(xn, (int)M, e->wv + qd, HD, D, v);
    /* heads: (rows, S, H, 64) -> per (row, head) keys of stride HD; gather
     * each head's K/V rows contiguous first */
#pragma omp parallel
    {
      float* kh = (float*)malloc(sizeof(float) * (size_t)S * 64);
      float* vh = (float*)malloc(sizeof(float) * (size_t)S * 64);
      float* s = (float*)malloc(sizeof(float) * (size_t)S);
#pragma omp for schedule(dynamic, 1)
      for (int rh = 0; rh < rows * H; ++rh) {
        const int r = rh / H, h = rh % H;
        for (int j = 0; j < S; ++j) {
          memcpy(kh + (size_t)j * 64, k + ((size_t)r * S + j) * HD + h * 64, 64 * sizeof(float));
          memcpy(vh + (size_t)j * 64, v + ((size_t)r * S + j) * HD + h * 64, 64 * sizeof(float));
        }
        for (int i = 0; i < S; ++i)
          attend(q + ((size_t)r * S + i) * HD + h * 64, kh, vh, S, NULL, at + ((size_t)r * S + i) * HD + h * 64, s);
      }
      free(kh);
      free(vh);
      free(s);
    }
    gemm(at, (int)M, e->wo + oq, D, HD, y);
    for (size_t i = 0; i < M * D; ++i) x[i] = R(x[i] + y[i]);
#pragma omp parallel for schedule(static)
    for (size_t m = 0; m < M; ++m) rms_norm(x + m * D, e->norm_ff + dd, D, xn + m * D);
    gemm(xn, (int)M, e->wi0 + fd, F, D, g);
    gemm(xn, (int)M, e->wi1 + fd, F, D, u);
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < M * F; ++i) g[i] = R(gelu_t(g[i]) * u[i]);
    gemm(g, (int)M, e->wo2 + df, D, F, y);
    for (size_t i = 0; i < M * D; ++i) x[i] = R(x[i] + y[i]);
  }
#pragma omp parallel for schedule(static)
  for (size_t m = 0; m < M; ++m) {
    float* t = y + m * D;
    rms_norm(x + m * D, e->enc_norm, D, t);
    memcpy(x + m * D, t, sizeof(float) * D);
  }
  free(xn);
  free(q);
  free(k);
  free(v);
  free(at);
  free(y);
  free(g);
  free(u);
}

/* precompute_cross_kv (modules.cpp:448-455): enc (2, S, D) -> ck, cv
 * (L, 2, H, S, 64) with wk / wv the stacked (L, HD, D) cross projections */
void df_cross_kv(const float* enc, int S, int L, int D, int HD, const float* wk, const float* wv, float* ck,
                 float* cv) {
  const int H = HD / 64;
  float* t = (float*)malloc(sizeof(float) * 2 * (size_t)S * HD);
  for (int li = 0; li < L; ++li)
    for (int kind = 0; kind < 2; ++kind) {
      gemm(enc, 2 * S, (kind ? wv : wk) + (size_t)li * HD * D, HD, D, t);
      float* dst = (kind ? cv : ck) + (size_t)li * 2 * H * S * 64;
      for (int r = 0; r < 2; ++r)
        for (int h = 0; h < H; ++h)
          for (int j = 0; j < S; ++j)
            memcpy(dst + (((size_t)r * H + h) * S + j) * 64, t + ((size_t)r * S + j) * HD + h * 64,
                   64 * sizeof(float));
    }
  free(t);
}

/* ---- the draw (decode.cpp:71-148) ------------------------------------------- */

/* Philox-4x32-10 (Salmon et al., SC'11): counter c, key k -> first output word */
static uint32_t philox_x0(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0, uint32_t k1) {
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint64_t p0 = (uint64_t)c0 * 0xD2511F53u, p1 = (uint64_t)c2 * 0xCD9E8D57u;
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
  }
  return c0;
}

/* Gumbel noise of candidate i of draw (frame, level): counter (i, level,
 * frame, 0x4D525444), u = ((x >> 9) + 0.5) 2^-23, g = -log(-log(u)) */
static float gumbel(uint64_t seed, int frame, int level, int i) {
  const uint32_t x = philox_x0((uint32_t)i, (uint32_t)level, (uint32_t)frame, 0x4D525444u, (uint32_t)seed,
                               (uint32_t)(seed >> 32));
  const float u = ((float)(x >> 9) + 0.5f) * (1.0f / 8388608.0f);
  return -logf(-logf(u));
}

static int cmp_desc(const void* a, const void* b) {
  const float x = *(const float*)a, y = *(const float*)b;
  return (x < y) - (x > y);
}

/* CFG (1+w) l0 - w l1 with each product rounded (decode.cpp:71-85), then
 * argmax at temperature 0, else top_k_logits (ties at the k-th largest kept,
 * decode.cpp:104-122) and the Gumbel-max draw (decode.cpp:124-148). */
static int draw(const float* l0, const float* l1, int C, float w, float T, int top_k, uint64_t seed, int frame,
                int level, float* s, float* tmp) {
  for (int c = 0; c < C; ++c) {
    const float a = (1.0f + w) * l0[c];
    const float b = w * l1[c];
    s[c] = a - b;
  }
  int best = 0;
  if (T == 0.0f) {
    for (int c = 1; c < C; ++c)
      if (s[c] > s[best]) best = c;
    return best;
  }
  for (int c = 0; c < C; ++c) s[c] = s[c] / T;
  float thr = -INFINITY;
  if (top_k > 0 && top_k < C) {
    memcpy(tmp, s, sizeof(float) * C);
    qsort(tmp, C, sizeof(float), cmp_desc);
    thr = tmp[top_k - 1];
  }
  float bv = -INFINITY;
  best = -1;
  for (int c = 0; c < C; ++c) {
    if (s[c] < thr) continue;
    const float vv = s[c] + gumbel(seed, frame, level, c);
    if (best < 0 || vv > bv) {
      bv = vv;
      best = c;
    }
  }
  return best;
}

/* generate_tokens (decode.cpp:239-573), non-speculative, one CFG pair:
 * frame 0 feeds emb(PAD = 0); per frame the temporal step, then L depth
 * steps on the level's lm_head slice [off + C l, + C), each followed by the
 * draw and the feedback of emb(token) (teacher[f * L + l] when teacher is
 * non-null); the frame mean R(R(sum) / R(L)) is the next temporal input.
 * tk/tv: temporal caches with Lmax_t >= frames slots; dk/dv depth caches with
 * L slots; ck/cv the cross K/V (S keys).  Optional records: slices (F, L, 2, C),
 * t_out (F, 2, D), fmean (F, 2, D), drawn (F, L). */
void df_generate(const df_stack* ts, const df_stack* ds, const float* emb, const float* dec_norm,
                 const float* lm_head, int frames, int L, int C, int off, float w, float T, int top_k,
                 uint64_t seed, const int* teacher, float* tk, float* tv, int Lmax_t, float* dk, float* dv,
                 const float* ck, const float* cv, int S, int* tokens, float* slices, float* t_out, float* fmean,
                 int* drawn) {
  const int D = ts->D;
  float* tin = (float*)malloc(sizeof(float) * 2 * (size_t)D);
  float* tout = (float*)malloc(sizeof(float) * 2 * (size_t)D);
  float* din = (float*)malloc(sizeof(float) * 2 * (size_t)D);
  float* fs = (float*)malloc(sizeof(float) * (size_t)D);
  float* lg = (float*)malloc(sizeof(float) * 2 * (size_t)C);
  float* s = (float*)malloc(sizeof(float) * (size_t)C);
  float* tmp = (float*)malloc(sizeof(float) * (size_t)C);
  const float div = R((float)L);
  for (int r = 0; r < 2; ++r) memcpy(tin + r * D, emb, sizeof(float) * D);
  for (int f = 0; f < frames; ++f) {
    df_temporal_step(ts, tin, f, tk, tv, Lmax_t, ck, cv, S, tout);
    if (t_out) memcpy(t_out + (size_t)f * 2 * D, tout, sizeof(float) * 2 * D);
    memcpy(din, tout, sizeof(float) * 2 * D);
    for (int l = 0; l < L; ++l) {
      df_depth_step(ds, din, l, dk, dv, L, dec_norm, lm_head + (size_t)(off + C * l) * D, C, lg);
      if (slices) memcpy(slices + ((size_t)f * L + l) * 2 * C, lg, sizeof(float) * 2 * C);
      const int d = off + C * l + draw(lg, lg + C, C, w, T, top_k, seed, f, l, s, tmp);
      const int tok = teacher ? teacher[f * L + l] : d;
      tokens[f * L + l] = tok;
      if (drawn) drawn[f * L + l] = d;
      const float* e = emb + (size_t)tok * D;
      for (int r = 0; r < 2; ++r) memcpy(din + r * D, e, sizeof(float) * D);
      for (int i = 0; i < D; ++i) fs[i] = l == 0 ? e[i] : R(fs[i] + e[i]);
    }
    for (int i = 0; i < D; ++i) tin[i] = tin[D + i] = R(fs[i] / div);
    if (fmean) memcpy(fmean + (size_t)f * 2 * D, tin, sizeof(float) * 2 * D);
  }
  free(tin);
  free(tout);
  free(din);
  free(fs);
  free(lg);
  free(s);
  free(tmp);
}
