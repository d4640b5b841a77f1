/*
 * sanitize_main.c -- runs every oracle function on small, ragged shapes with
 * exactly sized heap buffers, for the AddressSanitizer / UndefinedBehavior-
 * Sanitizer build of the oracle (make -C oracle sanitize).  TEST
 * INFRASTRUCTURE ONLY, like the oracle itself.
 *
 * Each buffer is malloc'ed at the size the function's contract gives, so an
 * access one element past it is reported; a few cross-checks between
 * restatements keep the run meaningful.  Prints "ok" and exits 0 when every
 * check holds.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint32_t rnd(void) {
  rng_state ^= rng_state << 13;
  rng_state ^= rng_state >> 7;
  rng_state ^= rng_state << 17;
  return (uint32_t)(rng_state >> 16);
}
static float rndf(void) { return ((float)(rnd() % 20001) - 10000.f) / 10000.f; }

static void *xmalloc(size_t n) {
  void *p = malloc(n ? n : 1);
  if (!p) {
    fprintf(stderr, "out of memory\n");
    exit(2);
  }
  return p;
}
static float *fbuf(int64_t n) {
  float *p = xmalloc(sizeof(float) * (size_t)n);
  for (int64_t i = 0; i < n; i++) p[i] = rndf();
  return p;
}
static uint8_t *bbuf(int64_t n) {
  uint8_t *p = xmalloc((size_t)n);
  for (int64_t i = 0; i < n; i++) p[i] = (uint8_t)rnd();
  return p;
}

static int failures = 0;
static void check(int cond, const char *what) {
  if (!cond) {
    fprintf(stderr, "FAILED: %s\n", what);
    failures++;
  }
}

static void int8_paths(void) {
  /* vpdpbusd lane op */
  uint8_t *a = bbuf(64);
  int8_t *b = (int8_t *)bbuf(64);
  int32_t *acc = xmalloc(64), *out = xmalloc(64);
  for (int i = 0; i < 16; i++) acc[i] = (int32_t)rnd();
  orc_vpdpbusd16(a, b, acc, out);
  free(a), free(b), free(acc), free(out);

  /* GEMMs with M % 4, K % 64 and N tails, both signednesses, both layouts */
  const int64_t shapes[][3] = {{1, 1, 1}, {5, 7, 67}, {9, 33, 130}, {4, 16, 64}, {3, 2, 200}};
  for (size_t s = 0; s < sizeof shapes / sizeof shapes[0]; s++) {
    const int64_t M = shapes[s][0], N = shapes[s][1], K = shapes[s][2];
    uint8_t *A = bbuf(M * K);
    int8_t *B = (int8_t *)bbuf(K * N), *BT = xmalloc((size_t)(N * K));
    for (int64_t k = 0; k < K; k++)
      for (int64_t n = 0; n < N; n++) BT[n * K + k] = B[k * N + n];
    int32_t *C0 = xmalloc(sizeof(int32_t) * (size_t)(M * N));
    int32_t *C1 = xmalloc(sizeof(int32_t) * (size_t)(M * N));
    for (int au = 0; au < 2; au++) {
      orc_matmul_i8(A, K, B, N, C0, N, M, N, K, au, 0);
      orc_matmul_i8_vnni(A, B, C1, M, N, K, au, 0, 1);
      check(memcmp(C0, C1, sizeof(int32_t) * (size_t)(M * N)) == 0, "vnni == textbook (B[K,N])");
      orc_matmul_i8(A, K, BT, K, C1, N, M, N, K, au, 1);
      check(memcmp(C0, C1, sizeof(int32_t) * (size_t)(M * N)) == 0, "textbook B_T == B");
      orc_matmul_i8_vnni(A, BT, C1, M, N, K, au, 1, 2);
      check(memcmp(C0, C1, sizeof(int32_t) * (size_t)(M * N)) == 0, "vnni B_T, 2 threads");
    }
    (void)orc_checksum_i32(C0, M * N);
    free(A), free(B), free(BT), free(C0), free(C1);
  }
  const int64_t n8 = 48;
  int8_t *RA = xmalloc((size_t)(n8 * n8)), *RB = xmalloc((size_t)(n8 * n8));
  orc_int8_recipe_inputs(n8, RA, RB);
  free(RA), free(RB);
}

static void int4_paths(void) {
  const int64_t dims[][3] = {{3, 5, 7}, {4, 8, 16}, {1, 1, 1}};
  for (size_t s = 0; s < sizeof dims / sizeof dims[0]; s++) {
    const int64_t M = dims[s][0], N = dims[s][1], K = dims[s][2];
    const int64_t la = (K + 1) / 2, lb = (N + 1) / 2;
    uint8_t *Ap = bbuf(M * la), *Bp = bbuf(K * lb);
    int16_t *C = xmalloc(sizeof(int16_t) * (size_t)(M * N));
    orc_matmul_i4(Ap, la, Bp, lb, C, N, M, N, K);
    (void)orc_checksum_i16(C, M * N);
    free(Ap), free(Bp), free(C);
  }
  const int64_t n = 9;
  uint8_t *Ap = xmalloc((size_t)(n * ((n + 1) / 2))), *Bp = xmalloc((size_t)(n * ((n + 1) / 2)));
  orc_int4_recipe_inputs(n, Ap, Bp);
  free(Ap), free(Bp);
}

static void fp32_paths(void) {
  const int64_t Bt = 2, M = 3, K = 5, N = 4;
  float *A = fbuf(Bt * M * K), *B = fbuf(Bt * K * N), *C = xmalloc(sizeof(float) * (size_t)(Bt * M * N));
  orc_batch_matmul_f32(A, B, C, Bt, M, K, N);
  double *Ad = xmalloc(sizeof(double) * (size_t)(Bt * M * K)), *Bd = xmalloc(sizeof(double) * (size_t)(Bt * K * N));
  double *Cd = xmalloc(sizeof(double) * (size_t)(Bt * M * N));
  for (int64_t i = 0; i < Bt * M * K; i++) Ad[i] = A[i];
  for (int64_t i = 0; i < Bt * K * N; i++) Bd[i] = B[i];
  orc_batch_matmul_f64(Ad, Bd, Cd, Bt, M, K, N);
  for (int64_t i = 0; i < Bt * M * N; i++) check(fabs(Cd[i] - C[i]) <= 1e-5, "batch f32 vs f64");
  free(Ad), free(Bd), free(Cd);
  /* builtin matmul at offsets: C[out_off ..] += A[lhs_off ..] * B[rhs_off ..] */
  float *acc = fbuf(7 + M * N);
  orc_matmul_f32_acc(A, B, acc, M, K, N, 2, 1, 7);
  free(acc);
  free(A), free(B), free(C);

  const int64_t n = 37;
  float *in = fbuf(n + 3), *w = fbuf(n + 2), *out = xmalloc(sizeof(float) * (size_t)(n + 4));
  orc_rmsnorm(in, w, out, n, 1e-5f, 2);
  orc_softmax(in, out, n, 3, 4);
  float s = 0.f;
  for (int64_t i = 0; i < n; i++) s += out[4 + i];
  check(fabsf(s - 1.f) < 1e-5f, "softmax sums to 1");
  orc_silu(in, out, n);
  free(in), free(w), free(out);
}

static void w4_paths(void) {
  /* reference format: three layers of rows x cols, gs 32 and 128 */
  const int64_t rows = 6, cols = 128, layers = 3;
  for (int64_t gs = 32; gs <= 128; gs *= 4) {
    const int64_t total = layers * rows * cols;
    float *w = fbuf(total);
    uint8_t *q = xmalloc((size_t)((total + 1) / 2));
    float *sc = xmalloc(sizeof(float) * (size_t)((total + gs - 1) / gs));
    float *ze = xmalloc(sizeof(float) * (size_t)((total + gs - 1) / gs));
    orc_quantize_f5(w, total, gs, q, sc, ze);
    float *x = fbuf(cols), *o1 = xmalloc(sizeof(float) * rows), *o2 = xmalloc(sizeof(float) * rows);
    for (int64_t l = 0; l < layers; l++) {
      orc_matmul_quant_f5(q, sc, ze, x, o1, rows, cols, gs, l * rows * cols);
      if (gs == 128) orc_matmul_quant_f5_refidx(q, sc, ze, x, o2, rows, cols, gs, l * rows * cols);
    }
    /* the whole array, exactly sized, from an odd start to the last element */
    float *d = xmalloc(sizeof(float) * (size_t)total);
    orc_dequant_w4(q, sc, ze, 1, total - 1, gs, d);
    free(d);
    free(w), free(q), free(sc), free(ze), free(x), free(o1), free(o2);
  }
  /* symmetric format: M x vectors, N rows, K = 3 groups of 32 */
  const int64_t M = 2, N = 5, K = 96, gs = 32;
  float *w = fbuf(N * K);
  uint8_t *q = xmalloc((size_t)(N * K / 2));
  float *sc = xmalloc(sizeof(float) * (size_t)(N * K / gs));
  orc_quantize_w4s(w, N, K, gs, q, sc);
  float *x = fbuf(M * K), *o1 = xmalloc(sizeof(float) * (size_t)(M * N));
  float *o2 = xmalloc(sizeof(float) * (size_t)(M * N)), *o3 = xmalloc(sizeof(float) * (size_t)(M * N));
  orc_matmul_w4s(q, sc, x, o1, M, N, K, gs);
  orc_matmul_w4s_f32(q, sc, x, o2, M, N, K, gs, 2);
  orc_matmul_w4s_lowering(q, sc, x, o3, M, N, K, gs, 1);
  for (int64_t i = 0; i < M * N; i++)
    check(fabsf(o1[i] - o2[i]) <= 1e-4f * (1.f + fabsf(o1[i])) &&
              fabsf(o1[i] - o3[i]) <= 1e-4f * (1.f + fabsf(o1[i])),
          "w4s restatements agree");
  free(w), free(q), free(sc), free(x), free(o1), free(o2), free(o3);
}

static void decode_paths(void) {
  /* GQA model, fp32 and W4 weights, a few positions with RoPE */
  orc_llama_cfg c = {.dim = 64, .hidden = 96, .n_layers = 2, .n_heads = 4, .n_kv_heads = 2,
                     .vocab = 50, .seq_len = 6, .eps = 1e-5f, .theta = 10000.f, .w4 = 0, .gs = 32};
  const int64_t D = c.dim, H = c.hidden, L = c.n_layers, V = c.vocab, S = c.seq_len;
  const int64_t kv = D * c.n_kv_heads / c.n_heads;
  float *emb = fbuf(V * D), *ra = fbuf(L * D), *rf = fbuf(L * D), *rfin = fbuf(D);
  float *wq = fbuf(L * D * D), *wk = fbuf(L * kv * D), *wv = fbuf(L * kv * D), *wo = fbuf(L * D * D);
  float *w1 = fbuf(L * H * D), *w2 = fbuf(L * D * H), *w3 = fbuf(L * H * D), *wcls = fbuf(V * D);
  orc_llama_weights w = {.emb = emb, .rms_att = ra, .rms_ffn = rf, .rms_final = rfin, .wq = wq,
                         .wk = wk, .wv = wv, .wo = wo, .w1 = w1, .w2 = w2, .w3 = w3, .wcls = wcls};
  float *kc = xmalloc(sizeof(float) * (size_t)(L * S * kv)), *vc = xmalloc(sizeof(float) * (size_t)(L * S * kv));
  float *logits = xmalloc(sizeof(float) * (size_t)V);
  for (int64_t pos = 0; pos < S; pos++) orc_llama_forward(&c, &w, kc, vc, (pos * 7) % V, pos, logits);
  check(orc_argmax(logits, V) >= 0, "argmax in range");

  /* the same model with F6 W4 matrices */
  c.w4 = 1;
  struct { const float *src; int64_t rows, cols; const uint8_t **q; const float **s; } mats[] = {
      {wq, L * D, D, &w.q_wq, &w.s_wq}, {wk, L * kv, D, &w.q_wk, &w.s_wk},
      {wv, L * kv, D, &w.q_wv, &w.s_wv}, {wo, L * D, D, &w.q_wo, &w.s_wo},
      {w1, L * H, D, &w.q_w1, &w.s_w1}, {w2, L * D, H, &w.q_w2, &w.s_w2},
      {w3, L * H, D, &w.q_w3, &w.s_w3}, {wcls, V, D, &w.q_wcls, &w.s_wcls}};
  for (size_t i = 0; i < sizeof mats / sizeof mats[0]; i++) {
    uint8_t *q = xmalloc((size_t)(mats[i].rows * mats[i].cols / 2));
    float *s = xmalloc(sizeof(float) * (size_t)(mats[i].rows * mats[i].cols / c.gs));
    orc_quantize_w4s(mats[i].src, mats[i].rows, mats[i].cols, c.gs, q, s);
    *mats[i].q = q;
    *mats[i].s = s;
  }
  for (int64_t pos = 0; pos < S; pos++) orc_llama_forward(&c, &w, kc, vc, (pos * 5) % V, pos, logits);
  for (size_t i = 0; i < sizeof mats / sizeof mats[0]; i++) {
    free((void *)*mats[i].q);
    free((void *)*mats[i].s);
  }

  /* llama2_quant_forward: the seven matrices in one flat reference-format array */
  orc_llama_cfg cq = c;
  cq.w4 = 0;
  cq.theta = 0.f;
  const int64_t per[7] = {D * D, D * kv, D * kv, D * D, H * D, D * H, H * D};
  const float *src[7] = {wq, wk, wv, wo, w1, w2, w3};
  int64_t off[7], total = 0;
  for (int i = 0; i < 7; i++) {
    off[i] = total;
    total += L * per[i];
  }
  const int64_t gs = 32;
  uint8_t *qw = xmalloc((size_t)(total / 2));
  float *sc = xmalloc(sizeof(float) * (size_t)(total / gs)), *ze = xmalloc(sizeof(float) * (size_t)(total / gs));
  for (int i = 0; i < 7; i++)
    orc_quantize_f5(src[i], L * per[i], gs, qw + off[i] / 2, sc + off[i] / gs, ze + off[i] / gs);
  for (int64_t pos = 0; pos < S; pos++)
    orc_llama_quant_forward(&cq, emb, ra, rf, rfin, wcls, qw, sc, ze, gs, off, kc, vc, (pos * 3) % V, pos, logits);
  free(qw), free(sc), free(ze);

  /* RoPE on q / k of one position */
  float *q = fbuf(D), *k = fbuf(kv);
  orc_rope(q, k, D, kv, D / c.n_heads, 3, 10000.f);
  free(q), free(k);

  /* llama32_forward program: int8 weights [out, in] (NT), int8 caches */
  const int64_t hd = D / c.n_heads, kv32 = c.n_kv_heads * hd;
  int8_t *x8 = (int8_t *)bbuf(D), *q8 = (int8_t *)bbuf(L * D * D), *k8 = (int8_t *)bbuf(L * kv32 * D);
  int8_t *v8 = (int8_t *)bbuf(L * kv32 * D), *o8 = (int8_t *)bbuf(L * D * D), *a8 = (int8_t *)bbuf(L * H * D);
  int8_t *b8 = (int8_t *)bbuf(L * D * H), *c8 = (int8_t *)bbuf(L * H * D);
  float *x = xmalloc(sizeof(float) * (size_t)D), *xb = xmalloc(sizeof(float) * (size_t)D);
  int8_t *xbi = xmalloc((size_t)D), *kc8 = xmalloc((size_t)(L * S * kv32)), *vc8 = xmalloc((size_t)(L * S * kv32));
  float *sco = xmalloc(sizeof(float) * (size_t)(c.n_heads * S)), *pro = xmalloc(sizeof(float) * (size_t)(c.n_heads * S));
  int32_t *ao = xmalloc(sizeof(int32_t) * (size_t)D);
  int8_t *hb = xmalloc((size_t)H);
  memset(kc8, 0, (size_t)(L * S * kv32));
  memset(vc8, 0, (size_t)(L * S * kv32));
  for (int64_t pos = 0; pos < S; pos++)
    (void)orc_llama32_int8_forward(&c, hd, x8, ra, rf, rfin, q8, k8, v8, o8, a8, b8, c8, wcls, x, xb,
                                   logits, xbi, kc8, vc8, sco, pro, ao, hb, pos);
  free(x8), free(q8), free(k8), free(v8), free(o8), free(a8), free(b8), free(c8);
  free(x), free(xb), free(xbi), free(kc8), free(vc8), free(sco), free(pro), free(ao), free(hb);

  free(emb), free(ra), free(rf), free(rfin), free(wq), free(wk), free(wv), free(wo);
  free(w1), free(w2), free(w3), free(wcls), free(kc), free(vc), free(logits);
}

static void sampler_paths(void) {
  orc_mt19937 g;
  orc_mt_seed(&g, 42);
  for (int i = 0; i < 1000; i++) (void)orc_mt_next(&g);
  float u = orc_uniform01f(&g);
  check(u >= 0.f && u < 1.f, "uniform in [0, 1)");
  const int64_t n = 33;
  float *l = fbuf(n);
  for (int t = 0; t < 3; t++) {
    const int64_t s = orc_sample(l, n, (float)t * 0.5f, &g);
    check(s >= 0 && s < n, "sample in range");
  }
  free(l);
}

int main(void) {
  int8_paths();
  int4_paths();
  fp32_paths();
  w4_paths();
  decode_paths();
  sampler_paths();
  if (failures) {
    fprintf(stderr, "%d check(s) failed\n", failures);
    return 1;
  }
  printf("ok\n");
  return 0;
}
