/*
 * cpu_decode.c -- the CPU baseline of the decode step, for bench.py's
 * cpu_baseline leg only (TEST INFRASTRUCTURE: never on the product path;
 * tests/test_oracle_decode.py checks it against orc_llama_forward).
 *
 * One token of stories110M.sl:44-247 (fp32 weights) or of the BASELINE W4
 * model (every linear weight signed nibbles in [-8,7], one fp32 scale per group
 * of gs along K, the matmul_quant loop of ConvertSimpToMemRef.cpp:3906-4005 with
 * the signed nibbles of :3016-3037), in fp32 throughout as the compiled program
 * runs it, on all the cores OpenMP is given:
 *   - every matrix-vector product is OpenMP over output rows, each row summed
 *     in 16 fp32 lanes (the tile-16 vectorized loops of the reference's MLIR
 *     pipeline, mlir_pipeline.cpp:265-393) with fused multiply-adds;
 *   - the W4 product dequantizes per group (q * scale, one scale per group)
 *     before the multiply-add, as the lowering's tile loop does;
 *   - attention is OpenMP over heads; RoPE, RMSNorm, softmax and SiLU are the
 *     oracle's fp32 restatements (orc_rope, orc_rmsnorm, orc_softmax, orc_silu).
 * The hot loops are compiled for AVX-512F, AVX2 and a generic target, chosen at
 * load time (the reference builds its programs for the host CPU).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#ifdef _OPENMP
#include <omp.h>
#endif

#define CPU_CLONES __attribute__((target_clones("avx512f", "avx2", "default")))

/* y[r] = sum_k W[r, k] x[k] for r in [r0, r1) */
CPU_CLONES static void mv_f32_rows(const float *W, const float *x, float *y, int64_t r0,
                                   int64_t r1, int64_t K) {
  for (int64_t r = r0; r < r1; r++) {
    const float *w = W + r * K;
    float acc[16] = {0};
    int64_t k = 0;
    for (; k + 16 <= K; k += 16)
      for (int j = 0; j < 16; j++) acc[j] += w[k + j] * x[k + j];
    float s = 0.0f;
    for (int j = 0; j < 16; j++) s += acc[j];
    for (; k < K; k++) s += w[k] * x[k];
    y[r] = s;
  }
}

/* W4 rows: Q[r] holds K/2 bytes (low nibble = even k), S[r] K/gs scales.  xe and
 * xo are the even and odd elements of x, so that the low and high nibbles of
 * 16 consecutive bytes meet 16 contiguous x values each. */
CPU_CLONES static void mv_w4s_rows(const uint8_t *Q, const float *S, const float *xe,
                                   const float *xo, float *y, int64_t r0, int64_t r1, int64_t K,
                                   int64_t gs) {
  const int64_t ng = K / gs, hb = gs / 2;
  for (int64_t r = r0; r < r1; r++) {
    const uint8_t *row = Q + r * (K / 2);
    const float *sr = S + r * ng;
    float accl[16] = {0}, acch[16] = {0};
    for (int64_t g = 0; g < ng; g++) {
      const float s = sr[g];
      for (int64_t t = 0; t < hb; t += 16) {   /* 32 weights per step */
        const uint8_t *b = row + g * hb + t;
        const float *ve = xe + g * hb + t, *vo = xo + g * hb + t;
        for (int j = 0; j < 16; j++) {
          const float lo = (float)((int8_t)(uint8_t)(b[j] << 4) >> 4);
          const float hi = (float)((int8_t)b[j] >> 4);
          accl[j] += (lo * s) * ve[j];
          acch[j] += (hi * s) * vo[j];
        }
      }
    }
    float sum = 0.0f;
    for (int j = 0; j < 16; j++) sum += accl[j] + acch[j];
    y[r] = sum;
  }
}

static void mv(const orc_llama_cfg *c, const float *wf, const uint8_t *wq, const float *ws,
               const float *x, float *y, int64_t rows, int64_t K, float *xe, float *xo) {
  if (c->w4) {
    for (int64_t i = 0; i < K / 2; i++) {
      xe[i] = x[2 * i];
      xo[i] = x[2 * i + 1];
    }
#pragma omp parallel
    {
#ifdef _OPENMP
      const int64_t nt = omp_get_num_threads(), t = omp_get_thread_num();
#else
      const int64_t nt = 1, t = 0;
#endif
      const int64_t per = (rows + nt - 1) / nt;
      const int64_t r0 = t * per, r1 = r0 + per < rows ? r0 + per : rows;
      if (r0 < r1) mv_w4s_rows(wq, ws, xe, xo, y, r0, r1, K, c->gs);
    }
    return;
  }
#pragma omp parallel
  {
#ifdef _OPENMP
    const int64_t nt = omp_get_num_threads(), t = omp_get_thread_num();
#else
    const int64_t nt = 1, t = 0;
#endif
    const int64_t per = (rows + nt - 1) / nt;
    const int64_t r0 = t * per, r1 = r0 + per < rows ? r0 + per : rows;
    if (r0 < r1) mv_f32_rows(wf, x, y, r0, r1, K);
  }
}

int cpu_llama_supported(const orc_llama_cfg *c) {
  return !c->w4 || (c->gs > 0 && c->gs % 32 == 0 && c->dim % c->gs == 0 &&
                    c->hidden % c->gs == 0);
}

void cpu_llama_forward(const orc_llama_cfg *c, const orc_llama_weights *w, float *key_cache,
                       float *value_cache, int64_t token, int64_t pos, float *logits) {
  const int64_t dim = c->dim, hid = c->hidden, hs = dim / c->n_heads;
  const int64_t kv_dim = dim * c->n_kv_heads / c->n_heads;
  const int64_t kmax = hid > dim ? hid : dim;
  float *x = malloc(sizeof(float) * dim), *xb = malloc(sizeof(float) * dim);
  float *xb2 = malloc(sizeof(float) * dim), *q = malloc(sizeof(float) * dim);
  float *kk = malloc(sizeof(float) * kv_dim), *vv = malloc(sizeof(float) * kv_dim);
  float *hb = malloc(sizeof(float) * hid), *hb2 = malloc(sizeof(float) * hid);
  float *xe = malloc(sizeof(float) * kmax / 2 + 4), *xo = malloc(sizeof(float) * kmax / 2 + 4);
  float *att = malloc(sizeof(float) * c->n_heads * (pos + 1) * 2);
  memcpy(x, w->emb + token * dim, sizeof(float) * dim);
  const float scale = sqrtf((float)hs);
  for (int64_t l = 0; l < c->n_layers; l++) {
#define WF(p, r, cl) ((p) ? (p) + l * (r) * (cl) : NULL)
#define WQ(p, r, cl) ((p) ? (p) + l * (r) * (cl) / 2 : NULL)
#define WS(p, r, cl) ((p) ? (p) + l * (r) * (cl) / c->gs : NULL)
    orc_rmsnorm(x, w->rms_att, xb, dim, c->eps, l * dim);              /* stories110M.sl:60-61 */
    mv(c, WF(w->wq, dim, dim), WQ(w->q_wq, dim, dim), WS(w->s_wq, dim, dim), xb, q, dim, dim, xe, xo);
    mv(c, WF(w->wk, kv_dim, dim), WQ(w->q_wk, kv_dim, dim), WS(w->s_wk, kv_dim, dim), xb, kk,
       kv_dim, dim, xe, xo);
    mv(c, WF(w->wv, kv_dim, dim), WQ(w->q_wv, kv_dim, dim), WS(w->s_wv, kv_dim, dim), xb, vv,
       kv_dim, dim, xe, xo);
    orc_rope(q, kk, dim, kv_dim, hs, pos, c->theta);                   /* :86-112 */
    float *kc = key_cache + l * c->seq_len * kv_dim, *vc = value_cache + l * c->seq_len * kv_dim;
    memcpy(kc + pos * kv_dim, kk, sizeof(float) * kv_dim);            /* :115-121 */
    memcpy(vc + pos * kv_dim, vv, sizeof(float) * kv_dim);
#pragma omp parallel for schedule(static)
    for (int64_t h = 0; h < c->n_heads; h++) {                        /* :124-164 */
      const int64_t kvh = h * c->n_kv_heads / c->n_heads;
      const float *qh = q + h * hs;
      float *a = att + h * (pos + 1) * 2, *p = a + (pos + 1);
      for (int64_t t = 0; t <= pos; t++) {
        const float *kt = kc + t * kv_dim + kvh * hs;
        float s = 0.0f;
        for (int64_t i = 0; i < hs; i++) s += qh[i] * kt[i];
        a[t] = s / scale;
      }
      orc_softmax(a, p, pos + 1, 0, 0);
      float *o = xb + h * hs;
      for (int64_t i = 0; i < hs; i++) o[i] = 0.0f;
      for (int64_t t = 0; t <= pos; t++) {
        const float *vt = vc + t * kv_dim + kvh * hs;
        for (int64_t i = 0; i < hs; i++) o[i] += p[t] * vt[i];
      }
    }
    mv(c, WF(w->wo, dim, dim), WQ(w->q_wo, dim, dim), WS(w->s_wo, dim, dim), xb, xb2, dim, dim,
       xe, xo);
    for (int64_t i = 0; i < dim; i++) x[i] += xb2[i];                 /* :177-180 */
    orc_rmsnorm(x, w->rms_ffn, xb, dim, c->eps, l * dim);
    mv(c, WF(w->w1, hid, dim), WQ(w->q_w1, hid, dim), WS(w->s_w1, hid, dim), xb, hb, hid, dim,
       xe, xo);
    mv(c, WF(w->w3, hid, dim), WQ(w->q_w3, hid, dim), WS(w->s_w3, hid, dim), xb, hb2, hid, dim,
       xe, xo);
    orc_silu(hb, hb, hid);                                             /* :199-212 */
    for (int64_t i = 0; i < hid; i++) hb[i] *= hb2[i];
    mv(c, WF(w->w2, dim, hid), WQ(w->q_w2, dim, hid), WS(w->s_w2, dim, hid), hb, xb, dim, hid,
       xe, xo);
    for (int64_t i = 0; i < dim; i++) x[i] += xb[i];                  /* :225-228 */
#undef WF
#undef WQ
#undef WS
  }
  orc_rmsnorm(x, w->rms_final, xb, dim, c->eps, 0);                    /* :232-244 */
  mv(c, w->wcls, w->q_wcls, w->s_wcls, xb, logits, c->vocab, dim, xe, xo);
  free(x); free(xb); free(xb2); free(q); free(kk); free(vv);
  free(hb); free(hb2); free(xe); free(xo); free(att);
}
