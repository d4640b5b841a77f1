/*
 * oracle.c -- CPU restatement of SimpLang's tensor-op hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for libsimp_hip.so, loaded by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg.  Never on the
 * product path.  Citations are relative to the SimpLang source tree.
 *
 * Parity pins (see tests/test_oracle.py):
 *   orc_vpdpbusd16            -- nine KATs of test_vnni_correctness.cpp + the
 *                                reference scalar function compiled in place
 *   orc_matmul_i8             -- closed forms (identity/one-hot/constant) +
 *                                reference VNNI kernel compiled in place
 *   orc_matmul_i8_vnni        -- equals orc_matmul_i8 bit for bit (both paths)
 *   orc_int8_recipe_inputs    -- recipe restated; equals the numpy closed form
 *                                ((i*N+j)%127)-64 with A = B^T element by element;
 *                                checksum vs reference kernel
 *   orc_matmul_i4             -- reference packed_matmul_int4<N> checksums (32, 64,
 *                                128) on orc_int4_recipe_inputs; equals the int8
 *                                product of the unpacked nibbles truncated to i16
 *   orc_matmul_f32_acc        -- f64 brute force, KAT 110 (tests/test_tensor_matmul_runner.cpp:39)
 *   orc_batch_matmul_f32/f64  -- KATs of simptensor/tests/test_matmul_dot.sl:135-199
 *                                and tests/test_tensor_matmul.sl:66-117; equal
 *                                orc_matmul_f32_acc batch by batch
 *   orc_rmsnorm/softmax/silu  -- KATs of examples/llama2/kernels/test_*_host.cpp
 *   orc_matmul_quant_f5       -- closed-form KAT of test_quant_roofline.cpp:71-92
 *                                (0x55 bytes, scale .01) + f64 dequant brute force
 *   orc_dequant_w4            -- 0x55 / scale .01 / zero 0 gives 5 * .01f
 *                                (test_quant_roofline.cpp:71-92); equals
 *                                orc_matmul_quant_f5 with one-hot inputs element by
 *                                element (a swapped nibble or group index fails it)
 *   orc_matmul_w4s            -- F6 == F5 with u = q+8, zero = -8*scale; brute force
 *   orc_rope                  -- pos 0 identity, rotation preserves pair norms,
 *                                closed-form angle for pair 0
 *   orc_llama_forward,
 *   orc_llama_quant_forward   -- the reference holds no golden logits
 *                                (docs/benchmark/llama_results.md:81-95): float64
 *                                brute force in another formulation, closed forms
 *                                and invariances (tests/test_oracle_decode.py)
 *   orc_matmul_quant_f5_refidx -- equals orc_matmul_quant_f5 at offset 0, gs 128;
 *                                rotated scales at offset > 0; overlapping-tile
 *                                closed form at gs 32
 *   orc_llama32_int8_forward  -- closed forms: zero weights, layer-0 cache rows,
 *                                one layer's FFN and final norm in int64 / float64,
 *                                inert attention, x86 wrap of ffn_hb, layer
 *                                offsets (tests/test_oracle.py)
 *   orc_quantize_w4s          -- properties: |dequant - w| <= scale/2 inside the
 *                                range, the group maximum maps to +-7 exactly,
 *                                all-zero groups; brute force in numpy
 *   orc_mt_next               -- the C++ standard's check value: the 10000th draw
 *                                of std::mt19937 default-seeded (5489) is
 *                                4123659995 ([rand.predef])
 *   orc_argmax                -- closed forms of sample_argmax's scan: ties give
 *                                the first index, NaN at 0 gives 0, NaN elsewhere
 *                                is skipped, all NaN / all -inf give 0; brute force
 *                                over every pattern of 5 values from {-inf, -1, 0,
 *                                -0, 1, NaN}
 *   orc_uniform01f, orc_sample -- equal the library's std::mt19937 /
 *                                uniform_real_distribution<float> sampler
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#if defined(__x86_64__)
#include <immintrin.h>
#define ORC_HAVE_X86 1
#else
#define ORC_HAVE_X86 0
#endif

/* ---------------------------------------------------------------- int8 -- */

void orc_vpdpbusd16(const uint8_t *a, const int8_t *b, const int32_t *acc,
                    int32_t *out) {
  for (int i = 0; i < 16; i++) {
    uint32_t s = (uint32_t)acc[i];
    for (int j = 0; j < 4; j++)
      s += (uint32_t)((int32_t)a[4 * i + j] * (int32_t)b[4 * i + j]);
    out[i] = (int32_t)s;
  }
}

static inline int32_t a_elem(const void *A, int64_t idx, int a_unsigned) {
  return a_unsigned ? (int32_t)((const uint8_t *)A)[idx]
                    : (int32_t)((const int8_t *)A)[idx];
}

void orc_matmul_i8(const void *A, int64_t lda, const int8_t *B, int64_t ldb,
                   int32_t *C, int64_t ldc, int64_t M, int64_t N, int64_t K,
                   int a_unsigned, int b_nk) {
  for (int64_t i = 0; i < M; i++) {
    for (int64_t j = 0; j < N; j++) {
      uint32_t s = 0;
      for (int64_t k = 0; k < K; k++) {
        int32_t b = b_nk ? (int32_t)B[j * ldb + k] : (int32_t)B[k * ldb + j];
        s += (uint32_t)(a_elem(A, i * lda + k, a_unsigned) * b);
      }
      C[i * ldc + j] = (int32_t)s;
    }
  }
}

/* B_T[N,K] from B[K,N] (ConvertSimpToMemRef.cpp:3168-3216 materialises it). */
static int8_t *make_bt(const int8_t *B, int64_t N, int64_t K) {
  int8_t *bt = (int8_t *)malloc((size_t)(N * K > 0 ? N * K : 1));
  for (int64_t k = 0; k < K; k++)
    for (int64_t j = 0; j < N; j++) bt[j * K + k] = B[k * N + j];
  return bt;
}

/* One (row block of up to 4 rows, column j) cell group, scalar emulation of
 * the VNNI pass's loop body (VNNIPass.cpp:752-906). */
static void vnni_cell_scalar(const uint8_t *A, const int8_t *bt, int32_t *C,
                             int64_t i0, int64_t rows, int64_t j, int64_t N,
                             int64_t K, int a_unsigned) {
  uint8_t flip = a_unsigned ? 0x00 : 0x80;
  uint32_t acc[4] = {0, 0, 0, 0}, bias = 0, tail[4] = {0, 0, 0, 0};
  int64_t k = 0;
  for (; k + 64 <= K; k += 64) {
    for (int64_t kk = k; kk < k + 64; kk++) {
      int32_t b = bt[j * K + kk];
      for (int r = 0; r < rows; r++)
        acc[r] += (uint32_t)((int32_t)(uint8_t)(A[(i0 + r) * K + kk] ^ flip) * b);
      bias += (uint32_t)b;
    }
  }
  for (; k < K; k++) { /* scalar tail, on the original operand type */
    int32_t b = bt[j * K + k];
    for (int r = 0; r < rows; r++) {
      int32_t a = a_unsigned ? (int32_t)A[(i0 + r) * K + k]
                             : (int32_t)(int8_t)A[(i0 + r) * K + k];
      tail[r] += (uint32_t)(a * b);
    }
  }
  uint32_t corr = a_unsigned ? 0u : bias * 128u;
  for (int r = 0; r < rows; r++) C[(i0 + r) * N + j] = (int32_t)(acc[r] + tail[r] - corr);
}

#if ORC_HAVE_X86
__attribute__((target("avx512f,avx512bw,avx512vnni")))
static void vnni_block_avx512(const uint8_t *A, const int8_t *bt, int32_t *C,
                              int64_t i0, int64_t rows, int64_t N, int64_t K,
                              int a_unsigned) {
  const __m512i flip = _mm512_set1_epi8(a_unsigned ? 0 : (char)0x80);
  const __m512i ones = _mm512_set1_epi8(1);
  for (int64_t j = 0; j < N; j++) {
    __m512i acc[4], bias = _mm512_setzero_si512();
    for (int r = 0; r < 4; r++) acc[r] = _mm512_setzero_si512();
    int64_t k = 0;
    for (; k + 64 <= K; k += 64) {
      __m512i vb = _mm512_loadu_si512((const void *)&bt[j * K + k]);
      for (int r = 0; r < rows; r++) {
        __m512i va = _mm512_xor_si512(
            _mm512_loadu_si512((const void *)&A[(i0 + r) * K + k]), flip);
        acc[r] = _mm512_dpbusd_epi32(acc[r], va, vb);
      }
      bias = _mm512_dpbusd_epi32(bias, ones, vb);
    }
    uint32_t tail[4] = {0, 0, 0, 0};
    for (; k < K; k++) {
      int32_t b = bt[j * K + k];
      for (int r = 0; r < rows; r++) {
        int32_t a = a_unsigned ? (int32_t)A[(i0 + r) * K + k]
                               : (int32_t)(int8_t)A[(i0 + r) * K + k];
        tail[r] += (uint32_t)(a * b);
      }
    }
    uint32_t corr = a_unsigned ? 0u : (uint32_t)_mm512_reduce_add_epi32(bias) * 128u;
    for (int r = 0; r < rows; r++)
      C[(i0 + r) * N + j] =
          (int32_t)((uint32_t)_mm512_reduce_add_epi32(acc[r]) + tail[r] - corr);
  }
}
#endif

static int host_has_vnni(void) {
#if ORC_HAVE_X86
  __builtin_cpu_init();
  return __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512bw");
#else
  return 0;
#endif
}

int orc_matmul_i8_vnni(const void *A, const int8_t *B, int32_t *C, int64_t M,
                       int64_t N, int64_t K, int a_unsigned, int b_nk,
                       int nthreads) {
  const uint8_t *a = (const uint8_t *)A;
  int8_t *bt_owned = b_nk ? NULL : make_bt(B, N, K);
  const int8_t *bt = b_nk ? B : bt_owned;
  int use_vnni = host_has_vnni();
  int64_t nblk = (M + 3) / 4;
  if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads)
  for (int64_t blk = 0; blk < nblk; blk++) {
    int64_t i0 = blk * 4;
    int64_t rows = M - i0 < 4 ? M - i0 : 4;
#if ORC_HAVE_X86
    if (use_vnni) {
      vnni_block_avx512(a, bt, C, i0, rows, N, K, a_unsigned);
      continue;
    }
#endif
    for (int64_t j = 0; j < N; j++) vnni_cell_scalar(a, bt, C, i0, rows, j, N, K, a_unsigned);
  }
  free(bt_owned);
  return use_vnni;
}

static inline int32_t i4_at(const uint8_t *row, int64_t e) {
  const uint8_t byte = row[e >> 1];
  const int nib = (e & 1) ? (byte >> 4) : (byte & 15);
  return nib >= 8 ? nib - 16 : nib;  /* nibble | 0xF0 as s8 */
}

void orc_matmul_i4(const uint8_t *Ap, int64_t lda_p, const uint8_t *Bp, int64_t ldb_p,
                   int16_t *C, int64_t ldc, int64_t M, int64_t N, int64_t K) {
  /* the lowering's phases: unpack A, unpack B to B_T, i32 K-innermost sum, trunc */
  int8_t *bt = (int8_t *)malloc((size_t)(N > 0 ? N : 1) * (size_t)(K > 0 ? K : 1));
  for (int64_t j = 0; j < N; j++)
    for (int64_t k = 0; k < K; k++) bt[j * K + k] = (int8_t)i4_at(Bp + k * ldb_p, j);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M; i++) {
    int8_t *a = (int8_t *)malloc((size_t)(K > 0 ? K : 1));
    for (int64_t k = 0; k < K; k++) a[k] = (int8_t)i4_at(Ap + i * lda_p, k);
    for (int64_t j = 0; j < N; j++) {
      uint32_t acc = 0;  /* i32 wraparound */
      const int8_t *b = bt + j * K;
      for (int64_t k = 0; k < K; k++) acc += (uint32_t)(int32_t)((int16_t)a[k] * (int16_t)b[k]);
      C[i * ldc + j] = (int16_t)(uint16_t)(acc & 0xffffu);
    }
    free(a);
  }
  free(bt);
}

void orc_int4_recipe_inputs(int64_t N, uint8_t *Ap, uint8_t *Bp) {
  const int64_t pd = (N + 1) / 2;
  for (int64_t i = 0; i < N; i++)
    for (int64_t j = 0; j < N; j += 2) {
      const int v0 = (int)((i * N + j) % 15) - 7;
      const int v1 = j + 1 < N ? (int)((i * N + j + 1) % 15) - 7 : 0;
      Ap[i * pd + j / 2] = (uint8_t)((v0 & 15) | ((v1 & 15) << 4));
    }
  for (int64_t k = 0; k < N; k++)
    for (int64_t j = 0; j < N; j += 2) {
      const int v0 = (int)((j * N + k) % 15) - 7;
      const int v1 = j + 1 < N ? (int)(((j + 1) * N + k) % 15) - 7 : 0;
      Bp[k * pd + j / 2] = (uint8_t)((v0 & 15) | ((v1 & 15) << 4));
    }
}

int32_t orc_checksum_i16(const int16_t *C, int64_t n) {
  uint32_t s = 0;
  for (int64_t i = 0; i < n; i++) s += (uint32_t)(int32_t)C[i];
  return (int32_t)s;
}

void orc_int8_recipe_inputs(int64_t N, int8_t *A, int8_t *B) {
  for (int64_t i = 0; i < N; i++)
    for (int64_t j = 0; j < N; j++) {
      int v = (int)((i * N + j) % 127) - 64;
      A[i * N + j] = (int8_t)v;
      B[j * N + i] = (int8_t)v;
    }
}

int32_t orc_checksum_i32(const int32_t *C, int64_t n) {
  uint32_t s = 0;
  for (int64_t i = 0; i < n; i++) s += (uint32_t)C[i];
  return (int32_t)s;
}

/* ------------------------------------------------------------ fp32 ops -- */

void orc_matmul_f32_acc(const float *lhs, const float *rhs, float *out,
                        int64_t m, int64_t k, int64_t n, int64_t lhs_off,
                        int64_t rhs_off, int64_t out_off) {
  const float *A = lhs + lhs_off, *B = rhs + rhs_off;
  float *C = out + out_off;
  for (int64_t i = 0; i < m; i++)
    for (int64_t j = 0; j < n; j++) {
      float acc = C[i * n + j];
      for (int64_t kk = 0; kk < k; kk++) acc += A[i * k + kk] * B[kk * n + j];
      C[i * n + j] = acc;
    }
}

void orc_batch_matmul_f32(const float *A, const float *B, float *C, int64_t Bt,
                          int64_t M, int64_t K, int64_t N) {
  for (int64_t b = 0; b < Bt; b++)
    for (int64_t i = 0; i < M; i++)
      for (int64_t j = 0; j < N; j++) {
        double acc = 0.0;
        for (int64_t k = 0; k < K; k++)
          acc += (double)A[(b * M + i) * K + k] * (double)B[(b * K + k) * N + j];
        C[(b * M + i) * N + j] = (float)acc;
      }
}

void orc_batch_matmul_f64(const double *A, const double *B, double *C, int64_t Bt,
                          int64_t M, int64_t K, int64_t N) {
  for (int64_t b = 0; b < Bt; b++)
    for (int64_t i = 0; i < M; i++)
      for (int64_t j = 0; j < N; j++) {
        double acc = 0.0;
        for (int64_t k = 0; k < K; k++)
          acc += A[(b * M + i) * K + k] * B[(b * K + k) * N + j];
        C[(b * M + i) * N + j] = acc;
      }
}

void orc_rmsnorm(const float *in, const float *w, float *out, int64_t size,
                 float eps, int64_t w_off) {
  float ss = 0.0f;
  for (int64_t i = 0; i < size; i++) ss += in[i] * in[i];
  float rms = sqrtf(ss / (float)size + eps);
  for (int64_t i = 0; i < size; i++) out[i] = (in[i] / rms) * w[w_off + i];
}

void orc_softmax(const float *in, float *out, int64_t size, int64_t in_off,
                 int64_t out_off) {
  float mx = in[in_off];
  for (int64_t i = 1; i < size; i++)
    if (in[in_off + i] > mx) mx = in[in_off + i];
  float sum = 0.0f;
  for (int64_t i = 0; i < size; i++) {
    float e = expf(in[in_off + i] - mx);
    out[out_off + i] = e;
    sum += e;
  }
  for (int64_t i = 0; i < size; i++) out[out_off + i] = out[out_off + i] / sum;
}

void orc_silu(const float *in, float *out, int64_t size) {
  for (int64_t i = 0; i < size; i++) out[i] = in[i] / (1.0f + expf(-in[i]));
}

/* ------------------------------------------------------------------ W4 -- */

/* DequantW4OpLowering (src/mlir/lowering/ConvertSimpToMemRef.cpp:2367-2429)
 * evaluated at idx .. idx+count-1: q = nibble idx%2 of byte idx/2 (low =
 * even), g = idx/gs, q*scales[g] rounded, then + zeros[g] rounded. */
void orc_dequant_w4(const uint8_t *qw, const float *scales, const float *zeros, int64_t idx,
                    int64_t count, int64_t gs, float *out) {
  for (int64_t i = 0; i < count; i++) {
    const int64_t e = idx + i, g = e / gs;
    const uint8_t byte = qw[e / 2];
    const uint32_t q = (e % 2 == 0) ? (uint32_t)byte & 15u : ((uint32_t)byte >> 4) & 15u;
    const float scaled = (float)q * scales[g];
    out[i] = scaled + zeros[g];
  }
}

void orc_matmul_quant_f5(const uint8_t *qw, const float *scales,
                         const float *zeros, const float *in, float *out,
                         int64_t rows, int64_t cols, int64_t gs, int64_t off) {
  int64_t ngroups = cols / gs, ntiles = gs / 16;
  for (int64_t i = 0; i < rows; i++) {
    int64_t row_off = i * cols;
    out[i] = 0.0f;
    for (int64_t g = 0; g < ngroups; g++) {
      int64_t gidx = (off + row_off) / gs + g;
      float s = scales[gidx], z = zeros[gidx];
      float acc = 0.0f;
      for (int64_t t = 0; t < ntiles; t++) {
        float tile[16];
        int64_t k0 = g * gs + t * 16;
        for (int j = 0; j < 16; j++) {
          int64_t widx = off + row_off + k0 + j;
          uint8_t byte = qw[widx >> 1];
          uint32_t q = (widx & 1) ? (uint32_t)(byte >> 4) & 15u : (uint32_t)byte & 15u;
          float scaled = (float)q * s;
          tile[j] = scaled + z;
        }
        for (int j = 0; j < 16; j++) {
          int64_t kg = k0 + j;
          if (kg < cols) {
            float prod = tile[j] * in[kg];
            acc = acc + prod;
          }
        }
      }
      out[i] = out[i] + acc;
    }
  }
}

void orc_matmul_quant_f5_refidx(const uint8_t *qw, const float *scales, const float *zeros,
                                const float *in, float *out, int64_t rows, int64_t cols,
                                int64_t gs, int64_t off) {
  int64_t ngroups = cols / gs;                           /* :3929 numGroups = cols / gs */
  for (int64_t i = 0; i < rows; i++) {
    int64_t row_off = i * cols;                          /* :3919 rowOffset */
    out[i] = 0.0f;                                       /* :3922 */
    for (int64_t g = 0; g < ngroups; g++) {
      int64_t gidx = row_off / gs + g;                   /* :3936-3937, offset not added */
      float s = scales[gidx], z = zeros[gidx];
      float acc = 0.0f;
      for (int64_t t = 0; t < 8; t++) {                  /* :3942 numTiles = 8 */
        float tile[16];
        int64_t k0 = g * gs + t * 16;                    /* :3947-3949 kStart */
        for (int j = 0; j < 16; j++) {                   /* :3953-3982, unmasked loads */
          int64_t widx = off + row_off + k0 + j;
          uint32_t q = 0;
          if (k0 + j < cols) {  /* the reference loads past the row here; the value is unused */
            uint8_t byte = qw[widx >> 1];
            q = (widx & 1) ? (uint32_t)(byte >> 4) & 15u : (uint32_t)byte & 15u;
          }
          tile[j] = (float)q * s + z;
        }
        for (int j = 0; j < 16; j++)                     /* :3985-4003, k < cols */
          if (k0 + j < cols) acc = acc + tile[j] * in[k0 + j];
      }
      out[i] = out[i] + acc;                             /* :4007-4010 */
    }
  }
}

void orc_quantize_f5(const float *w, int64_t total, int64_t gs, uint8_t *qw,
                     float *scales, float *zeros) {
  int64_t ng = (total + gs - 1) / gs;
  memset(qw, 0, (size_t)((total + 1) / 2));
  for (int64_t g = 0; g < ng; g++) {
    int64_t st = g * gs, en = st + gs < total ? st + gs : total;
    float mn = w[st], mx = w[st];
    for (int64_t i = st; i < en; i++) {
      mn = w[i] < mn ? w[i] : mn;
      mx = w[i] > mx ? w[i] : mx;
    }
    float sc = (mx - mn) / 15.0f;
    if (sc < 1e-8f) sc = 1e-8f;
    scales[g] = sc;
    zeros[g] = mn;
    for (int64_t i = st; i < en; i++) {
      int q = (int)roundf((w[i] - mn) / sc);
      q = q < 0 ? 0 : (q > 15 ? 15 : q);
      if (i % 2 == 0) qw[i / 2] = (uint8_t)q;
      else qw[i / 2] |= (uint8_t)(q << 4);
    }
  }
}

static inline int32_t s4_at(const uint8_t *row, int64_t k) {
  uint8_t byte = row[k >> 1];
  int32_t n = (k & 1) ? (byte >> 4) & 15 : byte & 15;
  return n >= 8 ? n - 16 : n; /* n | 0xF0 as i8, ConvertSimpToMemRef.cpp:3030-3035 */
}

void orc_matmul_w4s(const uint8_t *qw, const float *scales, const float *x,
                    float *out, int64_t M, int64_t N, int64_t K, int64_t gs) {
  int64_t ng = K / gs;
  for (int64_t m = 0; m < M; m++)
    for (int64_t n = 0; n < N; n++) {
      const uint8_t *row = qw + n * (K / 2);
      double acc = 0.0;
      for (int64_t k = 0; k < K; k++) {
        float w = (float)s4_at(row, k) * scales[n * ng + k / gs];
        acc += (double)w * (double)x[m * K + k];
      }
      out[m * N + n] = (float)acc;
    }
}

void orc_matmul_w4s_f32(const uint8_t *qw, const float *scales, const float *x,
                        float *out, int64_t M, int64_t N, int64_t K, int64_t gs,
                        int nthreads) {
  int64_t ng = K / gs;
  if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads)
  for (int64_t n = 0; n < N; n++) {
    const uint8_t *row = qw + n * (K / 2);
    for (int64_t m = 0; m < M; m++) {
      float acc = 0.0f;
      for (int64_t g = 0; g < ng; g++) {
        float s = scales[n * ng + g], part = 0.0f;
        for (int64_t k = g * gs; k < (g + 1) * gs; k++)
          part += (float)s4_at(row, k) * x[m * K + k];
        acc += part * s;
      }
      out[m * N + n] = acc;
    }
  }
}

void orc_matmul_w4s_lowering(const uint8_t *qw, const float *scales, const float *x,
                             float *out, int64_t M, int64_t N, int64_t K, int64_t gs,
                             int nthreads) {
  const int64_t ng = K / gs, ntiles = gs / 16;
  if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads)
  for (int64_t i = 0; i < N; i++) {                       /* row loop, :3916 */
    const uint8_t *row = qw + i * (K / 2);
    for (int64_t m = 0; m < M; m++) {
      const float *in = x + m * K;
      float o = 0.0f;                                      /* :3922 */
      for (int64_t g = 0; g < ng; g++) {                   /* group loop, :3929-3932 */
        const float scale = scales[i * ng + g];            /* :3938, no zero point */
        float acc = 0.0f;
        for (int64_t t = 0; t < ntiles; t++) {             /* tile loop, :3942-4005 */
          float tile[16];
          const int64_t k0 = g * gs + t * 16;
          for (int j = 0; j < 16; j++)                      /* dequantise 16, :3953-3982 */
            tile[j] = (float)s4_at(row, k0 + j) * scale;
          for (int j = 0; j < 16; j++)                      /* dot, :3985-4003 */
            if (k0 + j < K) acc = acc + tile[j] * in[k0 + j];
        }
        o = o + acc;                                       /* :4007-4010 */
      }
      out[m * N + i] = o;
    }
  }
}

/* -------------------------------------------------------------- decode -- */

void orc_rope(float *q, float *k, int64_t dim, int64_t kv_dim, int64_t hs,
              int64_t pos, float theta) {
  for (int64_t i = 0; i < dim; i += 2) {
    float hd = (float)(i % hs), hsf = (float)hs;
    float freq = 1.0f / powf(theta, hd / hsf);
    float val = (float)pos * freq;
    float fcr = cosf(val), fci = sinf(val);
    float q0 = q[i], q1 = q[i + 1];
    q[i] = q0 * fcr - q1 * fci;
    q[i + 1] = q0 * fci + q1 * fcr;
    if (i < kv_dim) {
      float k0 = k[i], k1 = k[i + 1];
      k[i] = k0 * fcr - k1 * fci;
      k[i + 1] = k0 * fci + k1 * fcr;
    }
  }
}

/* y[rows] = W[rows, cols] x, W either fp32 or F6 W4 (double accumulation). */
static void gemv(const orc_llama_cfg *c, const float *wf, const uint8_t *wq,
                 const float *ws, const float *x, float *y, int64_t rows,
                 int64_t cols) {
  if (c->w4) {
    int64_t ng = cols / c->gs;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
      const uint8_t *row = wq + r * (cols / 2);
      double acc = 0.0;
      for (int64_t k = 0; k < cols; k++) {
        float w = (float)s4_at(row, k) * ws[r * ng + k / c->gs];
        acc += (double)w * (double)x[k];
      }
      y[r] = (float)acc;
    }
    return;
  }
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; r++) {
    double acc = 0.0;
    for (int64_t j = 0; j < cols; j++) acc += (double)wf[r * cols + j] * (double)x[j];
    y[r] = (float)acc;
  }
}

void orc_llama_forward(const orc_llama_cfg *c, const orc_llama_weights *w,
                       float *key_cache, float *value_cache, int64_t token,
                       int64_t pos, float *logits) {
  int64_t dim = c->dim, hid = c->hidden, hs = dim / c->n_heads;
  int64_t kv_dim = dim * c->n_kv_heads / c->n_heads;
  float *x = (float *)malloc(sizeof(float) * dim);
  float *xb = (float *)malloc(sizeof(float) * dim);
  float *xb2 = (float *)malloc(sizeof(float) * dim);
  float *q = (float *)malloc(sizeof(float) * dim);
  float *kk = (float *)malloc(sizeof(float) * kv_dim);
  float *vv = (float *)malloc(sizeof(float) * kv_dim);
  float *hb = (float *)malloc(sizeof(float) * hid);
  float *hb2 = (float *)malloc(sizeof(float) * hid);
  float *att = (float *)malloc(sizeof(float) * (pos + 1));
  float *att_soft = (float *)malloc(sizeof(float) * (pos + 1));
  memcpy(x, w->emb + token * dim, sizeof(float) * dim);
  float scale = sqrtf((float)hs);
  int64_t sq_w4 = c->gs > 0 ? dim / c->gs : 0;
  for (int64_t l = 0; l < c->n_layers; l++) {
    orc_rmsnorm(x, w->rms_att, xb, dim, c->eps, l * dim);
    /* per-layer W4 slices: bytes rows*cols/2, scales rows*cols/gs */
#define WF(p, r, cl) ((p) ? (p) + l * (r) * (cl) : NULL)
#define WQ(p, r, cl) ((p) ? (p) + l * (r) * (cl) / 2 : NULL)
#define WS(p, r, cl) ((p) ? (p) + l * (r) * (cl) / c->gs : NULL)
    gemv(c, WF(w->wq, dim, dim), WQ(w->q_wq, dim, dim), c->w4 ? WS(w->s_wq, dim, dim) : NULL, xb, q, dim, dim);
    gemv(c, WF(w->wk, kv_dim, dim), WQ(w->q_wk, kv_dim, dim), c->w4 ? WS(w->s_wk, kv_dim, dim) : NULL, xb, kk, kv_dim, dim);
    gemv(c, WF(w->wv, kv_dim, dim), WQ(w->q_wv, kv_dim, dim), c->w4 ? WS(w->s_wv, kv_dim, dim) : NULL, xb, vv, kv_dim, dim);
    orc_rope(q, kk, dim, kv_dim, hs, pos, c->theta);
    float *kc = key_cache + l * c->seq_len * kv_dim, *vc = value_cache + l * c->seq_len * kv_dim;
    memcpy(kc + pos * kv_dim, kk, sizeof(float) * kv_dim);
    memcpy(vc + pos * kv_dim, vv, sizeof(float) * kv_dim);
    for (int64_t h = 0; h < c->n_heads; h++) {
      int64_t kvh = h * c->n_kv_heads / c->n_heads;
      const float *qh = q + h * hs;
      for (int64_t t = 0; t <= pos; t++) {
        const float *kt = kc + t * kv_dim + kvh * hs;
        double s = 0.0;
        for (int64_t i = 0; i < hs; i++) s += (double)qh[i] * (double)kt[i];
        att[t] = (float)s / scale;
      }
      orc_softmax(att, att_soft, pos + 1, 0, 0);
      for (int64_t i = 0; i < hs; i++) {
        double v = 0.0;
        for (int64_t t = 0; t <= pos; t++)
          v += (double)att_soft[t] * (double)vc[t * kv_dim + kvh * hs + i];
        xb[h * hs + i] = (float)v;
      }
    }
    gemv(c, WF(w->wo, dim, dim), WQ(w->q_wo, dim, dim), c->w4 ? WS(w->s_wo, dim, dim) : NULL, xb, xb2, dim, dim);
    for (int64_t i = 0; i < dim; i++) x[i] = x[i] + xb2[i];
    orc_rmsnorm(x, w->rms_ffn, xb, dim, c->eps, l * dim);
    gemv(c, WF(w->w1, hid, dim), WQ(w->q_w1, hid, dim), c->w4 ? WS(w->s_w1, hid, dim) : NULL, xb, hb, hid, dim);
    gemv(c, WF(w->w3, hid, dim), WQ(w->q_w3, hid, dim), c->w4 ? WS(w->s_w3, hid, dim) : NULL, xb, hb2, hid, dim);
    orc_silu(hb, hb, hid);
    for (int64_t i = 0; i < hid; i++) hb[i] = hb[i] * hb2[i];
    gemv(c, WF(w->w2, dim, hid), WQ(w->q_w2, dim, hid), c->w4 ? WS(w->s_w2, dim, hid) : NULL, hb, xb, dim, hid);
    for (int64_t i = 0; i < dim; i++) x[i] = x[i] + xb[i];
#undef WF
#undef WQ
#undef WS
  }
  (void)sq_w4;
  orc_rmsnorm(x, w->rms_final, xb, dim, c->eps, 0);
  gemv(c, w->wcls, w->q_wcls, w->s_wcls, xb, logits, c->vocab, dim);
  free(x); free(xb); free(xb2); free(q); free(kk); free(vv);
  free(hb); free(hb2); free(att); free(att_soft);
}

/* ----------------------------------------------- llama32_forward (int8) -- */

/* (i8) of an fp32 value as x86 code lowers it: cvttss2si to i32 (0x80000000 for
 * NaN and out-of-range), then the low byte. */
static int8_t l32_fptosi_i8(float v) {
  if (!(v > -2147483648.0f && v < 2147483648.0f)) return 0;
  return (int8_t)(uint8_t)(uint32_t)(int32_t)v;
}

/* val = v * 127.0; clamp to [-128, 127]; (i8)val (llama32_1b_int8_tensor.sl:90-96) */
static int8_t l32_quant127(float v) {
  float val = v * 127.0f;
  if (val > 127.0f) val = 127.0f;
  if (val < -128.0f) val = -128.0f;
  return (int8_t)(int32_t)val;
}

/* y[n] = sum_k x[k] * w[n*K + k], i8 x i8 -> i32 with wraparound
 * (tensor_matmul_nt on [1,K] x [N,K], ConvertSimpToMemRef.cpp:3373-3486). */
static void l32_mv_nt(const int8_t *x, const int8_t *w, int64_t N, int64_t K, int32_t *y) {
  for (int64_t n = 0; n < N; n++) {
    uint32_t acc = 0;
    for (int64_t k = 0; k < K; k++) acc += (uint32_t)((int32_t)x[k] * (int32_t)w[n * K + k]);
    y[n] = (int32_t)acc;
  }
}

float orc_llama32_int8_forward(const orc_llama_cfg *c, int64_t hs, const int8_t *x_i8,
                               const float *rms_att, const float *rms_ffn,
                               const float *rms_final, const int8_t *wq, const int8_t *wk,
                               const int8_t *wv, const int8_t *wo, const int8_t *w1,
                               const int8_t *w2, const int8_t *w3, const float *wcls,
                               float *x, float *xb, float *logits, int8_t *xb_i8,
                               int8_t *kc, int8_t *vc, float *att_scores, float *att_probs,
                               int32_t *attn_out, int8_t *ffn_hb, int64_t pos) {
  const int64_t dim = c->dim, hid = c->hidden, L = c->n_layers, nh = c->n_heads;
  const int64_t S = c->seq_len, kv = c->n_kv_heads * hs, n_rep = nh / c->n_kv_heads;
  const int64_t seq_len = pos + 1;
  int32_t *Q = malloc(sizeof(int32_t) * dim), *K = malloc(sizeof(int32_t) * kv);
  int32_t *V = malloc(sizeof(int32_t) * kv), *D = malloc(sizeof(int32_t) * dim);
  int32_t *G = malloc(sizeof(int32_t) * hid), *U = malloc(sizeof(int32_t) * hid);
  for (int64_t i = 0; i < dim; i++) x[i] = (float)x_i8[i] * 1.0f;           /* :79-83 */
  for (int64_t l = 0; l < L; l++) {
    orc_rmsnorm(x, rms_att, xb, dim, 1e-5f, l * dim);                      /* :93 */
    for (int64_t i = 0; i < dim; i++) xb_i8[i] = l32_quant127(xb[i]);      /* :96-102 */
    l32_mv_nt(xb_i8, wq + l * dim * dim, dim, dim, Q);                     /* :104-121 */
    l32_mv_nt(xb_i8, wk + l * kv * dim, kv, dim, K);
    l32_mv_nt(xb_i8, wv + l * kv * dim, kv, dim, V);
    const int64_t co = l * S * kv + pos * kv;                              /* :142-151 */
    for (int64_t i = 0; i < kv; i++) {
      kc[co + i] = (int8_t)(uint8_t)(uint64_t)((int64_t)K[i] / 256);
      vc[co + i] = (int8_t)(uint8_t)(uint64_t)((int64_t)V[i] / 256);
    }
    for (int64_t i = 0; i < dim; i++) attn_out[i] = 0;                    /* :155-159 */
    for (int64_t h = 0; h < nh; h++) {                                     /* :161-204 */
      const int64_t qo = h * hs, kho = (h / n_rep) * hs;
      for (int64_t t = 0; t < seq_len; t++) {
        float score = 0.0f;
        const int8_t *kp = kc + l * S * kv + t * kv + kho;
        for (int64_t d = 0; d < hs; d++) score = score + (float)Q[qo + d] * 1.0f * ((float)kp[d] * 1.0f);
        score = score / 8.0f;
        att_scores[h * S + t] = score;
      }
      orc_softmax(att_scores, att_probs, seq_len, h * S, h * S);
      for (int64_t d = 0; d < hs; d++) {
        float val = 0.0f;
        for (int64_t t = 0; t < seq_len; t++)
          val = val + att_probs[h * S + t] * ((float)vc[l * S * kv + t * kv + kho + d] * 1.0f);
        attn_out[qo + d] = (int32_t)val;
      }
    }
    for (int64_t i = 0; i < dim; i++) {                                    /* :208-216 */
      float val = (float)attn_out[i] * 1.0f / 256.0f;
      if (val > 127.0f) val = 127.0f;
      if (val < -128.0f) val = -128.0f;
      xb_i8[i] = (int8_t)(int32_t)val;
    }
    l32_mv_nt(xb_i8, wo + l * dim * dim, dim, dim, D);                    /* :218-222 */
    for (int64_t i = 0; i < dim; i++) x[i] = x[i] + (float)D[i] * 1.0f / 65536.0f;  /* :225-229 */
    orc_rmsnorm(x, rms_ffn, xb, dim, 1e-5f, l * dim);                      /* :232 */
    for (int64_t i = 0; i < dim; i++) xb_i8[i] = l32_quant127(xb[i]);      /* :235-242 */
    l32_mv_nt(xb_i8, w1 + l * hid * dim, hid, dim, G);                     /* :245-256 */
    l32_mv_nt(xb_i8, w3 + l * hid * dim, hid, dim, U);
    for (int64_t i = 0; i < hid; i++) {                                    /* :258-267 */
      const float gate_f = (float)G[i] * 1.0f / 65536.0f;
      const float silu = gate_f / (1.0f + expf(0.0f - gate_f));
      const float up_f = (float)U[i] * 1.0f / 65536.0f;
      ffn_hb[i] = l32_fptosi_i8(silu * up_f * 127.0f);
    }
    l32_mv_nt(ffn_hb, w2 + l * dim * hid, dim, hid, D);                   /* :269-272 */
    for (int64_t i = 0; i < dim; i++) x[i] = x[i] + (float)D[i] * 1.0f / 65536.0f;  /* :275-279 */
  }
  orc_rmsnorm(x, rms_final, xb, dim, 1e-5f, 0);                            /* :287 */
  for (int64_t i = 0; i < c->vocab; i++) {                                 /* :292-302 */
    float sum = 0.0f;
    for (int64_t j = 0; j < dim; j++) sum = sum + wcls[i * dim + j] * xb[j];
    logits[i] = sum;
  }
  free(Q); free(K); free(V); free(D); free(G); free(U);
  return logits[0];
}

void orc_llama_quant_forward(const orc_llama_cfg *c, const float *emb, const float *rms_att,
                             const float *rms_ffn, const float *rms_final, const float *wcls,
                             const uint8_t *qw, const float *scales, const float *zeros,
                             int64_t gs, const int64_t off[7], float *key_cache,
                             float *value_cache, int64_t token, int64_t pos, float *logits) {
  const int64_t dim = c->dim, hid = c->hidden, hs = dim / c->n_heads;
  const int64_t kv_dim = dim * c->n_kv_heads / c->n_heads;
  float *x = (float *)malloc(sizeof(float) * dim);
  float *xb = (float *)malloc(sizeof(float) * dim);
  float *xb2 = (float *)malloc(sizeof(float) * dim);
  float *q = (float *)malloc(sizeof(float) * dim);
  float *kk = (float *)malloc(sizeof(float) * kv_dim);
  float *vv = (float *)malloc(sizeof(float) * kv_dim);
  float *hb = (float *)malloc(sizeof(float) * hid);
  float *hb2 = (float *)malloc(sizeof(float) * hid);
  float *att = (float *)malloc(sizeof(float) * (pos + 1));
  float *att_soft = (float *)malloc(sizeof(float) * (pos + 1));
  memcpy(x, emb + token * dim, sizeof(float) * dim);                 /* :61-66 */
  for (int64_t l = 0; l < c->n_layers; l++) {
    orc_rmsnorm(x, rms_att, xb, dim, c->eps, l * dim);                /* :73 */
    /* :77-83, the matrix element offsets advance by rows*cols per layer */
    orc_matmul_quant_f5(qw, scales, zeros, xb, q, dim, dim, gs, off[0] + l * dim * dim);
    orc_matmul_quant_f5(qw, scales, zeros, xb, kk, kv_dim, dim, gs, off[1] + l * dim * kv_dim);
    orc_matmul_quant_f5(qw, scales, zeros, xb, vv, kv_dim, dim, gs, off[2] + l * dim * kv_dim);
    float *kc = key_cache + l * c->seq_len * kv_dim, *vc = value_cache + l * c->seq_len * kv_dim;
    memcpy(kc + pos * kv_dim, kk, sizeof(float) * kv_dim);          /* :86-92 */
    memcpy(vc + pos * kv_dim, vv, sizeof(float) * kv_dim);
    const float scale = sqrtf((float)hs);
    for (int64_t h = 0; h < c->n_heads; h++) {                       /* :95-133 */
      const int64_t kvh = h * c->n_kv_heads / c->n_heads;
      const float *qh = q + h * hs;
      for (int64_t t = 0; t <= pos; t++) {
        const float *kt = kc + t * kv_dim + kvh * hs;
        double sc = 0.0;
        for (int64_t i = 0; i < hs; i++) sc += (double)qh[i] * (double)kt[i];
        att[t] = (float)sc / scale;
      }
      orc_softmax(att, att_soft, pos + 1, 0, 0);
      for (int64_t i = 0; i < hs; i++) {
        double v = 0.0;
        for (int64_t t = 0; t <= pos; t++)
          v += (double)att_soft[t] * (double)vc[t * kv_dim + kvh * hs + i];
        xb2[h * hs + i] = (float)v;
      }
    }
    orc_matmul_quant_f5(qw, scales, zeros, xb2, xb, dim, dim, gs, off[3] + l * dim * dim); /* :136 */
    for (int64_t i = 0; i < dim; i++) x[i] = x[i] + xb[i];            /* :139-143 */
    orc_rmsnorm(x, rms_ffn, xb, dim, c->eps, l * dim);                /* :146 */
    orc_matmul_quant_f5(qw, scales, zeros, xb, hb, hid, dim, gs, off[4] + l * hid * dim);
    orc_matmul_quant_f5(qw, scales, zeros, xb, hb2, hid, dim, gs, off[6] + l * hid * dim);
    orc_silu(hb, hb, hid);                                            /* :163 */
    for (int64_t i = 0; i < hid; i++) hb[i] = hb[i] * hb2[i];         /* :165-169 */
    orc_matmul_quant_f5(qw, scales, zeros, hb, xb, dim, hid, gs, off[5] + l * dim * hid);
    for (int64_t i = 0; i < dim; i++) x[i] = x[i] + xb[i];            /* :174-178 */
  }
  orc_rmsnorm(x, rms_final, xb, dim, c->eps, 0);                      /* :184 */
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < c->vocab; i++) {                            /* :187-196 */
    double sm = 0.0;
    for (int64_t j = 0; j < dim; j++) sm += (double)wcls[i * dim + j] * (double)xb[j];
    logits[i] = (float)sm;
  }
  free(x); free(xb); free(xb2); free(q); free(kk); free(vv);
  free(hb); free(hb2); free(att); free(att_soft);
}

/* sample_argmax (examples/llama2/generate_stories110M.cpp:73-83): seeded with
 * logits[0], moves on a strict '>' (NaN compares false). */
int64_t orc_argmax(const float *logits, int64_t n) {
  int64_t best = 0;
  float mv = logits[0];
  for (int64_t i = 1; i < n; i++)
    if (logits[i] > mv) {
      mv = logits[i];
      best = i;
    }
  return best;
}


/* ---- symmetric W4 quantization (signed nibbles, one scale per group) ---- */
void orc_quantize_w4s(const float *w, int64_t rows, int64_t cols, int64_t gs, uint8_t *qw,
                      float *scales) {
  const int64_t gpr = cols / gs;
  memset(qw, 0, (size_t)(rows * cols / 2));
  for (int64_t r = 0; r < rows; r++)
    for (int64_t g = 0; g < gpr; g++) {
      const float *src = w + r * cols + g * gs;
      float amax = 0.f;
      for (int64_t i = 0; i < gs; i++) amax = fabsf(src[i]) > amax ? fabsf(src[i]) : amax;
      const float s = amax > 0.f ? amax / 7.0f : 1.0f;
      scales[r * gpr + g] = s;
      for (int64_t i = 0; i < gs; i++) {
        int q = (int)roundf(src[i] / s);
        q = q < -8 ? -8 : (q > 7 ? 7 : q);
        const int64_t k = g * gs + i;
        uint8_t *b = qw + r * (cols / 2) + k / 2;
        if (k % 2 == 0) *b = (uint8_t)(q & 15);
        else *b |= (uint8_t)((q & 15) << 4);
      }
    }
}

/* ---- MT19937 and the reference's temperature sampler ---- */
void orc_mt_seed(orc_mt19937 *g, uint32_t seed) {
  g->mt[0] = seed;
  for (int i = 1; i < 624; i++)
    g->mt[i] = 1812433253u * (g->mt[i - 1] ^ (g->mt[i - 1] >> 30)) + (uint32_t)i;
  g->idx = 624;
}

uint32_t orc_mt_next(orc_mt19937 *g) {
  if (g->idx >= 624) {
    for (int i = 0; i < 624; i++) {
      const uint32_t y = (g->mt[i] & 0x80000000u) | (g->mt[(i + 1) % 624] & 0x7fffffffu);
      g->mt[i] = g->mt[(i + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
    }
    g->idx = 0;
  }
  uint32_t y = g->mt[g->idx++];
  y ^= y >> 11;
  y ^= (y << 7) & 0x9d2c5680u;
  y ^= (y << 15) & 0xefc60000u;
  y ^= y >> 18;
  return y;
}

float orc_uniform01f(orc_mt19937 *g) {
  const float r = (float)orc_mt_next(g) / 4294967296.0f;
  return r >= 1.0f ? nextafterf(1.0f, 0.0f) : r;
}

int64_t orc_sample(const float *logits, int64_t n, float temperature, orc_mt19937 *g) {
  if (n <= 0) return -1;
  if (temperature == 0.0f) return orc_argmax(logits, n);
  float *p = (float *)malloc(sizeof(float) * (size_t)n);
  for (int64_t i = 0; i < n; i++) p[i] = logits[i] / temperature;
  float mx = p[0];
  for (int64_t i = 1; i < n; i++) mx = p[i] > mx ? p[i] : mx;
  float sum = 0.0f;
  for (int64_t i = 0; i < n; i++) {
    p[i] = expf(p[i] - mx);
    sum += p[i];
  }
  for (int64_t i = 0; i < n; i++) p[i] /= sum;
  const float r = orc_uniform01f(g);
  float cdf = 0.0f;
  int64_t tok = n - 1;
  for (int64_t i = 0; i < n; i++) {
    cdf += p[i];
    if (r < cdf) {
      tok = i;
      break;
    }
  }
  free(p);
  return tok;
}
