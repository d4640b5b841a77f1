/*
 * oracle.h -- CPU restatement of SimpLang's tensor-op hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP runtime
 * (libsimp_hip.so): it is loaded by tests/, by __graft_entry__.smoke() and by
 * bench.py's cpu_baseline leg, and by nothing on the product path.
 *
 * Every function cites the reference code it restates (paths relative to the
 * SimpLang source tree).  Parity status of each function, and what pins it,
 * is listed next to the declaration ("pinned by ...").
 */
#ifndef SIMP_ORACLE_H
#define SIMP_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- int8 -- */

/* vpdpbusd on one 512-bit register: 16 lanes, each lane
 *   out[i] = acc[i] + sum_{j<4} (u8)a[4i+j] * (s8)b[4i+j]     (i32 wraparound)
 * Restates scalar_vpdpbusd_reference, simptensor/tests/test_vnni_correctness.cpp:28-42.
 * Pinned by the nine known answers of that file (:76-361) and by the reference
 * function itself, compiled in place into oracle/_ref. */
void orc_vpdpbusd16(const uint8_t *a, const int8_t *b, const int32_t *acc,
                    int32_t *out);

/* Textbook int8 GEMM, C[M,N] = A[M,K] * B, i32 accumulation with wraparound.
 *   a_unsigned = 0 : A is s8 (SimpLang tensor_matmul, F1:
 *                    src/mlir/lowering/ConvertSimpToMemRef.cpp:3233-3239)
 *   a_unsigned = 1 : A is u8 (raw vpdpbusd semantics, test_vnni_correctness.cpp:28-42)
 *   b_nk = 0 : B is [K,N] row-major, ldb >= N (tensor_matmul)
 *   b_nk = 1 : B is B_T[N,K] row-major, ldb >= K (tensor_matmul_nt,
 *              ConvertSimpToMemRef.cpp:3373-3486)
 * Strides are in elements.  Pinned by closed forms (identity, one-hot) and the
 * reference's own VNNI kernel compiled in place. */
void orc_matmul_i8(const void *A, int64_t lda, const int8_t *B, int64_t ldb,
                   int32_t *C, int64_t ldc, int64_t M, int64_t N, int64_t K,
                   int a_unsigned, int b_nk);

/* The algorithm the reference's VNNI pass emits (src/mlir/passes/VNNIPass.cpp:597-999,
 * hand-written twin simptensor/benchmarks/bench_int8_matmul_multicore.cpp:88-132):
 * B is first transposed to B_T[N,K]; rows are taken 4 at a time (I=4); K runs
 * in 64-byte vpdpbusd steps; for s8 A the bytes are flipped (A^0x80 = A+128 as
 * u8) and 128*colsum(B) is subtracted; a scalar loop covers the K tail.  Unlike
 * the reference (defects D1/D2) it also handles M%4 != 0 and K%64 != 0.
 * Uses AVX-512 VNNI when the host has it, a scalar emulation of the same steps
 * otherwise.  nthreads > 1 splits the row blocks with OpenMP.  This is the
 * "port" CPU baseline timed by bench.py.  b_nk as in orc_matmul_i8.
 * Returns 1 if the AVX-512 VNNI path ran, 0 for the scalar path. */
int orc_matmul_i8_vnni(const void *A, const int8_t *B, int32_t *C, int64_t M,
                       int64_t N, int64_t K, int a_unsigned, int b_nk,
                       int nthreads);

/* Deterministic inputs of the reference's int8 benchmark:
 *   val = ((i*N + j) % 127) - 64;  A[i,j] = val;  B[j,i] = val
 * simptensor/benchmarks/bench_int8_matmul_runner.cpp:37-43. */
void orc_int8_recipe_inputs(int64_t N, int8_t *A, int8_t *B);

/* i32 wraparound sum of n values (bench_int8_matmul_runner.cpp:57-61). */
int32_t orc_checksum_i32(const int32_t *C, int64_t n);

/* ---------------------------------------------------------------- int4 -- */

/* Packed signed-nibble tensor_matmul (src/mlir/lowering/ConvertSimpToMemRef.cpp:
 * 2953-3133): A[M,K] packed along K into bytes Ap[M, lda_p] and B[K,N] packed
 * along N into Bp[K, ldb_p]; element e of a row sits in byte e/2, low nibble for
 * even e, sign-extended (>= 8 -> |0xF0).  Each C[i,j] is the i32 sum over K of
 * the products, truncated to i16 (:3119-3122). */
void orc_matmul_i4(const uint8_t *Ap, int64_t lda_p, const uint8_t *Bp, int64_t ldb_p,
                   int16_t *C, int64_t ldc, int64_t M, int64_t N, int64_t K);

/* Deterministic packed inputs of the reference's int4 benchmark
 * (simptensor/benchmarks/bench_int4_matmul_runner.cpp:76-113):
 * A[i,k] = ((i*N + k) % 15) - 7 packed along k;  B[k,j] = ((j*N + k) % 15) - 7
 * packed along j; an odd last nibble of a row is 0.  Ap and Bp are [N, (N+1)/2]. */
void orc_int4_recipe_inputs(int64_t N, uint8_t *Ap, uint8_t *Bp);

/* Sum of n i16 values as i32 (bench_int4_matmul_runner.cpp:139-143). */
int32_t orc_checksum_i16(const int16_t *C, int64_t n);

/* ------------------------------------------------------------ fp32 ops -- */

/* Rank-3 tensor_matmul: C[b,i,j] = sum_k A[b,i,k] * B[b,k,j] for A[Bt,M,K],
 * B[Bt,K,N], contiguous, C overwritten (linalg.batch_matmul into the zero-filled
 * result, src/mlir/lowering/ConvertSimpToMemRef.cpp:2926-2933,3286-3291).  The
 * sum is taken in double, k increasing, and rounded once.  Pinned by the known
 * answers of simptensor/tests/test_matmul_dot.sl:135-199 (20.0, 19.0) and
 * tests/test_tensor_matmul.sl:66-117 (C[0,0,0] = 20 from its fill formulas), and
 * by agreement with orc_matmul_f32_acc batch by batch. */
void orc_batch_matmul_f32(const float *A, const float *B, float *C, int64_t Bt,
                          int64_t M, int64_t K, int64_t N);
void orc_batch_matmul_f64(const double *A, const double *B, double *C, int64_t Bt,
                          int64_t M, int64_t K, int64_t N);

/* Array builtin matmul: C += A*B on 1-D arrays viewed as row-major matrices
 * at element offsets (src/mlir/lowering/ConvertSimpToMemRef.cpp:1794-1920,
 * F4).  K is summed in increasing order in fp32 starting from C. */
void orc_matmul_f32_acc(const float *lhs, const float *rhs, float *out,
                        int64_t m, int64_t k, int64_t n, int64_t lhs_off,
                        int64_t rhs_off, int64_t out_off);

/* rmsnorm: sequential fp32 sum of squares, rms = sqrtf(ss/size + eps),
 * out[i] = (in[i] / rms) * w[w_off + i]  (ConvertSimpToMemRef.cpp:2192-2233). */
void orc_rmsnorm(const float *in, const float *w, float *out, int64_t size,
                 float eps, int64_t w_off);

/* softmax with offsets: max seeded with in[in_off] and updated with strict '>',
 * out = expf(x - max), sequential sum, out /= sum (ConvertSimpToMemRef.cpp:2264-2316). */
void orc_softmax(const float *in, float *out, int64_t size, int64_t in_off,
                 int64_t out_off);

/* silu: out = x / (1 + expf(-x))  (ConvertSimpToMemRef.cpp:2345-2354). */
void orc_silu(const float *in, float *out, int64_t size);

/* ------------------------------------------------------------------ W4 -- */

/* dequant_w4 (ConvertSimpToMemRef.cpp:2367-2429) at idx .. idx+count-1:
 * unsigned nibble * scale + zero of the element's flat group. */
void orc_dequant_w4(const uint8_t *qw, const float *scales, const float *zeros, int64_t idx,
                    int64_t count, int64_t gs, float *out);

/* Reference W4 format (F5): unsigned nibbles, low nibble = even flat index,
 * w = q*scale + zero, groups are flat runs of gs weights.
 * Restates MatMulQuantOpLowering (ConvertSimpToMemRef.cpp:3906-4005): per row,
 * out = 0; per group an fp32 partial summed over gs/16 tiles of 16 in order,
 * then out += partial.  Two reference defects are fixed (D3): the group index
 * includes the weight offset, (off + i*cols)/gs + g, and the tile count is
 * gs/16 instead of a fixed 8.  Requires gs % 16 == 0 and cols % gs == 0. */
void orc_matmul_quant_f5(const uint8_t *qw, const float *scales,
                         const float *zeros, const float *in, float *out,
                         int64_t rows, int64_t cols, int64_t gs, int64_t off);

/* MatMulQuantOpLowering exactly as the reference emits it
 * (src/mlir/lowering/ConvertSimpToMemRef.cpp:3906-4011), defects included:
 * the scale/zero index is (i*cols)/gs + g without the weight offset, and every
 * group runs a fixed 8 tiles of 16 weights from g*gs, so for gs < 128 the tiles
 * of neighbouring groups overlap (weights k with k < cols only; each is
 * dequantised with the scale of the group whose loop reads it).  Used by tests
 * to show where orc_matmul_quant_f5 (and the GPU) differ from the reference:
 * equal for off = 0 and gs = 128, otherwise not. */
void orc_matmul_quant_f5_refidx(const uint8_t *qw, const float *scales, const float *zeros,
                                const float *in, float *out, int64_t rows, int64_t cols,
                                int64_t gs, int64_t off);

/* Reference quantizer for F5 (examples/llama2/bench_llama_quant.cpp:51-93):
 * per flat group, scale = max((max-min)/15, 1e-8), zero = min,
 * q = clamp(round((w-min)/scale), 0, 15). */
void orc_quantize_f5(const float *w, int64_t total, int64_t gs, uint8_t *qw,
                     float *scales, float *zeros);

/* Symmetric W4 format (F6): signed nibbles in [-8,7] (sign-extended as in
 * ConvertSimpToMemRef.cpp:3016-3037, low nibble = even k), W[N,K] packed along
 * K (row = K/2 bytes), one fp32 scale per group of gs along K (scales[N, K/gs]),
 * no zero point.  out[m,n] = sum_k (q[n,k]*s[n,k/gs]) * x[m,k], accumulated in
 * double (the exact value the GPU is compared against). */
void orc_matmul_w4s(const uint8_t *qw, const float *scales, const float *x,
                    float *out, int64_t M, int64_t N, int64_t K, int64_t gs);

/* Same math as orc_matmul_w4s with fp32 accumulation and OpenMP over rows:
 * the CPU baseline for the W4 GEMV (bench.py). */
void orc_matmul_w4s_f32(const uint8_t *qw, const float *scales, const float *x,
                        float *out, int64_t M, int64_t N, int64_t K, int64_t gs,
                        int nthreads);

/* The symmetric format through the loop structure MatMulQuantOpLowering emits
 * (ConvertSimpToMemRef.cpp:3906-4011): per output row, per group an fp32
 * partial over gs/16 tiles of 16 weights, each tile dequantised into a buffer
 * (q * scale; this format has no zero point) and then dotted with x in order,
 * the partial added to the row's sum.  One x row after another (the reference
 * op takes one); OpenMP over output rows.  The CPU baseline of the W4 GEMV
 * (bench.py); agrees with orc_matmul_w4s to fp32 rounding. */
void orc_matmul_w4s_lowering(const uint8_t *qw, const float *scales, const float *x,
                             float *out, int64_t M, int64_t N, int64_t K, int64_t gs,
                             int nthreads);

/* -------------------------------------------------------------- decode -- */

/* RoPE of the LLaMA programs (examples/llama2/stories110M.sl:86-112):
 * for even i < dim: f = 1/powf(theta, (i % hs)/hs), v = pos*f,
 * rotate (q[i], q[i+1]) by v; k likewise when i < kv_dim. */
void orc_rope(float *q, float *k, int64_t dim, int64_t kv_dim, int64_t hs,
              int64_t pos, float theta);

/* Model shape of one decode step (examples/llama2/stories110M.sl:5-44,
 * examples/llama2/llama2_quant.sl:7-56, made shape-parametric: D4). */
typedef struct {
  int64_t dim, hidden, n_layers, n_heads, n_kv_heads, vocab, seq_len;
  float eps, theta;
  int64_t w4; /* 0: fp32 weights, 1: F6 W4 weights with group gs */
  int64_t gs;
} orc_llama_cfg;

/* Weights.  fp32 layout: wq[L,dim,dim], wk/wv[L,kv_dim,dim], wo[L,dim,dim],
 * w1/w3[L,hidden,dim], w2[L,dim,hidden], wcls[vocab,dim], emb[vocab,dim],
 * rms_att/rms_ffn[L,dim], rms_final[dim].  W4 layout: the same matrices as F6
 * packed bytes (q_*) plus scales (s_*), one matrix after another per layer. */
typedef struct {
  const float *emb, *rms_att, *rms_ffn, *rms_final;
  const float *wq, *wk, *wv, *wo, *w1, *w2, *w3, *wcls;
  const uint8_t *q_wq, *q_wk, *q_wv, *q_wo, *q_w1, *q_w2, *q_w3, *q_wcls;
  const float *s_wq, *s_wk, *s_wv, *s_wo, *s_w1, *s_w2, *s_w3, *s_wcls;
} orc_llama_weights;

/* One token of the decode step of stories110M.sl:44-247 with the GQA head map
 * of llama2_quant.sl:98 and score scale 1/sqrt(hs) (F11).  key_cache and
 * value_cache are [L, seq_len, kv_dim]; logits[vocab] is written.  Matrix-vector
 * products accumulate in double (exact reference for the tolerance check);
 * everything else is fp32 as in the program.  Pinned (tests/test_oracle_decode.py)
 * by a float64 brute force in another formulation (whole sequence with a causal
 * mask, RoPE as complex rotation) for MHA / GQA / MQA, closed forms (zero
 * projections, pos-0 independence of wq / wk / theta, wq = 0 gives the mean of
 * V), GQA = MHA with duplicated K/V heads, and W4 = fp32 on dequantized
 * matrices; planted mistakes (no RoPE, reversed RoPE, wrong head map, no score
 * scale) fail those pins. */
void orc_llama_forward(const orc_llama_cfg *cfg, const orc_llama_weights *w,
                       float *key_cache, float *value_cache, int64_t token,
                       int64_t pos, float *logits);

/* The CPU baseline of the same step (cpu_decode.c): fp32 throughout, OpenMP
 * GEMVs over output rows summed in 16 fp32 lanes, W4 dequantized per group
 * before the multiply-add.  For bench.py's cpu_baseline leg; checked against
 * orc_llama_forward to 1e-4 (tests/test_oracle_decode.py).  W4 needs gs a
 * multiple of 32 dividing dim and hidden (cpu_llama_supported). */
int cpu_llama_supported(const orc_llama_cfg *cfg);
void cpu_llama_forward(const orc_llama_cfg *cfg, const orc_llama_weights *w,
                       float *key_cache, float *value_cache, int64_t token,
                       int64_t pos, float *logits);

/* One token of llama2_quant_forward (examples/llama2/llama2_quant.sl:57-198):
 * the reference's W4 format F5 for the seven layer matrices (one flat nibble
 * array qw with scales/zeros per flat group of gs, per-matrix element offsets
 * wq_off.. advanced per layer by rows*cols as in :77-79,136,156-158), no RoPE,
 * score scale 1/sqrt(head_size), fp32 classifier wcls[vocab, dim].  Dims are
 * taken from cfg (the program hard-codes 1536/6144/128, deviation D4).
 * cfg->w4 / gs / theta are ignored; group size is `gs`.  Pinned
 * (tests/test_oracle_decode.py) by the float64 brute force without RoPE on the
 * matrices dequantized from the flat array at the per-layer offsets (gs 32 and
 * 128), and at pos 0 by orc_llama_forward on the same dequantized matrices. */
void orc_llama_quant_forward(const orc_llama_cfg *cfg, const float *emb, const float *rms_att,
                             const float *rms_ffn, const float *rms_final, const float *wcls,
                             const uint8_t *qw, const float *scales, const float *zeros,
                             int64_t gs, const int64_t off[7], float *key_cache,
                             float *value_cache, int64_t token, int64_t pos, float *logits);

/* One call of llama32_forward, the int8 LLaMA-3.2 program
 * examples/llama2/llama32_1b_int8_tensor.sl:16-305 (as bound by
 * examples/llama2/bench_llama32_1b_int8.cpp:36-61), statement by statement with
 * SimpLang's typing (float literals f32, integer literals i64,
 * src/mlir/mlir_codegen.cpp:305-390,608-625): x = (float)x_i8; per layer
 * rmsnorm, xb*127 clamped to [-128,127] and truncated to i8, Q/K/V =
 * tensor_matmul_nt (i8 x i8 -> i32), no RoPE (the program computes factors and
 * discards them, :123-140), K/V cached as (i8)(v / 256) (i64 division, integer
 * truncation), per head scores sum_d (float)Q * (float)k / 8 (fp32, in order),
 * softmax, attn_out = (i32) sum_t p * v, Wo on (i8)clamp(attn_out / 256), x +=
 * Wo / 65536, FFN rmsnorm, Gate/Up on the re-quantized xb (the program's xb_mat
 * views xb_i8), ffn_hb = (i8)(silu(g/65536) * (u/65536) * 127) with the x86
 * lowering of an out-of-range conversion (truncate to i32, keep the low byte;
 * NaN or beyond i32 gives 0), x += Down / 65536, final rmsnorm, fp32 classifier.
 * cfg: dim, hidden, n_layers, n_heads, n_kv_heads, vocab, seq_len (max_seq_len);
 * head_dim given separately (kv_dim = n_kv_heads * head_dim).  Every array of
 * the program is written as the program writes it.  Returns logits[0]. */
float orc_llama32_int8_forward(const orc_llama_cfg *cfg, int64_t head_dim, const int8_t *x_i8,
                               const float *rms_att, const float *rms_ffn,
                               const float *rms_final, const int8_t *wq, const int8_t *wk,
                               const int8_t *wv, const int8_t *wo, const int8_t *w1,
                               const int8_t *w2, const int8_t *w3, const float *wcls,
                               float *x, float *xb, float *logits, int8_t *xb_i8,
                               int8_t *k_cache, int8_t *v_cache, float *att_scores,
                               float *att_probs, int32_t *attn_out, int8_t *ffn_hb,
                               int64_t pos);

/* Strict-'>' argmax, first maximum wins (examples/llama2/generate_stories110M.cpp:73-83). */
int64_t orc_argmax(const float *logits, int64_t n);

/* Symmetric W4 quantization (the format above; no reference counterpart):
 * per row of cols, groups of gs: scale = max|w| / 7 (1 for an all-zero group),
 * q = clamp(round(w / scale), -8, 7), two's-complement nibbles, low = even k. */
void orc_quantize_w4s(const float *w, int64_t rows, int64_t cols, int64_t gs, uint8_t *qw,
                      float *scales);

/* MT19937 (Matsumoto & Nishimura 1998; the std::mt19937 of the C++ standard):
 * state of 624 words, seeded as std::mt19937(seed). */
typedef struct {
  uint32_t mt[624];
  int idx;
} orc_mt19937;
void orc_mt_seed(orc_mt19937 *g, uint32_t seed);
uint32_t orc_mt_next(orc_mt19937 *g);
/* std::uniform_real_distribution<float>(0, 1) on a 32-bit generator as
 * libstdc++ implements it (generate_canonical<float, 24>: one draw,
 * float(x) / 2^32, values >= 1 replaced by the largest float below 1). */
float orc_uniform01f(orc_mt19937 *g);
/* sample_temperature of examples/llama2/generate_stories110M.cpp:86-116 on a copy
 * of logits (argmax for temperature 0, :73-83), one draw from g. */
int64_t orc_sample(const float *logits, int64_t n, float temperature, orc_mt19937 *g);

#ifdef __cplusplus
}
#endif
#endif
