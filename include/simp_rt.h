/*
 * simp_rt.h -- C ABI of libsimp_hip.so, the MI355X (gfx950) runtime for the
 * tensor ops SimpLang's MLIR backend lowers into.
 *
 * Argument convention (the reference's host ABI, F10 of the reference
 * programs: examples/llama2/bench_llama_quant.cpp:10-28,
 * simptensor/benchmarks/bench_int8_parallel_runner.cpp:13-16): every array
 * operand is an MLIR memref descriptor expanded into scalars,
 *   rank 1 (T[] arrays):       T* alloc, T* aligned, i64 offset, i64 size, i64 stride
 *   rank 2 (tensors):          T* alloc, T* aligned, i64 offset,
 *                              i64 size0, i64 size1, i64 stride0, i64 stride1
 *   rank 3 / rank 4:           the same with three / four sizes, then as many strides
 * Elements live at aligned + offset + i*stride0 + j*stride1 (+ ...) (row-major:
 * the innermost stride must be 1 and each outer stride must step over the
 * dimensions inside it).  `alloc` is carried for ABI fidelity and is not read.
 * Scalars follow in the operand order fixed by SimpLang's builtin parser
 * (src/mlir/mlir_codegen.cpp:1388-1531,2068-2292).
 *
 * Pointers may be device memory (used in place), host ranges registered with
 * simp_rt_register (their device mirror is used), or plain host memory
 * (staged through device memory; the call then blocks until the outputs are
 * back on the host).  With device / registered operands a call is
 * asynchronous on the calling thread's stream (simp_rt_set_stream).
 *
 * Every entry point returns 0 on success or a negative SIMP_RT_E* status and
 * leaves a message for simp_rt_last_error().  The reference ops have no
 * status (they are inlined loops, src/mlir/lowering/ConvertSimpToMemRef.cpp).
 */
#ifndef SIMP_RT_H
#define SIMP_RT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SIMP_RT_ABI_VERSION 1

#define SIMP_RT_OK 0
#define SIMP_RT_EINVAL (-1)      /* bad shape, stride, offset or null pointer */
#define SIMP_RT_EHIP (-2)        /* HIP runtime error */
#define SIMP_RT_ENOMEM (-3)      /* device allocation failed */
#define SIMP_RT_EUNSUPPORTED (-4)/* valid request this build does not handle */
#define SIMP_RT_ENODEV (-5)      /* no HIP device */

/* simp_rt_register flags */
#define SIMP_RT_REG_IMMUTABLE 1  /* weights: uploaded once, never an output */

/* ------------------------------------------------------------ runtime -- */
/* No reference counterpart: the reference runs in-process on the CPU.  The
 * loader it replaces is KernelRunner (runtime/include/kernel_runner.hpp:27-103). */
const char *simp_rt_last_error(void);
/* Number of errors raised on the calling thread so far.  The model-level exports
 * return a float (NaN on error, as the compiled programs have no status); a
 * caller compares this count before and after the call to tell an error from a
 * NaN the arithmetic produced.  Those exports also clear the message on entry. */
int64_t simp_rt_error_count(void);
int32_t simp_rt_version(void);
int32_t simp_rt_init(void);
int32_t simp_rt_set_stream(void *hip_stream); /* per calling thread; NULL = null stream */
void *simp_rt_get_stream(void);
int32_t simp_rt_sync(void);
int32_t simp_rt_register(const void *host_ptr, int64_t bytes, int32_t flags);
int32_t simp_rt_unregister(const void *host_ptr);
int32_t simp_rt_device_ptr(const void *host_ptr, void **dev_ptr);
int32_t simp_rt_sync_to_host(const void *host_ptr, int64_t bytes);
int32_t simp_rt_malloc(void **dev_ptr, int64_t bytes);
int32_t simp_rt_free(void *dev_ptr);
int32_t simp_rt_memcpy(void *dst, const void *src, int64_t bytes); /* any direction, blocking */
/* Per-kernel timing for profiling (no reference counterpart).  simp_rt_timing(1)
 * clears earlier records and brackets every later launch of the library's main
 * kernels with HIP events on its stream; simp_rt_timing(0) stops and clears.
 * simp_rt_timing_query waits for the recorded launches of one kernel (e.g.
 * "gemm_i8_nt16", "gemm_i8_mfma", "transpose_i8", "w4s_gemv") and returns their
 * summed duration and count.  Launches under stream capture are not recorded. */
int32_t simp_rt_timing(int32_t on);
int32_t simp_rt_timing_query(const char *kernel, double *total_ms, int64_t *launches);

/* --------------------------------------------------------------- int8 -- */

/* tensor_matmul on i8 tensors: C[M,N] = A[M,K] x B[K,N], s8 x s8 -> i32,
 * C overwritten.  Replaces TensorMatMulOpLowering's i8 branch
 * (src/mlir/lowering/ConvertSimpToMemRef.cpp:3136-3279, F1) together with the
 * VNNI rewrite of its K loop (src/mlir/passes/VNNIPass.cpp:597-999); the
 * caller-owned C follows TensorMatMulIntoOpLowering (:3490-3627). */
int32_t simp_rt_tensor_matmul_i8(
    const int8_t *a_alloc, const int8_t *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const int8_t *b_alloc, const int8_t *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_st0, int64_t b_st1,
    int32_t *c_alloc, int32_t *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1);

/* tensor_matmul_nt on i8: C[M,N] = A[M,K] x B_T[N,K]^T, s8 x s8 -> i32.
 * Replaces TensorMatMulNTOpLowering (ConvertSimpToMemRef.cpp:3373-3486). */
int32_t simp_rt_tensor_matmul_nt_i8(
    const int8_t *a_alloc, const int8_t *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const int8_t *bt_alloc, const int8_t *bt, int64_t bt_off, int64_t bt_s0, int64_t bt_s1, int64_t bt_st0, int64_t bt_st1,
    int32_t *c_alloc, int32_t *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1);

/* Raw vpdpbusd semantics, u8 x s8 -> i32: C[M,N] = A[M,K](u8) x B[K,N](s8).
 * Replaces the hand-written VNNI GEMMs the reference benchmarks against
 * (simptensor/benchmarks/bench_int8_matmul_runner.cpp:91-185, scalar
 * semantics simptensor/tests/test_vnni_correctness.cpp:28-42). */
int32_t simp_rt_matmul_u8s8_i32(
    const uint8_t *a_alloc, const uint8_t *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const int8_t *b_alloc, const int8_t *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_st0, int64_t b_st1,
    int32_t *c_alloc, int32_t *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1);

/* u8 x s8 -> i32 with B given transposed, B_T[N,K] (the layout the reference's
 * VNNI kernels read, bench_int8_matmul_multicore.cpp:39-89). */
int32_t simp_rt_matmul_nt_u8s8_i32(
    const uint8_t *a_alloc, const uint8_t *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const int8_t *bt_alloc, const int8_t *bt, int64_t bt_off, int64_t bt_s0, int64_t bt_s1, int64_t bt_st0, int64_t bt_st1,
    int32_t *c_alloc, int32_t *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1);

/* No counterpart in the reference: an allocation-free variant of
 * simp_rt_matmul_u8s8_i32 (same operands, same result bits) for callers that
 * cannot allocate device memory -- code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc.  It calls no hipMalloc / hipFree:
 * A, B and C must already be device memory (or inside simp_rt_register'd
 * ranges); host pointers are rejected (SIMP_RT_EINVAL).  Its kernels use a
 * static device array of 64 MiB + 64 KiB per GPU (held until the process ends)
 * where the large-tile path cannot read B in place (K % 64 != 0, or rows of B
 * not 16-byte aligned): B transposed (K*N bytes) and its column sums (4*N,
 * rounded up to 256).  Where it reads B in place the kernel forms the column
 * sums itself and the array is not used.  Larger requests (e.g. K*N above
 * 64 MiB with K % 64 != 0) are rejected with SIMP_RT_EINVAL.
 * All calls on one GPU share that array: calls that overlap on one GPU (other
 * streams or threads) race and must be ordered by the caller.  The device
 * address of each GPU's copy is looked up by simp_rt_init() or by the first
 * call on that device. */
int32_t simp_rt_matmul_u8s8_i32_noalloc(
    const uint8_t *a_alloc, const uint8_t *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const int8_t *b_alloc, const int8_t *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_st0, int64_t b_st1,
    int32_t *c_alloc, int32_t *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1);

/* tensor_matvecmul on i8 tensors: the same s8 x s8 -> i32 product as
 * simp_rt_tensor_matmul_i8 (A[M,K] x B[K,N], C overwritten).  Replaces
 * TensorMatVecMulOpLowering's int8 branch (ConvertSimpToMemRef.cpp:3632-3762),
 * whose B transpose for N < K is a layout choice made internally here too. */
int32_t simp_rt_tensor_matvecmul_i8(
    const int8_t *a_alloc, const int8_t *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const int8_t *b_alloc, const int8_t *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_st0, int64_t b_st1,
    int32_t *c_alloc, int32_t *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1);

/* tensor_matmul on packed i4 tensors: C[M,N] (i16) = A[M,K] x B[K,N], where A
 * is passed packed as int8 [M,(K+1)/2] (two signed nibbles per byte along K, low
 * nibble = even index) and B packed as int8 [K,(N+1)/2] along N.  Each C is the
 * i32 sum truncated to i16.  Replaces TensorMatMulOpLowering's packed-i4 branch
 * (src/mlir/lowering/ConvertSimpToMemRef.cpp:2953-3133) with the i4 memref
 * packing of its type converter (:48-66); C is caller-owned. */
int32_t simp_rt_tensor_matmul_i4(
    const int8_t *a_alloc, const int8_t *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const int8_t *b_alloc, const int8_t *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_st0, int64_t b_st1,
    int16_t *c_alloc, int16_t *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1);

/* ------------------------------------------- int8 benchmark programs -- */

/* The reference's compiled int8 benchmark programs, with their symbols and
 * signatures, so its own hosts can dlopen this library.
 *
 * benchmark_int8_matmul_<N>() replaces fn benchmark_int8_matmul_<N>() -> i32 of
 * simptensor/benchmarks/bench_int8_matmul.sl:11-335 (looked up by
 * bench_int8_matmul_runner.cpp:24,247): it builds val = ((i*N + j) % 127) - 64,
 * A[i,j] = B[j,i] = val, computes C = tensor_matmul(A, B) (s8 x s8 -> i32) and
 * returns the i32 wraparound sum of C.  The program has no error path; here an
 * error returns 0 and raises simp_rt_error_count(). */
int32_t benchmark_int8_matmul_32(void);
int32_t benchmark_int8_matmul_64(void);
int32_t benchmark_int8_matmul_128(void);
int32_t benchmark_int8_matmul_256(void);
int32_t benchmark_int8_matmul_384(void);
int32_t benchmark_int8_matmul_512(void);
int32_t benchmark_int8_matmul_768(void);
int32_t benchmark_int8_matmul_1024(void);
int32_t benchmark_int8_matmul_2048(void);
int32_t benchmark_int8_matmul_4096(void);

/* kernel_main() replaces fn kernel_main() -> i32 of
 * simptensor/benchmarks/bench_int8_matmul.sl:337-339, which returns
 * benchmark_int8_matmul_256(): the entry point the generic runner looks up
 * (runtime/include/kernel_runner.hpp:39-56, runtime/src/host.cpp:158-193).
 * The program returns i32; a host binds it as int32_t (*)(void). */
int32_t kernel_main(void);

/* int8_chunk_<N>(i8[] A, i8[] B, i32[] C, i64 row_start) replaces
 * fn int8_chunk_<N> of simptensor/benchmarks/bench_int8_matmul_parallel.sl:5-73
 * (typedef ChunkFunc, bench_int8_parallel_runner.cpp:13-16, looked up at :122):
 * C rows [row_start, row_start + N/8) = A rows [row_start, row_start + N/8) x B,
 * all N x N row-major in rank-1 arrays.  Returns 0, or a negative SIMP_RT_E*
 * status (the program always returns 0).  Safe to call from several host
 * threads on disjoint rows, as that runner does. */
#define SIMP_RT_INT8_CHUNK(N)                                                                   \
  int32_t int8_chunk_##N(int8_t *A_alloc, int8_t *A, int64_t A_off, int64_t A_size,             \
                         int64_t A_stride, int8_t *B_alloc, int8_t *B, int64_t B_off,            \
                         int64_t B_size, int64_t B_stride, int32_t *C_alloc, int32_t *C,         \
                         int64_t C_off, int64_t C_size, int64_t C_stride, int64_t row_start)
SIMP_RT_INT8_CHUNK(256);
SIMP_RT_INT8_CHUNK(512);
SIMP_RT_INT8_CHUNK(768);
SIMP_RT_INT8_CHUNK(1024);
SIMP_RT_INT8_CHUNK(2048);

/* ----------------------------------------------------------------- W4 -- */

/* matmul_quant(qweights, scales, zeros, input, output, rows, cols, group_size,
 * offset): output[i] = sum_k (q*scale + zero) * input[k] for the rows x cols
 * matrix whose weights start at element `offset` of the packed array
 * (unsigned nibbles, low nibble = even element; flat groups of group_size).
 * Replaces MatMulQuantOpLowering (src/mlir/lowering/ConvertSimpToMemRef.cpp:3853-4013),
 * operand order of src/mlir/mlir_codegen.cpp:1502-1531.  The scale/zero index
 * includes `offset` (the reference drops it, so every layer but the first
 * reads the wrong scales) and any group_size works (the reference requires 128). */
int32_t simp_rt_matmul_quant(
    const int8_t *qw_alloc, const int8_t *qw, int64_t qw_off, int64_t qw_size, int64_t qw_stride,
    const float *s_alloc, const float *s, int64_t s_off, int64_t s_size, int64_t s_stride,
    const float *z_alloc, const float *z, int64_t z_off, int64_t z_size, int64_t z_stride,
    const float *in_alloc, const float *in, int64_t in_off, int64_t in_size, int64_t in_stride,
    float *out_alloc, float *out, int64_t out_off, int64_t out_size, int64_t out_stride,
    int64_t rows, int64_t cols, int64_t group_size, int64_t offset);

/* dequant_w4(qweights, scales, zeros, idx, group_size) over a range:
 * out[i] = q(idx + i) * scales[(idx + i) / group_size] + zeros[(idx + i) / group_size]
 * for 0 <= i < count, q(e) the unsigned nibble of flat element e (low nibble =
 * even e), fp32 multiply then add, each rounded.  Replaces DequantW4OpLowering
 * (src/mlir/lowering/ConvertSimpToMemRef.cpp:2367-2429; builtin operands of
 * src/mlir/mlir_codegen.cpp:1482-1500, in that order, then the destination and
 * the element count).  The builtin is a scalar expression the program
 * evaluates per element inside its own loops; one device call per element
 * would cost a launch per weight, so the entry point takes a range. */
int32_t simp_rt_dequant_w4(
    const int8_t *qw_alloc, const int8_t *qw, int64_t qw_off, int64_t qw_size, int64_t qw_stride,
    const float *s_alloc, const float *s, int64_t s_off, int64_t s_size, int64_t s_stride,
    const float *z_alloc, const float *z, int64_t z_off, int64_t z_size, int64_t z_stride,
    int64_t idx, int64_t group_size, float *out_alloc, float *out, int64_t out_off,
    int64_t out_size, int64_t out_stride, int64_t count);

/* Symmetric W4 GEMV / skinny GEMM: out[M,N] = x[M,K] * W^T with W[N,K] packed
 * as signed nibbles in [-8,7] (low nibble = even k, rows of K/2 bytes) and one
 * fp32 scale per group of group_size along K (scales[N, K/group_size]).  The
 * signed-nibble convention is the reference's i4 tensor packing
 * (ConvertSimpToMemRef.cpp:48-66,3016-3037); it is the matmul_quant computation
 * with zero = -8*scale and u = q+8. */
int32_t simp_rt_matmul_w4s(
    const uint8_t *w_alloc, const uint8_t *w, int64_t w_off, int64_t w_s0, int64_t w_s1, int64_t w_st0, int64_t w_st1,
    const float *s_alloc, const float *s, int64_t s_off, int64_t s_s0, int64_t s_s1, int64_t s_st0, int64_t s_st1,
    const float *x_alloc, const float *x, int64_t x_off, int64_t x_s0, int64_t x_s1, int64_t x_st0, int64_t x_st1,
    float *o_alloc, float *o, int64_t o_off, int64_t o_s0, int64_t o_s1, int64_t o_st0, int64_t o_st1,
    int64_t group_size);

/* --------------------------------------------------------------- fp32 -- */

/* matmul(lhs, rhs, output, m, k, n, lhs_offset, rhs_offset, output_offset):
 * output[m,n] += lhs[m,k] * rhs[k,n] on 1-D arrays viewed as row-major
 * matrices at the given element offsets; the caller zeroes output first when
 * it wants a plain product.  Replaces MatMulOpLowering
 * (src/mlir/lowering/ConvertSimpToMemRef.cpp:1794-1920), operand order of
 * src/mlir/mlir_codegen.cpp:1388-1412. */
int32_t simp_rt_matmul_f32(
    const float *lhs_alloc, const float *lhs, int64_t lhs_doff, int64_t lhs_size, int64_t lhs_stride,
    const float *rhs_alloc, const float *rhs, int64_t rhs_doff, int64_t rhs_size, int64_t rhs_stride,
    float *out_alloc, float *out, int64_t out_doff, int64_t out_size, int64_t out_stride,
    int64_t m, int64_t k, int64_t n, int64_t lhs_offset, int64_t rhs_offset, int64_t output_offset);

/* tensor_matmul on f32 tensors: C[M,N] = A[M,K] * B[K,N] into a caller buffer.
 * Replaces the f32 branch of TensorMatMulOpLowering (ConvertSimpToMemRef.cpp:3280-3284). */
int32_t simp_rt_tensor_matmul_f32(
    const float *a_alloc, const float *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const float *b_alloc, const float *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_st0, int64_t b_st1,
    float *c_alloc, float *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1);

/* tensor_matmul_nt on f32: C[M,N] = A[M,K] x B_T[N,K]^T, C overwritten.
 * Replaces the float branch of TensorMatMulNTOpLowering (ConvertSimpToMemRef.cpp:
 * 3445-3481).  M == 1 runs as a GEMV over the rows of B_T. */
int32_t simp_rt_tensor_matmul_nt_f32(
    const float *a_alloc, const float *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const float *bt_alloc, const float *bt, int64_t bt_off, int64_t bt_s0, int64_t bt_s1, int64_t bt_st0, int64_t bt_st1,
    float *c_alloc, float *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1);

/* tensor_matvecmul on f32: the same product as simp_rt_tensor_matmul_f32.
 * Replaces TensorMatVecMulOpLowering's float loops (ConvertSimpToMemRef.cpp:3763-3787). */
int32_t simp_rt_tensor_matvecmul_f32(
    const float *a_alloc, const float *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const float *b_alloc, const float *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_st0, int64_t b_st1,
    float *c_alloc, float *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1);

/* tensor_matmul on f64 tensors: C[M,N] = A[M,K] * B[K,N], C overwritten.
 * Replaces the general linalg.matmul branch for f64 (ConvertSimpToMemRef.cpp:
 * 3280-3284; tests/test_tensor_matmul.sl uses f64 tensors). */
int32_t simp_rt_tensor_matmul_f64(
    const double *a_alloc, const double *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const double *b_alloc, const double *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_st0, int64_t b_st1,
    double *c_alloc, double *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1);

/* tensor_matmul on rank-3 tensors: C[b] = A[b] x B[b] for A[Bt,M,K], B[Bt,K,N],
 * C[Bt,M,N], C overwritten.  Replaces the 3-D linalg.batch_matmul case of
 * TensorMatMulOpLowering (ConvertSimpToMemRef.cpp:3286-3291, into the result the
 * lowering zero-fills at :2926-2933).  _i8 is s8 x s8 -> i32 (linalg sign-extends). */
int32_t simp_rt_tensor_batch_matmul_f32(
    const float *a_alloc, const float *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_s2,
    int64_t a_st0, int64_t a_st1, int64_t a_st2,
    const float *b_alloc, const float *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_s2,
    int64_t b_st0, int64_t b_st1, int64_t b_st2,
    float *c_alloc, float *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_s2,
    int64_t c_st0, int64_t c_st1, int64_t c_st2);
int32_t simp_rt_tensor_batch_matmul_f64(
    const double *a_alloc, const double *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_s2,
    int64_t a_st0, int64_t a_st1, int64_t a_st2,
    const double *b_alloc, const double *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_s2,
    int64_t b_st0, int64_t b_st1, int64_t b_st2,
    double *c_alloc, double *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_s2,
    int64_t c_st0, int64_t c_st1, int64_t c_st2);
int32_t simp_rt_tensor_batch_matmul_i8(
    const int8_t *a_alloc, const int8_t *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_s2,
    int64_t a_st0, int64_t a_st1, int64_t a_st2,
    const int8_t *b_alloc, const int8_t *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_s2,
    int64_t b_st0, int64_t b_st1, int64_t b_st2,
    int32_t *c_alloc, int32_t *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_s2,
    int64_t c_st0, int64_t c_st1, int64_t c_st2);

/* tensor_matmul of an NHWC tensor by a [C_out, C_in] weight matrix (a fully
 * connected layer): out[n,h,w,o] = sum_i in[n,h,w,i] * weights[o,i].  Replaces
 * the 4-D x 2-D case of TensorMatMulOpLowering (ConvertSimpToMemRef.cpp:
 * 3293-3361: collapse (N,H,W), multiply by the transposed weights, expand).
 * (N,H,W) of input and output must collapse into one run of rows. */
int32_t simp_rt_tensor_matmul_nhwc_f32(
    const float *x_alloc, const float *x, int64_t x_off, int64_t x_s0, int64_t x_s1, int64_t x_s2,
    int64_t x_s3, int64_t x_st0, int64_t x_st1, int64_t x_st2, int64_t x_st3,
    const float *w_alloc, const float *w, int64_t w_off, int64_t w_s0, int64_t w_s1, int64_t w_st0,
    int64_t w_st1,
    float *y_alloc, float *y, int64_t y_off, int64_t y_s0, int64_t y_s1, int64_t y_s2,
    int64_t y_s3, int64_t y_st0, int64_t y_st1, int64_t y_st2, int64_t y_st3);
int32_t simp_rt_tensor_matmul_nhwc_f64(
    const double *x_alloc, const double *x, int64_t x_off, int64_t x_s0, int64_t x_s1, int64_t x_s2,
    int64_t x_s3, int64_t x_st0, int64_t x_st1, int64_t x_st2, int64_t x_st3,
    const double *w_alloc, const double *w, int64_t w_off, int64_t w_s0, int64_t w_s1, int64_t w_st0,
    int64_t w_st1,
    double *y_alloc, double *y, int64_t y_off, int64_t y_s0, int64_t y_s1, int64_t y_s2,
    int64_t y_s3, int64_t y_st0, int64_t y_st1, int64_t y_st2, int64_t y_st3);

/* ------------------------------------------------------ normalisations -- */

/* rmsnorm(input, weight, output, size, epsilon, weight_offset):
 * out[i] = (in[i] / sqrt(sum(in^2)/size + eps)) * weight[weight_offset + i].
 * Replaces RMSNormOpLowering (ConvertSimpToMemRef.cpp:2157-2236); epsilon is
 * the op's AnyFloat operand, narrowed to f32 as the lowering does. */
int32_t simp_rt_rmsnorm(
    const float *in_alloc, const float *in, int64_t in_off, int64_t in_size, int64_t in_stride,
    const float *w_alloc, const float *w, int64_t w_off, int64_t w_size, int64_t w_stride,
    float *out_alloc, float *out, int64_t out_off, int64_t out_size, int64_t out_stride,
    int64_t size, double epsilon, int64_t weight_offset);

/* softmax(input, output, size, input_offset, output_offset) over
 * in[input_offset .. +size) into out[output_offset .. +size).
 * Replaces SoftmaxOpLowering (ConvertSimpToMemRef.cpp:2239-2322). */
int32_t simp_rt_softmax(
    const float *in_alloc, const float *in, int64_t in_off, int64_t in_size, int64_t in_stride,
    float *out_alloc, float *out, int64_t out_off, int64_t out_size, int64_t out_stride,
    int64_t size, int64_t input_offset, int64_t output_offset);

/* silu(input, output, size): out = x / (1 + exp(-x)).
 * Replaces SiLUOpLowering (ConvertSimpToMemRef.cpp:2325-2360). */
int32_t simp_rt_silu(
    const float *in_alloc, const float *in, int64_t in_off, int64_t in_size, int64_t in_stride,
    float *out_alloc, float *out, int64_t out_off, int64_t out_size, int64_t out_stride,
    int64_t size);

/* SwiGLU gate: out = silu(gate) * up, the silu call plus the elementwise
 * product loop of examples/llama2/stories110M.sl:200-212 in one pass. */
int32_t simp_rt_swiglu(
    const float *g_alloc, const float *gate, int64_t g_off, int64_t g_size, int64_t g_stride,
    const float *u_alloc, const float *up, int64_t u_off, int64_t u_size, int64_t u_stride,
    float *o_alloc, float *out, int64_t o_off, int64_t o_size, int64_t o_stride,
    int64_t size);

/* RoPE in place on q[dim] and k[kv_dim] at position pos: for even i,
 * f = theta^-((i % head_size)/head_size), rotate (x[i], x[i+1]) by pos*f; k
 * only for i < kv_dim.  The scalar loop of examples/llama2/stories110M.sl:86-112. */
int32_t simp_rt_rope(
    float *q_alloc, float *q, int64_t q_off, int64_t q_size, int64_t q_stride,
    float *k_alloc, float *k, int64_t k_off, int64_t k_size, int64_t k_stride,
    int64_t dim, int64_t kv_dim, int64_t head_size, int64_t pos, double theta);

/* ------------------------------------------------------- decode step -- */

#define SIMP_RT_W_F32 0 /* fp32 weight matrices */
#define SIMP_RT_W_W4S 1 /* symmetric W4 (simp_rt_matmul_w4s format) */

/* Shape of the LLaMA programs examples/llama2/stories110M.sl:5-44 and
 * examples/llama2/llama2_quant.sl:7-56 (their hyperparameter arguments),
 * plus the weight format. */
typedef struct {
  int64_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len;
  float eps;        /* RMSNorm epsilon (the programs pass 1e-5) */
  float rope_theta; /* 10000 in the programs */
  int32_t weight_format;
  int32_t group_size; /* W4S: weights per scale along K */
} simp_rt_llama_config;

/* Weights, laid out as the arrays of stories110M_forward: token_embedding
 * [vocab,dim], rms_att/rms_ffn [n_layers,dim], rms_final [dim], and per
 * layer wq/wo [dim,dim], wk/wv [kv_dim,dim], w1/w3 [hidden,dim], w2
 * [dim,hidden], one layer after another, wcls [vocab,dim].  SIMP_RT_W_F32
 * uses the fp32 pointers; SIMP_RT_W_W4S the packed q_* ([rows, cols/2] per
 * layer) and scales s_* ([rows, cols/group_size] per layer).  All must be
 * device memory or registered ranges. */
typedef struct {
  const float *token_embedding, *rms_att, *rms_ffn, *rms_final;
  const float *wq, *wk, *wv, *wo, *w1, *w2, *w3, *wcls;
  const uint8_t *q_wq, *q_wk, *q_wv, *q_wo, *q_w1, *q_w2, *q_w3, *q_wcls;
  const float *s_wq, *s_wk, *s_wv, *s_wo, *s_w1, *s_w2, *s_w3, *s_wcls;
} simp_rt_llama_weights;

typedef struct simp_rt_llama simp_rt_llama;

/* A decode-step engine over the given weights, with its own activations and
 * fp32 KV cache [n_layers, seq_len, kv_dim] in device memory.  The step is the
 * single-token forward of stories110M_forward (stories110M.sl:44-247; W4:
 * llama2_quant_forward, llama2_quant.sl:57-198), fused into 5 kernels per layer. */
int32_t simp_rt_llama_create(const simp_rt_llama_config *cfg, const simp_rt_llama_weights *w,
                             simp_rt_llama **model);
int32_t simp_rt_llama_destroy(simp_rt_llama *model);
/* One step at (token, pos); logits[vocab] (device or host) receives the output.
 * Blocks until done.  Replaces one call of stories110M_forward as driven by
 * examples/llama2/generate_stories110M.cpp:236-257. */
int32_t simp_rt_llama_forward(simp_rt_llama *model, int64_t token, int64_t pos, float *logits);
/* Greedy generation (strict-'>' argmax, generate_stories110M.cpp:73-83): runs
 * the prompt then n_new sampled tokens; out_tokens[n_prompt + n_new] (host)
 * receives prompt and samples.  use_graph != 0 replays one captured HIP graph
 * per step with the token/position state kept on the device. */
int32_t simp_rt_llama_generate(simp_rt_llama *model, const int32_t *prompt, int64_t n_prompt,
                               int64_t n_new, int32_t *out_tokens, int32_t use_graph);

/* ------------------------------------------------ model-level exports -- */
/* The compiled program's entry point, byte-identical signature: every f32[]
 * argument is a rank-1 memref descriptor (alloc, aligned, offset, size, stride),
 * followed by the nine i64 hyperparameters; one token per call, logits written,
 * logits[0] returned.  Replaces stories110M_forward
 * (examples/llama2/stories110M.sl:5-44) as bound by
 * examples/llama2/generate_stories110M.cpp:15-21,136,236-257, so an unmodified
 * host can dlopen this library instead of the compiled .so.
 * Weights may be device memory (used in place) or host memory (mirrored once
 * on the device as immutable and assumed unchanged afterwards).  The KV cache
 * is kept on the device; each call copies the K and V rows at pos back into
 * key_cache / value_cache.  The scratch activation arrays (x ... att_soft) are
 * left untouched.  On error the return is NaN and simp_rt_last_error() says why. */
#define SIMP_RT_DESC_F32(n) float *n##_alloc, float *n, int64_t n##_off, int64_t n##_size, int64_t n##_stride
float stories110M_forward(
    SIMP_RT_DESC_F32(token_embedding_table), SIMP_RT_DESC_F32(rms_att_w), SIMP_RT_DESC_F32(wq),
    SIMP_RT_DESC_F32(wk), SIMP_RT_DESC_F32(wv), SIMP_RT_DESC_F32(wo), SIMP_RT_DESC_F32(rms_ffn_w),
    SIMP_RT_DESC_F32(w1), SIMP_RT_DESC_F32(w2), SIMP_RT_DESC_F32(w3), SIMP_RT_DESC_F32(rms_final_w),
    SIMP_RT_DESC_F32(wcls), SIMP_RT_DESC_F32(x), SIMP_RT_DESC_F32(xb), SIMP_RT_DESC_F32(xb2),
    SIMP_RT_DESC_F32(hb), SIMP_RT_DESC_F32(hb_silu), SIMP_RT_DESC_F32(q), SIMP_RT_DESC_F32(k),
    SIMP_RT_DESC_F32(v), SIMP_RT_DESC_F32(att), SIMP_RT_DESC_F32(att_soft), SIMP_RT_DESC_F32(logits),
    SIMP_RT_DESC_F32(key_cache), SIMP_RT_DESC_F32(value_cache), int64_t token, int64_t pos,
    int64_t dim, int64_t hidden_dim, int64_t n_layers, int64_t n_heads, int64_t n_kv_heads,
    int64_t vocab_size, int64_t seq_len);
/* The reference W4 program's entry point, byte-identical signature (f32[] and
 * i8[] rank-1 descriptors, then token, pos, seven dims incl. group_size, and the
 * seven element offsets of wq..w3 in qweights).  Replaces llama2_quant_forward
 * (examples/llama2/llama2_quant.sl:7-56) as bound by
 * examples/llama2/bench_llama_quant.cpp:15-24,320.  The layer matrices are in
 * the reference W4 format (u4 + scale/zero per flat group, matmul_quant
 * semantics with the offset-aware group index), the classifier is fp32 and no
 * RoPE is applied, as in the program; dims come from the arguments.  Weights,
 * KV cache, scratch arrays and errors are handled as for stories110M_forward. */
#define SIMP_RT_DESC_I8(n) int8_t *n##_alloc, int8_t *n, int64_t n##_off, int64_t n##_size, int64_t n##_stride
float llama2_quant_forward(
    SIMP_RT_DESC_F32(token_emb), SIMP_RT_DESC_F32(rms_att_w), SIMP_RT_DESC_F32(rms_ffn_w),
    SIMP_RT_DESC_F32(rms_final_w), SIMP_RT_DESC_F32(wcls), SIMP_RT_DESC_I8(qweights),
    SIMP_RT_DESC_F32(scales), SIMP_RT_DESC_F32(zeros), SIMP_RT_DESC_F32(x), SIMP_RT_DESC_F32(xb),
    SIMP_RT_DESC_F32(xb2), SIMP_RT_DESC_F32(q), SIMP_RT_DESC_F32(k), SIMP_RT_DESC_F32(v),
    SIMP_RT_DESC_F32(att), SIMP_RT_DESC_F32(att_soft), SIMP_RT_DESC_F32(hb),
    SIMP_RT_DESC_F32(hb_silu), SIMP_RT_DESC_F32(hb2), SIMP_RT_DESC_F32(logits),
    SIMP_RT_DESC_F32(key_cache), SIMP_RT_DESC_F32(value_cache), int64_t token, int64_t pos,
    int64_t dim, int64_t hidden_dim, int64_t n_layers, int64_t n_heads, int64_t n_kv_heads,
    int64_t vocab_size, int64_t seq_len, int64_t group_size, int64_t wq_off, int64_t wk_off,
    int64_t wv_off, int64_t wo_off, int64_t w1_off, int64_t w2_off, int64_t w3_off);
/* The int8 LLaMA-3.2 program's entry point, byte-identical signature (i8[], f32[]
 * and i32[] rank-1 descriptors, then pos and the eight i64 dims).  Replaces
 * llama32_forward (examples/llama2/llama32_1b_int8_tensor.sl:16-305) as bound by
 * examples/llama2/bench_llama32_1b_int8.cpp:36-61,124.  The program's
 * arithmetic: int8 weights pre-transposed for tensor_matmul_nt, activations
 * quantized as xb*127 clamped and truncated, int8 KV cache of (i32 / 256),
 * fixed-point rescales by 1/256 and 1/65536, fp32 norms, softmax and classifier;
 * the program's RoPE loop discards its results and is not run.  Dims come from
 * the arguments (the program hard-codes 2048/512/8192, deviation D4); dim and
 * hidden_dim and head_dim must be multiples of 16 and the int8 weights
 * 16-byte aligned.
 * The KV cache is kept on the device and the rows at pos are copied back into
 * k_cache / v_cache; logits, x_fp32, xb_fp32 and attn_out (the last layer's,
 * as the program leaves it; its int32 truncation of an fp32 sum may differ by 1
 * where the summation order moves the sum across an integer) are written;
 * xb_i8, att_scores, att_probs and ffn_hb are left untouched.  Weights and
 * errors as for stories110M_forward. */
#define SIMP_RT_DESC_I32(n) int32_t *n##_alloc, int32_t *n, int64_t n##_off, int64_t n##_size, int64_t n##_stride
float llama32_forward(
    SIMP_RT_DESC_I8(x_i8), SIMP_RT_DESC_F32(rms_att_w), SIMP_RT_DESC_F32(rms_ffn_w),
    SIMP_RT_DESC_F32(rms_final_w), SIMP_RT_DESC_I8(wq_t), SIMP_RT_DESC_I8(wk_t),
    SIMP_RT_DESC_I8(wv_t), SIMP_RT_DESC_I8(wo_t), SIMP_RT_DESC_I8(w1_t), SIMP_RT_DESC_I8(w2_t),
    SIMP_RT_DESC_I8(w3_t), SIMP_RT_DESC_F32(wcls), SIMP_RT_DESC_F32(x_fp32),
    SIMP_RT_DESC_F32(xb_fp32), SIMP_RT_DESC_F32(logits), SIMP_RT_DESC_I8(xb_i8),
    SIMP_RT_DESC_I8(k_cache), SIMP_RT_DESC_I8(v_cache), SIMP_RT_DESC_F32(att_scores),
    SIMP_RT_DESC_F32(att_probs), SIMP_RT_DESC_I32(attn_out), SIMP_RT_DESC_I8(ffn_hb), int64_t pos,
    int64_t dim, int64_t hidden_dim, int64_t n_layers, int64_t n_heads, int64_t n_kv_heads,
    int64_t vocab_size, int64_t max_seq_len, int64_t head_dim);
/* Frees the engines and device mirrors the model-level exports created (no
 * reference counterpart). */
int32_t simp_rt_forward_cache_clear(void);
/* How the model-level exports notice edits of weight arrays held in host
 * memory (no reference counterpart: the compiled programs read every weight on
 * every call).  0 (default): a call that starts a sequence re-hashes every
 * 64 KiB chunk, any other call one chunk per array in rotation, and a changed
 * chunk re-checks its whole array, so an edit confined to chunks not sampled
 * can go unseen until the rotation reaches them or the next sequence start.
 * 1: every call re-hashes every chunk (the reference's semantics, at the cost
 * of hashing all host weights per call: about 14 ms for 706 MB).  Device-
 * resident and simp_rt_register'd weights are used in place either way. */
int32_t simp_rt_export_verify_all(int32_t on);

/* ------------------------------------------------------- model files -- */
/* llama2.c checkpoint header, as read by
 * examples/llama2/generate_stories110M.cpp:25-33,143-150 (vocab_size < 0: the
 * classifier is stored after the other tensors instead of sharing the
 * embedding table). */
typedef struct {
  int32_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len;
} simp_rt_ckpt_config;
int32_t simp_rt_ckpt_read_config(const char *path, simp_rt_ckpt_config *cfg);
/* Reads the whole fp32 checkpoint (generate_stories110M.cpp:150-191, in the
 * llama2.c layout: wk/wv of kv_dim rows, legacy RoPE tables skipped before an
 * unshared classifier) into one device allocation *blob (free it with
 * simp_rt_free) and points w's fp32 fields into it, ready for
 * simp_rt_llama_create with SIMP_RT_W_F32. */
int32_t simp_rt_ckpt_load_f32(const char *path, simp_rt_ckpt_config *cfg, simp_rt_llama_weights *w,
                              void **blob);

/* Tokenizer file of generate_stories110M.cpp:36-70: max_token_length, then per
 * token a float score, an int32 length and the bytes. */
typedef struct simp_rt_tokenizer simp_rt_tokenizer;
int32_t simp_rt_tokenizer_load(const char *path, int32_t vocab_size, simp_rt_tokenizer **tok);
/* Tokenizer::decode (generate_stories110M.cpp:64-69): the token's bytes (not
 * NUL-terminated; *len receives the length), "?" when out of range. */
const char *simp_rt_tokenizer_decode(const simp_rt_tokenizer *tok, int32_t token, int32_t *len);
float simp_rt_tokenizer_score(const simp_rt_tokenizer *tok, int32_t token);
int32_t simp_rt_tokenizer_max_token_length(const simp_rt_tokenizer *tok);
int32_t simp_rt_tokenizer_free(simp_rt_tokenizer *tok);

/* Token sampling of generate_stories110M.cpp:73-116 on host logits: temperature
 * 0 is sample_argmax (strict '>' from index 0); otherwise sample_temperature
 * with a std::mt19937 seeded here (the reference seeds it from
 * std::random_device).  Returns the token, or a negative status. */
typedef struct simp_rt_sampler simp_rt_sampler;
int32_t simp_rt_sampler_create(uint32_t seed, simp_rt_sampler **s);
int32_t simp_rt_sampler_sample(simp_rt_sampler *s, const float *logits, int32_t n, float temperature);
int32_t simp_rt_sampler_free(simp_rt_sampler *s);

/* W4 quantizers on the GPU (device arrays, asynchronous on the thread's stream).
 * _w4u: the reference's quantize_w4 (examples/llama2/bench_llama_quant.cpp:51-93)
 * over one tensor of n floats: flat groups of group_size (even), q[(n+1)/2]
 * bytes (low nibble = even index), scales/zeros[ceil(n/group_size)].
 * _w4s: the symmetric format of simp_rt_matmul_w4s, per row of cols (a multiple
 * of group_size): scale = max|w|/7 (1 for an all-zero group),
 * q = clamp(round(w/scale), -8, 7); no reference counterpart. */
int32_t simp_rt_quantize_w4u(const float *w, int64_t n, int32_t group_size, uint8_t *q, float *scales,
                             float *zeros);
int32_t simp_rt_quantize_w4s(const float *w, int64_t rows, int64_t cols, int32_t group_size, uint8_t *q,
                             float *scales);

/* Packed W4 model files written from a llama2.c checkpoint (offline
 * quantization; no reference counterpart: the reference quantizes in memory at
 * start-up, bench_llama_quant.cpp:189-210).  A 64-byte header (magic, the
 * llama2.c config, group size), then 256-byte-aligned sections.
 *   "SIMPW4S1" (_w4s_): fp32 embedding and norms, then q and scales of wq, wk,
 *     wv, wo, w1, w2, w3 and the classifier; _w4s_file_load points the fields
 *     of a simp_rt_llama_weights, format SIMP_RT_W_W4S, into one device
 *     allocation.
 *   "SIMPW4U1" (_w4u_): the arrays of llama2_quant_forward: seven element
 *     offsets, fp32 embedding, norms and classifier, then qweights, scales and
 *     zeros of wq..w3 quantized tensor by tensor as the reference does. */
int32_t simp_rt_w4s_file_write(const char *ckpt_path, const char *out_path, int32_t group_size);
int32_t simp_rt_w4s_file_load(const char *path, simp_rt_llama_config *cfg, simp_rt_llama_weights *w,
                              void **blob);
typedef struct {
  const float *token_embedding, *rms_att, *rms_ffn, *rms_final, *wcls, *scales, *zeros;
  const int8_t *qweights;
  int64_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len, group_size;
  int64_t qweights_bytes, n_groups;
  int64_t offsets[7]; /* wq_off .. w3_off of llama2_quant_forward */
} simp_rt_w4u_model;
int32_t simp_rt_w4u_file_write(const char *ckpt_path, const char *out_path, int32_t group_size);
int32_t simp_rt_w4u_file_load(const char *path, simp_rt_w4u_model *m, void **blob);

#ifdef __cplusplus
}
#endif
#endif /* SIMP_RT_H */
