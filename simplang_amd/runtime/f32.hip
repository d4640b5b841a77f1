// f32.hip -- fp32 matmul entry points.
//   matmul (array builtin)  C += A*B on 1-D arrays viewed as row-major matrices
//                           at element offsets (MatMulOpLowering,
//                           ConvertSimpToMemRef.cpp:1794-1920: linalg.matmul
//                           accumulates into the caller's buffer, F4)
//   tensor_matmul (f32)     C = A*B into a caller buffer (ConvertSimpToMemRef.cpp:3280-3284)
//   tensor_matmul_nt (f32)  C = A*B_T^T (naive float branch, :3445-3481)
//   tensor_matvecmul (f32)  the same product as tensor_matmul (:3632-3792, f32 loops :3763-3787)
// n == 1 (every LLaMA decode projection, stories110M.sl:77-83) is an HBM-bound
// GEMV: one wave per output row at a time, lanes along K with 16-byte loads, x
// held in registers for the whole kernel, the next row's loads in flight while
// the current row is reduced.  n > 1 runs an LDS-tiled fp32 GEMM.
#include <algorithm>

#include "rt_device.h"
#include "rt_internal.h"

namespace simp {
namespace {

// y[i] = beta*y[i] + sum_k A[i*lda + k] x[k]; J = float4 slots of x per lane (K <= 256*J).
template <int J>
__global__ void __launch_bounds__(256)
    gemv_f32(const float *__restrict__ A, int64_t lda, const float *__restrict__ x,
             float *__restrict__ y, int rows, int K, float beta) {
  const int lane = threadIdx.x & 63;
  const int nw = gridDim.x * 4;
  int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  float4 xv[J];
#pragma unroll
  for (int j = 0; j < J; j++) {
    const int k = 4 * lane + 256 * j;
    xv[j] = k < K ? *(const float4 *)(x + k) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float4 a[J];
  auto load = [&](int r, float4 (&v)[J]) {
    const float *p = A + (int64_t)r * lda;
#pragma unroll
    for (int j = 0; j < J; j++) {
      const int k = 4 * lane + 256 * j;
      v[j] = k < K ? *(const float4 *)(p + k) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  if (row < rows) load(row, a);
  for (; row < rows; row += nw) {
    float4 b[J];
    if (row + nw < rows) load(row + nw, b);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < J; j++) {
      s = fmaf(a[j].x, xv[j].x, s);
      s = fmaf(a[j].y, xv[j].y, s);
      s = fmaf(a[j].z, xv[j].z, s);
      s = fmaf(a[j].w, xv[j].w, s);
    }
    s = wave_sum(s);
    if (lane == 0) y[row] = beta != 0.f ? y[row] + s : s;
#pragma unroll
    for (int j = 0; j < J; j++) a[j] = b[j];
  }
}

// Scalar-load GEMV for misaligned / long rows (x read from global, L1-resident).
__global__ void __launch_bounds__(256)
    gemv_f32_any(const float *__restrict__ A, int64_t lda, const float *__restrict__ x,
                 float *__restrict__ y, int rows, int K, float beta) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float *p = A + (int64_t)row * lda;
  float s = 0.f;
  for (int k = lane; k < K; k += 64) s = fmaf(p[k], x[k], s);
  s = wave_sum(s);
  if (lane == 0) y[row] = beta != 0.f ? y[row] + s : s;
}

// C = beta*C + A*B, 64x64 tile per 256 threads, each thread a 4x4 block.
// BT: B is given transposed, B_T[N,K] (row n holds column n of B).
template <bool BT>
__global__ void __launch_bounds__(256)
    gemm_f32(const float *__restrict__ A, int64_t lda, const float *__restrict__ B, int64_t ldb,
             float *__restrict__ C, int64_t ldc, int M, int N, int K, float beta) {
  __shared__ float sa[16][64 + 1];
  __shared__ float sb[16][64 + 1];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
    for (int i = threadIdx.x; i < 16 * 64; i += 256) {
      const int kk = i & 15, mm = i >> 4;  // A tile, k fastest
      const int gm = m0 + mm, gk = k0 + kk;
      sa[kk][mm] = (gm < M && gk < K) ? A[(int64_t)gm * lda + gk] : 0.f;
      if constexpr (BT) {
        const int gn = n0 + mm;  // B_T tile, k fastest (rows of B_T are contiguous in k)
        sb[kk][mm] = (gn < N && gk < K) ? B[(int64_t)gn * ldb + gk] : 0.f;
      } else {
        const int nn = i & 63, kb = i >> 6;  // B tile, n fastest
        const int gn = n0 + nn, gk2 = k0 + kb;
        sb[kb][nn] = (gn < N && gk2 < K) ? B[(int64_t)gk2 * ldb + gn] : 0.f;
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; kk++) {
      float av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; i++) av[i] = sa[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; j++) bv[j] = sb[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int gm = m0 + ty * 4 + i, gn = n0 + tx * 4 + j;
      if (gm < M && gn < N) {
        float *c = C + (int64_t)gm * ldc + gn;
        *c = beta != 0.f ? *c + acc[i][j] : acc[i][j];
      }
    }
}

// y[0..rows) = beta*y + W x: W rows of lda floats, x and y contiguous.
int launch_gemv_f32(const float *W, int64_t lda, const float *x, float *y, int rows, int K,
                    float beta, hipStream_t st) {
  const bool vec = K % 4 == 0 && lda % 4 == 0 && ((uintptr_t)W & 15) == 0 &&
                   ((uintptr_t)x & 15) == 0;
  const int blocks_cap = num_cus() * 4;
  const unsigned grid = (unsigned)std::min<int64_t>(cdiv(rows, 4), blocks_cap);
  if (vec && K > 0 && K <= 256 * 16) {
    const int J = (int)cdiv(K, 256);
#define GEMV_CASE(JJ) \
  case JJ: hipLaunchKernelGGL(gemv_f32<JJ>, dim3(grid), dim3(256), 0, st, W, lda, x, y, rows, K, beta); break;
    switch (J) {
      GEMV_CASE(1) GEMV_CASE(2) GEMV_CASE(3) GEMV_CASE(4) GEMV_CASE(5) GEMV_CASE(6)
      GEMV_CASE(7) GEMV_CASE(8) GEMV_CASE(9) GEMV_CASE(10) GEMV_CASE(11) GEMV_CASE(12)
      GEMV_CASE(13) GEMV_CASE(14) GEMV_CASE(15) GEMV_CASE(16)
      default: break;
    }
#undef GEMV_CASE
  } else {
    hipLaunchKernelGGL(gemv_f32_any, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, st, W, lda, x, y,
                       rows, K, beta);
  }
  SIMP_HIP(hipGetLastError());
  return SIMP_RT_OK;
}

}  // namespace

int launch_matmul_f32(const float *A, int64_t lda, const float *B, int64_t ldb, float *C,
                      int64_t ldc, int M, int N, int K, float beta, hipStream_t st) {
  if (M == 0 || N == 0) return SIMP_RT_OK;
  // column vector operand (B[k*ldb], ldb == 1) and a contiguous C column: GEMV
  if (N == 1 && ldb == 1 && ldc == 1) return launch_gemv_f32(A, lda, B, C, M, K, beta, st);
  dim3 grid((unsigned)cdiv(N, 64), (unsigned)cdiv(M, 64));
  hipLaunchKernelGGL(gemm_f32<false>, grid, dim3(256), 0, st, A, lda, B, ldb, C, ldc, M, N, K, beta);
  SIMP_HIP(hipGetLastError());
  return SIMP_RT_OK;
}

namespace {
// C = A * B_T^T (fresh C): a single row of A against B_T[N,K] is a GEMV over the
// rows of B_T.
int launch_matmul_nt_f32(const float *A, int64_t lda, const float *BT, int64_t ldb, float *C,
                         int64_t ldc, int M, int N, int K, hipStream_t st) {
  if (M == 0 || N == 0) return SIMP_RT_OK;
  if (M == 1) return launch_gemv_f32(BT, ldb, A, C, N, K, 0.f, st);
  dim3 grid((unsigned)cdiv(N, 64), (unsigned)cdiv(M, 64));
  hipLaunchKernelGGL(gemm_f32<true>, grid, dim3(256), 0, st, A, lda, BT, ldb, C, ldc, M, N, K, 0.f);
  SIMP_HIP(hipGetLastError());
  return SIMP_RT_OK;
}
}  // namespace

}  // namespace simp

namespace simp {
namespace {
// Shared body of the rank-2 fp32 entry points: C[M,N] = A[M,K] x B (B[K,N], or
// B_T[N,K] when BT), C overwritten.
template <bool BT>
int tensor_f32_entry(const char *name, const float *a_alloc, const float *a, int64_t a_off,
                     int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
                     const float *b_alloc, const float *b, int64_t b_off, int64_t b_s0,
                     int64_t b_s1, int64_t b_st0, int64_t b_st1, float *c_alloc, float *c,
                     int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1) {
  (void)a_alloc; (void)b_alloc; (void)c_alloc;
  int rc;
  if ((rc = check_desc2("A", a, a_off, a_s0, a_s1, a_st0, a_st1))) return rc;
  if ((rc = check_desc2("B", b, b_off, b_s0, b_s1, b_st0, b_st1))) return rc;
  if ((rc = check_desc2("C", c, c_off, c_s0, c_s1, c_st0, c_st1))) return rc;
  const int64_t M = a_s0, K = a_s1, N = BT ? b_s0 : b_s1;
  const int64_t Kb = BT ? b_s1 : b_s0;
  if (Kb != K || c_s0 != M || c_s1 != N)
    return set_error(SIMP_RT_EINVAL, "%s: shape mismatch A[%lld,%lld] B%s[%lld,%lld] C[%lld,%lld]",
                     name, (long long)a_s0, (long long)a_s1, BT ? "_T" : "", (long long)b_s0,
                     (long long)b_s1, (long long)c_s0, (long long)c_s1);
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return set_error(SIMP_RT_EUNSUPPORTED, "%s: dimension above 2^31-1", name);
  if (M == 0 || N == 0) return SIMP_RT_OK;
  Operand oa, ob, oc;
  const size_t ab = K ? 4 * (size_t)((M - 1) * a_st0 + K) : 0;
  const size_t bb = (b_s0 && b_s1) ? 4 * (size_t)((b_s0 - 1) * b_st0 + b_s1) : 0;
  const size_t cb = 4 * (size_t)((M - 1) * c_st0 + N);
  if ((rc = oa.bind(a + a_off, ab, Operand::kIn, "A"))) return rc;
  if ((rc = ob.bind(b + b_off, bb, Operand::kIn, "B"))) return rc;
  if ((rc = oc.bind(c + c_off, cb, Operand::kOut, "C"))) return rc;
  if constexpr (BT)
    rc = launch_matmul_nt_f32((const float *)oa.dev(), a_st0, (const float *)ob.dev(), b_st0,
                              (float *)oc.dev(), c_st0, (int)M, (int)N, (int)K, cur_stream());
  else
    rc = launch_matmul_f32((const float *)oa.dev(), a_st0, (const float *)ob.dev(), b_st0,
                           (float *)oc.dev(), c_st0, (int)M, (int)N, (int)K, 0.f, cur_stream());
  if (rc) return rc;
  Operand *ops[] = {&oa, &ob, &oc};
  return finish(ops, 3);
}
}  // namespace
}  // namespace simp

using namespace simp;

extern "C" {

int32_t simp_rt_matmul_f32(const float *a_alloc, const float *lhs, int64_t a_doff, int64_t a_size,
                           int64_t a_stride, const float *b_alloc, const float *rhs,
                           int64_t b_doff, int64_t b_size, int64_t b_stride, float *c_alloc,
                           float *out, int64_t c_doff, int64_t c_size, int64_t c_stride, int64_t m,
                           int64_t k, int64_t n, int64_t lhs_offset, int64_t rhs_offset,
                           int64_t out_offset) {
  (void)a_alloc; (void)b_alloc; (void)c_alloc;
  int rc;
  if ((rc = check_desc1("lhs", lhs, a_doff, a_size, a_stride))) return rc;
  if ((rc = check_desc1("rhs", rhs, b_doff, b_size, b_stride))) return rc;
  if ((rc = check_desc1("output", out, c_doff, c_size, c_stride))) return rc;
  if (m < 0 || k < 0 || n < 0 || lhs_offset < 0 || rhs_offset < 0 || out_offset < 0 ||
      lhs_offset + m * k > a_size || rhs_offset + k * n > b_size || out_offset + m * n > c_size)
    return set_error(SIMP_RT_EINVAL, "matmul: m=%lld k=%lld n=%lld with offsets exceeds arrays",
                     (long long)m, (long long)k, (long long)n);
  if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX)
    return set_error(SIMP_RT_EUNSUPPORTED, "matmul: dimension above 2^31-1");
  if (m == 0 || n == 0) return SIMP_RT_OK;
  Operand oa, ob, oc;
  if ((rc = oa.bind(lhs + a_doff + lhs_offset, 4 * (size_t)(m * k), Operand::kIn, "lhs"))) return rc;
  if ((rc = ob.bind(rhs + b_doff + rhs_offset, 4 * (size_t)(k * n), Operand::kIn, "rhs"))) return rc;
  if ((rc = oc.bind(out + c_doff + out_offset, 4 * (size_t)(m * n), Operand::kInOut, "output"))) return rc;
  if ((rc = launch_matmul_f32((const float *)oa.dev(), k, (const float *)ob.dev(), n,
                              (float *)oc.dev(), n, (int)m, (int)n, (int)k, 1.f, cur_stream())))
    return rc;
  Operand *ops[] = {&oa, &ob, &oc};
  return finish(ops, 3);
}

int32_t simp_rt_tensor_matmul_f32(
    const float *a_alloc, const float *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const float *b_alloc, const float *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_st0, int64_t b_st1,
    float *c_alloc, float *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1) {
  return tensor_f32_entry<false>("tensor_matmul_f32", a_alloc, a, a_off, a_s0, a_s1, a_st0, a_st1,
                                 b_alloc, b, b_off, b_s0, b_s1, b_st0, b_st1, c_alloc, c, c_off,
                                 c_s0, c_s1, c_st0, c_st1);
}

int32_t simp_rt_tensor_matmul_nt_f32(
    const float *a_alloc, const float *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const float *bt_alloc, const float *bt, int64_t bt_off, int64_t bt_s0, int64_t bt_s1, int64_t bt_st0, int64_t bt_st1,
    float *c_alloc, float *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1) {
  return tensor_f32_entry<true>("tensor_matmul_nt_f32", a_alloc, a, a_off, a_s0, a_s1, a_st0,
                                a_st1, bt_alloc, bt, bt_off, bt_s0, bt_s1, bt_st0, bt_st1, c_alloc,
                                c, c_off, c_s0, c_s1, c_st0, c_st1);
}

int32_t simp_rt_tensor_matvecmul_f32(
    const float *a_alloc, const float *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const float *b_alloc, const float *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_st0, int64_t b_st1,
    float *c_alloc, float *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1) {
  return tensor_f32_entry<false>("tensor_matvecmul_f32", a_alloc, a, a_off, a_s0, a_s1, a_st0,
                                 a_st1, b_alloc, b, b_off, b_s0, b_s1, b_st0, b_st1, c_alloc, c,
                                 c_off, c_s0, c_s1, c_st0, c_st1);
}

}  // extern "C"
