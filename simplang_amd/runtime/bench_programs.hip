// bench_programs.hip -- the reference's compiled int8 benchmark programs as
// exports with their symbol names and signatures, so the reference's own hosts
// can dlopen this library in place of the SimpLang-built object:
//   int32_t benchmark_int8_matmul_<N>(void), N in {32, 64, 128, 256, 384, 512,
//       768, 1024, 2048, 4096}: simptensor/benchmarks/bench_int8_matmul.sl:11-335,
//       looked up by bench_int8_matmul_runner.cpp:24,247.  Builds the
//       deterministic inputs val = ((i*N + j) % 127) - 64, A[i,j] = B[j,i] = val,
//       runs tensor_matmul (s8 x s8 -> i32) and returns the i32 wraparound sum
//       of C.  The programs have no error path; here an error returns 0 and
//       raises simp_rt_error_count() (message in simp_rt_last_error()).
//   int32_t kernel_main(void): the program's entry point,
//       bench_int8_matmul.sl:337-339, = benchmark_int8_matmul_256().
//   int32_t int8_chunk_<N>(i8[] A, i8[] B, i32[] C, i64 row_start), N in {256,
//       512, 768, 1024, 2048} with chunks of N/8 rows:
//       simptensor/benchmarks/bench_int8_matmul_parallel.sl:5-73, typedef and
//       lookup bench_int8_parallel_runner.cpp:13-16,122.  C rows [row_start,
//       row_start + N/8) = A rows [row_start, ...) x B, all N x N row-major.
//       Returns 0 as the program does, or a negative SIMP_RT_E* status.
// Both run on the device through the library's int8 GEMM; the benchmark
// programs keep their inputs in a per-stream workspace, so every call of one
// size after the first allocates nothing.
#include <algorithm>

#include "rt_internal.h"

namespace simp {
namespace {

__global__ void __launch_bounds__(256)
    recipe_inputs_k(int8_t *__restrict__ A, int8_t *__restrict__ B, int N) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)N * N) return;
  const int64_t i = idx / N, j = idx - i * N;
  const int8_t v = (int8_t)((idx % 127) - 64);  // ((i*N + j) % 127) - 64
  A[idx] = v;
  B[j * N + i] = v;
}

// out[0] += sum of C (unsigned 32-bit, i.e. i32 wraparound; integer adds in
// any order give the same bits).
__global__ void __launch_bounds__(256)
    checksum_i32_k(const int32_t *__restrict__ C, int64_t n, uint32_t *__restrict__ out) {
  uint32_t s = 0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    s += (uint32_t)C[i];
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  __shared__ uint32_t part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) atomicAdd(out, part[0] + part[1] + part[2] + part[3]);
}

__global__ void zero_u32_k(uint32_t *p) { *p = 0u; }

int bench_program(int N, int32_t *checksum) {
  hipStream_t st = cur_stream();
  const size_t nn = (size_t)N * N;
  // A [N,N] i8 | B [N,N] i8 | C [N,N] i32 | checksum; slot 2 is this file's
  void *ws = nullptr;
  int rc = workspace(st, 6 * nn + 256, &ws, 2);
  if (rc) return rc;
  int8_t *A = (int8_t *)ws, *B = A + nn;
  int32_t *C = (int32_t *)(B + nn);
  uint32_t *sum = (uint32_t *)(C + nn);
  hipLaunchKernelGGL(recipe_inputs_k, dim3((unsigned)cdiv((int64_t)nn, 256)), dim3(256), 0, st, A,
                     B, N);
  SIMP_HIP(hipGetLastError());
  rc = simp_rt_tensor_matmul_i8(A, A, 0, N, N, N, 1, B, B, 0, N, N, N, 1, C, C, 0, N, N, N, 1);
  if (rc) return rc;
  hipLaunchKernelGGL(zero_u32_k, dim3(1), dim3(1), 0, st, sum);
  const unsigned blocks = (unsigned)std::min<int64_t>(cdiv((int64_t)nn, 256 * 8), 2048);
  hipLaunchKernelGGL(checksum_i32_k, dim3(blocks), dim3(256), 0, st, (const int32_t *)C,
                     (int64_t)nn, sum);
  SIMP_HIP(hipGetLastError());
  uint32_t h = 0;
  SIMP_HIP(hipMemcpyAsync(&h, sum, 4, hipMemcpyDeviceToHost, st));
  SIMP_HIP(hipStreamSynchronize(st));
  *checksum = (int32_t)h;
  return SIMP_RT_OK;
}

int32_t chunk_program(const char *name, int64_t N, const int8_t *A, int64_t a_off, int64_t a_size,
                      int64_t a_stride, const int8_t *B, int64_t b_off, int64_t b_size,
                      int64_t b_stride, int32_t *C, int64_t c_off, int64_t c_size,
                      int64_t c_stride, int64_t row_start) {
  const int64_t rows = N / 8;
  int rc;
  if ((rc = check_desc1("A", A, a_off, a_size, a_stride)) ||
      (rc = check_desc1("B", B, b_off, b_size, b_stride)) ||
      (rc = check_desc1("C", C, c_off, c_size, c_stride)))
    return rc;
  if (row_start < 0 || row_start + rows > N)
    return set_error(SIMP_RT_EINVAL, "%s: row_start %lld outside [0, %lld]", name,
                     (long long)row_start, (long long)(N - rows));
  const int64_t end = (row_start + rows) * N;
  if (a_size < end || b_size < N * N || c_size < end)
    return set_error(SIMP_RT_EINVAL, "%s: arrays hold %lld / %lld / %lld elements, need %lld / "
                     "%lld / %lld", name, (long long)a_size, (long long)b_size,
                     (long long)c_size, (long long)end, (long long)(N * N), (long long)end);
  // A_local = tensor_from_array(A, row_start*N) as i8<rows, N>, B_local as i8<N, N>,
  // R = tensor_matmul(A_local, B_local) stored into C's rows
  return simp_rt_tensor_matmul_i8(A, A, a_off + row_start * N, rows, N, N, 1, B, B, b_off, N, N, N,
                                  1, C, C, c_off + row_start * N, rows, N, N, 1);
}

}  // namespace
}  // namespace simp

using namespace simp;

extern "C" {

#define SIMP_BENCH(N)                               \
  int32_t benchmark_int8_matmul_##N(void) {         \
    clear_error();                                  \
    int32_t sum = 0;                                \
    return bench_program(N, &sum) ? 0 : sum;        \
  }
SIMP_BENCH(32)
SIMP_BENCH(64)
SIMP_BENCH(128)
SIMP_BENCH(256)
SIMP_BENCH(384)
SIMP_BENCH(512)
SIMP_BENCH(768)
SIMP_BENCH(1024)
SIMP_BENCH(2048)
SIMP_BENCH(4096)
#undef SIMP_BENCH

// fn kernel_main() -> i32 { return benchmark_int8_matmul_256(); }
// (bench_int8_matmul.sl:337-339): the symbol the generic runner dlsyms
// (runtime/include/kernel_runner.hpp:39-56, runtime/src/host.cpp:158-193).
int32_t kernel_main(void) { return benchmark_int8_matmul_256(); }

#define SIMP_CHUNK(N)                                                                            \
  int32_t int8_chunk_##N(int8_t *A_alloc, int8_t *A, int64_t A_off, int64_t A_size,              \
                         int64_t A_stride, int8_t *B_alloc, int8_t *B, int64_t B_off,             \
                         int64_t B_size, int64_t B_stride, int32_t *C_alloc, int32_t *C,          \
                         int64_t C_off, int64_t C_size, int64_t C_stride, int64_t row_start) {    \
    (void)A_alloc; (void)B_alloc; (void)C_alloc;                                                 \
    clear_error();                                                                                \
    return chunk_program("int8_chunk_" #N, N, A, A_off, A_size, A_stride, B, B_off, B_size,       \
                         B_stride, C, C_off, C_size, C_stride, row_start);                       \
  }
SIMP_CHUNK(256)
SIMP_CHUNK(512)
SIMP_CHUNK(768)
SIMP_CHUNK(1024)
SIMP_CHUNK(2048)
#undef SIMP_CHUNK

}  // extern "C"
