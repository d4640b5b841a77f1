// Exports the reference's hand-written VNNI int8 GEMM, compiled in place from
// /root/reference (include path from oracle/Makefile).  Used only by
// tests/test_oracle.py to pin the oracle's int8 GEMM and the checksum recipe.
//   vnni_matmul_single_thread<N> : simptensor/benchmarks/bench_int8_matmul_multicore.cpp:39-89
//   scalar_matmul_int4<N>, packed_matmul_int4<N> :
//                                  simptensor/benchmarks/bench_int4_matmul_runner.cpp:34-150
#define main simp_ref_multicore_main
#define g_sink simp_ref_sink_gemm
#include "bench_int8_matmul_multicore.cpp"
#undef main

#define REF_GEMM(N)                                                          \
  extern "C" void ref_vnni_matmul_##N(const int8_t *A, const int8_t *B_T,    \
                                      int32_t *C) {                          \
    vnni_matmul_single_thread<N>(A, B_T, C);                                 \
  }
REF_GEMM(64)
REF_GEMM(128)
REF_GEMM(256)
REF_GEMM(512)
REF_GEMM(1024)
REF_GEMM(2048)
