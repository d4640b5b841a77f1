// Exports the reference's int4 GEMM checksums (signed nibble packing, F6's
// convention), compiled in place from /root/reference.  Test-only.
//   scalar_matmul_int4<N>, packed_matmul_int4<N> :
//       simptensor/benchmarks/bench_int4_matmul_runner.cpp:34-150
#define main simp_ref_int4_main
#define g_sink simp_ref_sink_int4
#include "bench_int4_matmul_runner.cpp"
#undef main

#define REF_I4(N)                                                             \
  extern "C" int32_t ref_scalar_int4_##N(void) { return scalar_matmul_int4<N>(); } \
  extern "C" int32_t ref_packed_int4_##N(void) { return packed_matmul_int4<N>(); }
REF_I4(32)
REF_I4(64)
REF_I4(128)
