// Exports functions of the reference's own VNNI test, compiled in place from
// /root/reference (the include path is given by oracle/Makefile).  Used only
// by tests/test_oracle.py to pin the oracle; never shipped, never on the GPU.
//   scalar_vpdpbusd_reference : simptensor/tests/test_vnni_correctness.cpp:28-42
#define main simp_ref_vnni_test_main
#include "test_vnni_correctness.cpp"
#undef main

extern "C" void ref_scalar_vpdpbusd(const uint8_t *a, const int8_t *b,
                                    const int32_t *acc, int32_t *out) {
  scalar_vpdpbusd_reference(a, b, acc, out);
}
extern "C" void ref_hw_vpdpbusd(const uint8_t *a, const int8_t *b,
                                const int32_t *acc, int32_t *out) {
  vnni_vpdpbusd(a, b, acc, out);
}
