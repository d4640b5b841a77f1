// rt_internal.h -- shared host-side plumbing of libsimp_hip.so (not installed).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "simp_rt.h"

namespace simp {

// Thread-local error text behind simp_rt_last_error().
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Empties the message (the model-level exports call it first: their NaN return
// cannot carry a status, so an old message must not be read as theirs).
void clear_error();
int hip_fail(hipError_t e, const char *what);

#define SIMP_HIP(call)                                         \
  do {                                                         \
    hipError_t _e = (call);                                    \
    if (_e != hipSuccess) return ::simp::hip_fail(_e, #call);  \
  } while (0)

// Stream the calling thread launches on (simp_rt_set_stream, default null stream).
hipStream_t cur_stream();

// Device of the calling thread, initialised once per device on first use.
int ensure_device();

// A caller pointer made usable by a kernel.  Device memory (hipMalloc'd,
// managed) is used as-is; a host range inside a simp_rt_register'd buffer maps
// to its device mirror; any other host pointer is staged through a temporary
// device buffer (copied in when it is an input, copied back when it is an
// output, and the call then synchronises its stream).
class Operand {
 public:
  enum Dir { kIn = 1, kOut = 2, kInOut = 3 };
  Operand() = default;
  Operand(const Operand &) = delete;
  Operand &operator=(const Operand &) = delete;
  ~Operand();
  // Returns SIMP_RT_OK or a negative status.
  int bind(const void *p, size_t bytes, Dir dir, const char *name);
  void *dev() const { return dev_; }
  bool staged() const { return staged_; }
  // Copies a staged output back to its host range (on the current stream).
  int commit();

 private:
  const void *host_ = nullptr;
  void *dev_ = nullptr;
  size_t bytes_ = 0;
  Dir dir_ = kIn;
  bool staged_ = false;
};

// Device address of a caller range that must already be device-resident
// (device memory, or inside a simp_rt_register'd range); no staging.
int device_view(const void *p, size_t bytes, const void **dev, const char *name);
// The same lookup without an error: false when p is plain host memory.
bool try_device_view(const void *p, size_t bytes, const void **dev);

// Weight arrays of one model-level export entry (export_state.hip).  Device
// memory and simp_rt_register'd ranges are used in place; any other host array
// gets a private device copy with a fingerprint per 64 KiB chunk, re-checked by
// verify(): every chunk when `full` (a call that starts a sequence), else the
// next chunk of each array in rotation (a mismatch re-checks that whole
// array); changed chunks are uploaded again.  The caller must not have kernels
// reading the copies in flight (the exports synchronise before returning).
class ExportWeights {
 public:
  int bind(const void *p, size_t bytes, const void **dev, const char *name);
  int verify(bool full);
  void release();
  int64_t refreshed_chunks() const { return refreshed_; }

 private:
  struct Range {
    const char *host = nullptr;
    size_t bytes = 0;
    char *dev = nullptr;
    std::vector<uint64_t> hash;
    size_t cursor = 0;
  };
  int refresh(Range &r, bool all, size_t first);
  std::vector<Range> ranges_;
  bool fresh_ = true;
  int64_t refreshed_ = 0;
};

// Position continuity of a model-level export's KV cache.  prepare() is called
// before a step at `pos`: unless the call continues the previous one (pos is
// the previous pos + 1 with the same caller cache arrays) it copies the
// caller's rows [0, pos) of every layer into the engine's cache (layout
// [layers, seq_len, kv_dim], `pitch_bytes` per layer) and reports a restart.
// done() records a completed step.
struct KvState {
  int64_t next_pos = -1;
  const void *k = nullptr, *v = nullptr;
  int prepare(int64_t pos, const void *caller_k, const void *caller_v, void *dev_k, void *dev_v,
              size_t row_bytes, size_t pitch_bytes, int64_t layers, hipStream_t st,
              bool *restart);
  void done(int64_t pos) { next_pos = pos + 1; }
};

// Device address of the allocation-free int8 entry point's static scratch on
// the current device (looked up on first use per device, then cached).
int noalloc_scratch(void **ptr);

// Frees the engines of llama32_forward (part of simp_rt_forward_cache_clear).
void l32_cache_clear();

// Finishes an entry point: commits staged outputs and, when anything was
// staged, waits for the stream so host buffers are valid on return.
int finish(Operand *const *ops, int n);

// Geometry checks shared by entry points.
int check_desc2(const char *name, const void *aligned, int64_t off, int64_t s0,
                int64_t s1, int64_t st0, int64_t st1);
int check_desc1(const char *name, const void *aligned, int64_t off, int64_t size,
                int64_t stride);
// Rank-n descriptor (n <= 4): innermost stride 1, each outer stride at least the
// span of the level inside it (no two elements alias).  *span receives the
// element extent from the first to one past the last element (0 when empty).
int check_descn(const char *name, const void *aligned, int64_t off, int rank,
                const int64_t *sizes, const int64_t *strides, int64_t *span);

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Number of CUs of the current device (cached per device).
int num_cus();

// Library-owned device scratch for (current device, stream, slot), grown on
// demand and kept until the process ends.  Calls on one stream are ordered, so
// they may share it; calls on different streams get different buffers.  Slot 0
// belongs to the int8 GEMM dispatch; an entry point that stages operands for it
// (the i4 product) uses slot 1.
int workspace(hipStream_t stream, size_t bytes, void **ptr, int slot = 0);

// Optional per-kernel timing (simp_rt_timing): while enabled, a KernelTimer
// brackets the launches between its construction and stop() with HIP events on
// their stream, recorded under the given kernel name.  Inactive (no events) when
// timing is off or the stream is being captured.
class KernelTimer {
 public:
  KernelTimer(hipStream_t st, const char *name);
  KernelTimer(const KernelTimer &) = delete;
  KernelTimer &operator=(const KernelTimer &) = delete;
  void stop();
  ~KernelTimer() { stop(); }

 private:
  hipStream_t st_;
  hipEvent_t end_ = nullptr;
};

// Kernel launchers on device pointers, shared by the op entry points and the
// decode step.
int launch_w4s(const uint8_t *W, int64_t ldw, const float *S, int64_t lds, const float *X,
               int64_t ldx, float *O, int64_t ldo, int M, int N, int K, int gs, hipStream_t st);
int launch_w4u(const uint8_t *Q, const float *S, const float *Z, const float *X, float *O, int rows,
               int cols, int gs, int64_t off, hipStream_t st);
int launch_rmsnorm(const float *x, const float *w, float *out, int n, float eps, hipStream_t st);

// Symmetric W4 GEMV with one x vector on v_dot8_i32_i4 (w4d8.hip).  Up to three
// row segments, each with its own weights [rows, ldw bytes], scales
// [rows, lds floats] and output; x = x0, or rmsnorm(x0) * nw when nw is set;
// out_mode 0 stores, 1 adds to the output, 2 pairs row i of segment 0 (W1)
// with row i of segment 1 (W3) and stores silu(h1) * h3 into segment 0's output.
// With zeros Z (laid out like S; every segment or none, one x vector) the
// nibbles are unsigned and a weight is q * s + z (the reference W4 format).
struct W4D8Seg {
  const uint8_t *W;
  const float *S;
  float *out;
  int64_t ldw, lds;
  int rows;
  const float *Z = nullptr;
};
struct W4D8Args {
  W4D8Seg s[3];
  int n;
  int K, gs;
  const float *x0, *nw;
  float eps;
  int out_mode;
  int bstart[3];  // first block of each segment (set by launch_w4d8)
  // mx > 1 (at most 4) x vectors, rows ldx floats apart, outputs rows ldo apart
  // (one segment, out_mode 0, no norm)
  int mx = 1;
  int64_t ldx = 0, ldo = 0;
  // cws set: x is the combination of split-attention partials instead of x0
  // (one segment, out_mode 1, no norm).  Chunk s of head h sits at
  // cws + (h * cmax + s) * (chs + 4): the unnormalised o[chs], then m and l;
  // x[h * chs + d] = sum_s e^(m_s - M) o_s[d] / sum_s e^(m_s - M) l_s over the
  // cn chunks, M = max_s m_s.
  const float *cws = nullptr;
  int chs = 0, cmax = 0, cn = 0;
};
// K a multiple of 32 and of gs (a multiple of 32), K <= 20480, x0 and nw 16-byte aligned.
bool w4d8_supported(int K, int gs, const void *x0, const void *nw);
int launch_w4d8(const W4D8Args &a, hipStream_t st);
// C = beta*C + A*B (beta 0 or 1), row-major with leading dimensions in elements.
int launch_matmul_f32(const float *A, int64_t lda, const float *B, int64_t ldb, float *C,
                      int64_t ldc, int M, int N, int K, float beta, hipStream_t st);

}  // namespace simp
