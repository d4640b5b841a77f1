// rt_core.hip -- errors, streams, device-buffer registry and operand residency
// for libsimp_hip.so.
//
// The reference's compiled programs take plain host arrays as MLIR memref
// descriptors (examples/llama2/bench_llama_quant.cpp:10-28) and have no
// status codes; SimpLang's loader reports failures with std::runtime_error
// (runtime/include/kernel_runner.hpp:40-56).  Here every entry point returns an
// int32 status and leaves the message in a thread-local string.
#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <vector>

#include <atomic>
#include "rt_internal.h"

namespace simp {

static thread_local std::string t_err;
static thread_local int64_t t_err_count = 0;
static thread_local hipStream_t t_stream = nullptr;

int set_error(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  t_err = buf;
  t_err_count++;
  return code;
}

void clear_error() { t_err.clear(); }

int hip_fail(hipError_t e, const char *what) {
  return set_error(SIMP_RT_EHIP, "%s failed: %s", what, hipGetErrorString(e));
}

hipStream_t cur_stream() { return t_stream; }

namespace {
struct Mirror {
  void *dev;
  size_t bytes;
  int flags;
  int device;
};
std::mutex g_mu;
std::map<uintptr_t, Mirror> g_reg;  // host start -> mirror
std::vector<int> g_cus;            // CU count per device, 0 = unknown
}  // namespace

int ensure_device() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  return dev;
}

int num_cus() {
  int dev = ensure_device();
  if (dev < 0) return 0;
  std::lock_guard<std::mutex> lk(g_mu);
  if ((int)g_cus.size() <= dev) g_cus.resize(dev + 1, 0);
  if (g_cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      n = 256;
    g_cus[dev] = n > 0 ? n : 256;
  }
  return g_cus[dev];
}

namespace {
struct WsKey {
  int dev;
  hipStream_t stream;
  int slot;
  bool operator<(const WsKey &o) const {
    if (dev != o.dev) return dev < o.dev;
    if (stream != o.stream) return (uintptr_t)stream < (uintptr_t)o.stream;
    return slot < o.slot;
  }
};
struct WsBuf {
  void *ptr = nullptr;
  size_t bytes = 0;
};
std::map<WsKey, WsBuf> g_ws;
}  // namespace

int workspace(hipStream_t stream, size_t bytes, void **ptr, int slot) {
  int dev = ensure_device();
  if (dev < 0) return dev;
  std::lock_guard<std::mutex> lk(g_mu);
  WsBuf &b = g_ws[WsKey{dev, stream, slot}];
  if (b.bytes < bytes) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
      return set_error(SIMP_RT_EUNSUPPORTED,
                       "workspace of %zu bytes needed while the stream is being captured; "
                       "make one uncaptured call of the same size on this stream first", bytes);
    if (b.ptr) {
      SIMP_HIP(hipStreamSynchronize(stream));  // earlier calls may still read it
      SIMP_HIP(hipFree(b.ptr));
      b.ptr = nullptr;
      b.bytes = 0;
    }
    size_t want = std::max(bytes, (size_t)1 << 20);
    hipError_t e = hipMalloc(&b.ptr, want);
    if (e != hipSuccess) {
      b.ptr = nullptr;
      return set_error(SIMP_RT_ENOMEM, "workspace of %zu bytes: %s", want, hipGetErrorString(e));
    }
    b.bytes = want;
  }
  *ptr = b.ptr;
  return SIMP_RT_OK;
}

// Looks p up in the registry; returns the device address or nullptr.
static void *find_mirror(const void *p, size_t bytes, int *flags) {
  std::lock_guard<std::mutex> lk(g_mu);
  uintptr_t a = (uintptr_t)p;
  auto it = g_reg.upper_bound(a);
  if (it == g_reg.begin()) return nullptr;
  --it;
  if (a < it->first || a + bytes > it->first + it->second.bytes) return nullptr;
  if (flags) *flags = it->second.flags;
  return (char *)it->second.dev + (a - it->first);
}

static bool is_device_memory(const void *p) {
  hipPointerAttribute_t attr;
  std::memset(&attr, 0, sizeof attr);
  hipError_t e = hipPointerGetAttributes(&attr, p);
  if (e != hipSuccess) {
    (void)hipGetLastError();  // unregistered host memory: clear the sticky error
    return false;
  }
  return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}

bool try_device_view(const void *p, size_t bytes, const void **dev) {
  if (!p) return false;
  if (is_device_memory(p)) {
    *dev = p;
    return true;
  }
  if (void *m = find_mirror(p, bytes, nullptr)) {
    *dev = m;
    return true;
  }
  return false;
}

int device_view(const void *p, size_t bytes, const void **dev, const char *name) {
  if (!p) return set_error(SIMP_RT_EINVAL, "%s: null pointer", name);
  if (try_device_view(p, bytes, dev)) return SIMP_RT_OK;
  return set_error(SIMP_RT_EINVAL,
                   "%s: must be device memory or inside a simp_rt_register'd range", name);
}

Operand::~Operand() {
  if (staged_ && dev_) (void)hipFree(dev_);
}

int Operand::bind(const void *p, size_t bytes, Dir dir, const char *name) {
  host_ = p;
  bytes_ = bytes;
  dir_ = dir;
  if (bytes == 0) {
    dev_ = const_cast<void *>(p);
    return SIMP_RT_OK;
  }
  if (!p) return set_error(SIMP_RT_EINVAL, "%s: null pointer", name);
  if (is_device_memory(p)) {
    dev_ = const_cast<void *>(p);
    return SIMP_RT_OK;
  }
  int flags = 0;
  if (void *m = find_mirror(p, bytes, &flags)) {
    if ((dir & kOut) && (flags & SIMP_RT_REG_IMMUTABLE))
      return set_error(SIMP_RT_EINVAL,
                       "%s: output lies in a buffer registered as immutable", name);
    dev_ = m;
    return SIMP_RT_OK;
  }
  hipError_t e = hipMalloc(&dev_, bytes);
  if (e != hipSuccess) {
    dev_ = nullptr;
    return set_error(SIMP_RT_ENOMEM, "%s: staging %zu bytes: %s", name, bytes,
                     hipGetErrorString(e));
  }
  staged_ = true;
  // Outputs are staged in too: a strided view's span holds bytes between its
  // rows (or batches) that the kernels never write, and commit() copies the
  // whole span back, so those bytes must return to the host as they were.
  if (dir & (kIn | kOut)) {
    e = hipMemcpyAsync(dev_, p, bytes, hipMemcpyHostToDevice, cur_stream());
    if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(stage in)");
  }
  return SIMP_RT_OK;
}

int Operand::commit() {
  if (!staged_ || !(dir_ & kOut) || bytes_ == 0) return SIMP_RT_OK;
  SIMP_HIP(hipMemcpyAsync(const_cast<void *>(host_), dev_, bytes_,
                          hipMemcpyDeviceToHost, cur_stream()));
  return SIMP_RT_OK;
}

int finish(Operand *const *ops, int n) {
  bool any = false;
  for (int i = 0; i < n; i++) {
    int rc = ops[i]->commit();
    if (rc) return rc;
    any = any || ops[i]->staged();
  }
  SIMP_HIP(hipGetLastError());
  if (any) SIMP_HIP(hipStreamSynchronize(cur_stream()));
  return SIMP_RT_OK;
}

int check_desc2(const char *name, const void *aligned, int64_t off, int64_t s0,
                int64_t s1, int64_t st0, int64_t st1) {
  if (s0 < 0 || s1 < 0 || off < 0)
    return set_error(SIMP_RT_EINVAL, "%s: negative size or offset", name);
  if (s0 > 0 && s1 > 0) {
    if (!aligned) return set_error(SIMP_RT_EINVAL, "%s: null pointer", name);
    if (st1 != 1)
      return set_error(SIMP_RT_EINVAL, "%s: inner stride %lld != 1 (row-major required)",
                       name, (long long)st1);
    if (st0 < s1)
      return set_error(SIMP_RT_EINVAL, "%s: row stride %lld < row length %lld", name,
                       (long long)st0, (long long)s1);
  }
  return SIMP_RT_OK;
}

int check_descn(const char *name, const void *aligned, int64_t off, int rank,
                const int64_t *sizes, const int64_t *strides, int64_t *span) {
  *span = 0;
  if (off < 0) return set_error(SIMP_RT_EINVAL, "%s: negative offset", name);
  bool empty = false;
  for (int i = 0; i < rank; i++) {
    if (sizes[i] < 0) return set_error(SIMP_RT_EINVAL, "%s: negative size", name);
    empty |= sizes[i] == 0;
  }
  if (empty) return SIMP_RT_OK;
  if (!aligned) return set_error(SIMP_RT_EINVAL, "%s: null pointer", name);
  if (strides[rank - 1] != 1)
    return set_error(SIMP_RT_EINVAL, "%s: inner stride %lld != 1 (row-major required)", name,
                     (long long)strides[rank - 1]);
  int64_t inner = sizes[rank - 1];  // span of the levels inside level i
  for (int i = rank - 2; i >= 0; i--) {
    if (strides[i] < inner)
      return set_error(SIMP_RT_EINVAL, "%s: stride %d (%lld) < span %lld of the dimensions inside it",
                       name, i, (long long)strides[i], (long long)inner);
    if (sizes[i] - 1 > (INT64_MAX - inner) / strides[i])
      return set_error(SIMP_RT_EINVAL, "%s: extent overflows", name);
    inner += (sizes[i] - 1) * strides[i];
  }
  *span = inner;
  return SIMP_RT_OK;
}

int check_desc1(const char *name, const void *aligned, int64_t off, int64_t size,
                int64_t stride) {
  if (size < 0 || off < 0) return set_error(SIMP_RT_EINVAL, "%s: negative size or offset", name);
  if (size > 0 && !aligned) return set_error(SIMP_RT_EINVAL, "%s: null pointer", name);
  if (size > 0 && stride != 1)
    return set_error(SIMP_RT_EINVAL, "%s: stride %lld != 1", name, (long long)stride);
  return SIMP_RT_OK;
}

// ------------------------------------------------------------ kernel timing
namespace {
struct TimedLaunch {
  std::string name;
  hipEvent_t start, end;
};
std::atomic<bool> g_timing{false};
std::mutex g_timing_mu;
std::vector<TimedLaunch> g_timed;

void clear_timed() {
  std::lock_guard<std::mutex> lk(g_timing_mu);
  for (auto &t : g_timed) {
    (void)hipEventDestroy(t.start);
    (void)hipEventDestroy(t.end);
  }
  g_timed.clear();
}
}  // namespace

KernelTimer::KernelTimer(hipStream_t st, const char *name) : st_(st) {
  if (!g_timing.load(std::memory_order_relaxed)) return;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return;
  hipEvent_t a = nullptr, b = nullptr;
  if (hipEventCreate(&a) != hipSuccess) return;
  if (hipEventCreate(&b) != hipSuccess) {
    (void)hipEventDestroy(a);
    return;
  }
  if (hipEventRecord(a, st) != hipSuccess) {
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    return;
  }
  end_ = b;
  std::lock_guard<std::mutex> lk(g_timing_mu);
  g_timed.push_back(TimedLaunch{name, a, b});
}

void KernelTimer::stop() {
  if (!end_) return;
  (void)hipEventRecord(end_, st_);
  end_ = nullptr;
}

}  // namespace simp

using namespace simp;

extern "C" {

int32_t simp_rt_timing(int32_t on) {
  g_timing.store(false);
  clear_timed();
  g_timing.store(on != 0);
  return SIMP_RT_OK;
}

int32_t simp_rt_timing_query(const char *kernel, double *total_ms, int64_t *launches) {
  if (!kernel || !total_ms || !launches)
    return set_error(SIMP_RT_EINVAL, "timing_query: null argument");
  double tot = 0.0;
  int64_t n = 0;
  std::lock_guard<std::mutex> lk(g_timing_mu);
  for (auto &t : g_timed) {
    if (t.name != kernel) continue;
    SIMP_HIP(hipEventSynchronize(t.end));
    float ms = 0.f;
    SIMP_HIP(hipEventElapsedTime(&ms, t.start, t.end));
    tot += ms;
    n++;
  }
  *total_ms = tot;
  *launches = n;
  return SIMP_RT_OK;
}

const char *simp_rt_last_error(void) { return t_err.c_str(); }

int64_t simp_rt_error_count(void) { return t_err_count; }

int32_t simp_rt_version(void) { return SIMP_RT_ABI_VERSION; }

int32_t simp_rt_init(void) {
  int n = 0;
  SIMP_HIP(hipGetDeviceCount(&n));
  if (n <= 0) return set_error(SIMP_RT_ENODEV, "no HIP device visible");
  int dev = ensure_device();
  if (dev < 0) return dev;
  if (num_cus() <= 0) return SIMP_RT_ENODEV;
  void *scratch = nullptr;  // set-up of simp_rt_matmul_u8s8_i32_noalloc on this device
  return noalloc_scratch(&scratch);
}

int32_t simp_rt_set_stream(void *stream) {
  t_stream = (hipStream_t)stream;
  return SIMP_RT_OK;
}

void *simp_rt_get_stream(void) { return (void *)t_stream; }

int32_t simp_rt_sync(void) {
  SIMP_HIP(hipStreamSynchronize(t_stream));
  return SIMP_RT_OK;
}

int32_t simp_rt_register(const void *host_ptr, int64_t bytes, int32_t flags) {
  if (!host_ptr || bytes <= 0) return set_error(SIMP_RT_EINVAL, "register: bad range");
  int dev = ensure_device();
  if (dev < 0) return dev;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    uintptr_t a = (uintptr_t)host_ptr;
    auto it = g_reg.upper_bound(a + (uintptr_t)bytes - 1);
    if (it != g_reg.begin()) {
      --it;
      if (it->first + it->second.bytes > a)
        return set_error(SIMP_RT_EINVAL, "register: range overlaps a registered buffer");
    }
  }
  void *d = nullptr;
  hipError_t e = hipMalloc(&d, (size_t)bytes);
  if (e != hipSuccess)
    return set_error(SIMP_RT_ENOMEM, "register: hipMalloc(%lld): %s", (long long)bytes,
                     hipGetErrorString(e));
  e = hipMemcpy(d, host_ptr, (size_t)bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(d);
    return hip_fail(e, "register: hipMemcpy");
  }
  std::lock_guard<std::mutex> lk(g_mu);
  g_reg[(uintptr_t)host_ptr] = Mirror{d, (size_t)bytes, flags, dev};
  return SIMP_RT_OK;
}

int32_t simp_rt_unregister(const void *host_ptr) {
  Mirror m;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_reg.find((uintptr_t)host_ptr);
    if (it == g_reg.end()) return set_error(SIMP_RT_EINVAL, "unregister: not registered");
    m = it->second;
    g_reg.erase(it);
  }
  SIMP_HIP(hipDeviceSynchronize());
  SIMP_HIP(hipFree(m.dev));
  return SIMP_RT_OK;
}

int32_t simp_rt_device_ptr(const void *host_ptr, void **dev_ptr) {
  if (!dev_ptr) return set_error(SIMP_RT_EINVAL, "device_ptr: null out pointer");
  void *m = find_mirror(host_ptr, 1, nullptr);
  if (!m) return set_error(SIMP_RT_EINVAL, "device_ptr: pointer not registered");
  *dev_ptr = m;
  return SIMP_RT_OK;
}

int32_t simp_rt_sync_to_host(const void *host_ptr, int64_t bytes) {
  int flags = 0;
  void *m = find_mirror(host_ptr, (size_t)bytes, &flags);
  if (!m) return set_error(SIMP_RT_EINVAL, "sync_to_host: range not registered");
  SIMP_HIP(hipMemcpyAsync(const_cast<void *>(host_ptr), m, (size_t)bytes,
                          hipMemcpyDeviceToHost, t_stream));
  SIMP_HIP(hipStreamSynchronize(t_stream));
  return SIMP_RT_OK;
}

int32_t simp_rt_malloc(void **dev_ptr, int64_t bytes) {
  if (!dev_ptr || bytes < 0) return set_error(SIMP_RT_EINVAL, "malloc: bad arguments");
  hipError_t e = hipMalloc(dev_ptr, (size_t)(bytes > 0 ? bytes : 1));
  if (e != hipSuccess)
    return set_error(SIMP_RT_ENOMEM, "malloc(%lld): %s", (long long)bytes, hipGetErrorString(e));
  return SIMP_RT_OK;
}

int32_t simp_rt_free(void *dev_ptr) {
  SIMP_HIP(hipFree(dev_ptr));
  return SIMP_RT_OK;
}

int32_t simp_rt_memcpy(void *dst, const void *src, int64_t bytes) {
  if (bytes < 0) return set_error(SIMP_RT_EINVAL, "memcpy: negative size");
  SIMP_HIP(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyDefault, t_stream));
  SIMP_HIP(hipStreamSynchronize(t_stream));
  return SIMP_RT_OK;
}

}  // extern "C"
