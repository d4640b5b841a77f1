// export_state.hip -- what the model-level exports (stories110M_forward,
// llama2_quant_forward, llama32_forward) keep between calls, and how they keep
// it faithful to the caller's arrays.
//
// The compiled programs read every weight and both KV caches from the caller's
// arrays on every call (examples/llama2/stories110M.sl:5-247,
// llama2_quant.sl:7-198, llama32_1b_int8_tensor.sl:16-305).  The exports keep
// device copies instead, so they must notice when the caller's arrays change:
//   * weights held in host memory get a private device copy with a 64-bit
//     fingerprint per 64 KiB chunk.  A call that starts a sequence (pos 0, or
//     any pos that does not follow the previous call's) re-hashes every chunk
//     and re-uploads the chunks that changed; any other call re-hashes one
//     chunk of each array, in rotation, and a mismatch there re-checks the
//     whole array (simp_rt_export_verify_all(1): every chunk on every call).
//     Device-resident weights and ranges the caller registered
//     with simp_rt_register are used in place (the caller owns their contents).
//   * the engine's device KV cache is refilled from the caller's cache rows
//     [0, pos) of every layer whenever a call does not continue the previous
//     one (first call, a jump or a restart, other cache arrays).
#include <algorithm>
#include <atomic>
#include <cstring>
#include <thread>

#include <sched.h>

#include "rt_internal.h"

namespace simp {

namespace {

constexpr size_t kChunk = size_t(1) << 16;

inline uint64_t rotl(uint64_t v, int r) { return (v << r) | (v >> (64 - r)); }

// Four independent multiply-rotate lanes over 8-byte words, then a final mix
// (a fingerprint for change detection, not a cryptographic hash).
uint64_t fingerprint_mul(const char *p, size_t n) {
  const uint64_t P1 = 0x9E3779B185EBCA87ull, P2 = 0xC2B2AE3D27D4EB4Full;
  uint64_t h[4] = {P1, P2, P1 ^ P2, ~P1};
  size_t i = 0;
  for (; i + 32 <= n; i += 32) {
    uint64_t w[4];
    std::memcpy(w, p + i, 32);
    for (int k = 0; k < 4; k++) h[k] = rotl((h[k] ^ w[k]) * P1, 31) * P2;
  }
  uint64_t t = n;
  for (; i < n; i++) t = (t ^ (uint8_t)p[i]) * P1;
  uint64_t r = t;
  for (int k = 0; k < 4; k++) r = rotl(r ^ h[k], 27) * P1 + P2;
  r ^= r >> 33;
  r *= P2;
  r ^= r >> 29;
  return r;
}

// The same role on the SSE4.2 CRC32C instruction: four independent CRC
// streams over 8-byte words (one instruction per word, pipelined across the
// streams), combined by a multiply-xorshift mix.  About 1.5x the rate of the
// multiply-rotate lanes over host memory (706 MB on 8 threads: 14 against
// 21 ms), which is what a sequence start of a host-array export pays (7.6 ms
// on 16 threads).
__attribute__((target("sse4.2"))) uint64_t fingerprint_crc(const char *p, size_t n) {
  uint64_t c[4] = {0x243F6A88u, 0x85A308D3u, 0x13198A2Eu, 0x03707344u};
  size_t i = 0;
  for (; i + 32 <= n; i += 32) {
    uint64_t w[4];
    std::memcpy(w, p + i, 32);
    for (int k = 0; k < 4; k++) c[k] = __builtin_ia32_crc32di(c[k], w[k]);
  }
  for (; i < n; i++) c[0] = __builtin_ia32_crc32qi((uint32_t)c[0], (uint8_t)p[i]);
  const uint64_t P1 = 0x9E3779B185EBCA87ull, P2 = 0xC2B2AE3D27D4EB4Full;
  uint64_t r = ((c[0] | (c[1] << 32)) ^ rotl(c[2] | (c[3] << 32), 29)) * P1 + n;
  r ^= r >> 33;
  r *= P2;
  r ^= r >> 29;
  return r;
}

uint64_t fingerprint(const char *p, size_t n) {
  static const bool crc = __builtin_cpu_supports("sse4.2");
  return crc ? fingerprint_crc(p, n) : fingerprint_mul(p, n);
}

// Threads for host-side hashing: the CPUs this process may run on (its
// affinity mask, not every CPU of the host), at most 16.
unsigned host_threads() {
  cpu_set_t set;
  CPU_ZERO(&set);
  int n = sched_getaffinity(0, sizeof set, &set) == 0 ? CPU_COUNT(&set) : 0;
  if (n <= 0) n = (int)std::thread::hardware_concurrency();
  return (unsigned)std::max(1, std::min(n, 16));
}

// Runs f(i) for i in [0, n), on host_threads() threads when there is enough work.
template <class F>
void parallel_for(size_t n, size_t bytes, F f) {
  static const unsigned nt = host_threads();
  if (bytes < (size_t(64) << 20) || nt <= 1 || n < 2 * nt) {
    for (size_t i = 0; i < n; i++) f(i);
    return;
  }
  std::vector<std::thread> th;
  for (unsigned t = 0; t < nt; t++)
    th.emplace_back([&, t] {
      for (size_t i = t; i < n; i += nt) f(i);
    });
  for (auto &x : th) x.join();
}

}  // namespace

int ExportWeights::bind(const void *p, size_t bytes, const void **dev, const char *name) {
  if (!p) return set_error(SIMP_RT_EINVAL, "%s: null pointer", name);
  if (try_device_view(p, bytes, dev)) return SIMP_RT_OK;
  Range r;
  r.host = (const char *)p;
  r.bytes = bytes;
  hipError_t e = hipMalloc((void **)&r.dev, std::max<size_t>(bytes, 1));
  if (e != hipSuccess)
    return set_error(SIMP_RT_ENOMEM, "%s: device copy of %zu bytes: %s", name, bytes,
                     hipGetErrorString(e));
  e = hipMemcpy(r.dev, p, bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(r.dev);
    return hip_fail(e, "export weights: hipMemcpy");
  }
  r.hash.resize(cdiv((int64_t)bytes, (int64_t)kChunk));
  parallel_for(r.hash.size(), bytes, [&](size_t c) {
    const size_t at = c * kChunk;
    r.hash[c] = fingerprint(r.host + at, std::min(kChunk, bytes - at));
  });
  ranges_.push_back(std::move(r));
  *dev = ranges_.back().dev;
  return SIMP_RT_OK;
}

int ExportWeights::refresh(Range &r, bool all, size_t first) {
  const size_t n = r.hash.size();
  std::vector<uint8_t> changed(n, 0);
  if (all) {
    parallel_for(n, r.bytes, [&](size_t c) {
      const size_t at = c * kChunk;
      const uint64_t h = fingerprint(r.host + at, std::min(kChunk, r.bytes - at));
      if (h != r.hash[c]) {
        r.hash[c] = h;
        changed[c] = 1;
      }
    });
  } else {
    const size_t at = first * kChunk;
    const uint64_t h = fingerprint(r.host + at, std::min(kChunk, r.bytes - at));
    if (h == r.hash[first]) return SIMP_RT_OK;
    return refresh(r, true, 0);  // one chunk changed: look at the whole array
  }
  for (size_t c = 0; c < n;) {  // upload runs of changed chunks
    if (!changed[c]) {
      c++;
      continue;
    }
    size_t e = c;
    while (e < n && changed[e]) e++;
    const size_t at = c * kChunk, len = std::min(e * kChunk, r.bytes) - at;
    SIMP_HIP(hipMemcpy(r.dev + at, r.host + at, len, hipMemcpyHostToDevice));
    refreshed_ += e - c;
    c = e;
  }
  return SIMP_RT_OK;
}

// simp_rt_export_verify_all: every call re-checks every chunk (as a sequence
// start does), so that any edit of a host array is seen by the next call.
std::atomic<int> g_verify_all{0};

int ExportWeights::verify(bool full) {
  if (fresh_) {  // the copies were made (and hashed) by this very call
    fresh_ = false;
    return SIMP_RT_OK;
  }
  full = full || g_verify_all.load(std::memory_order_relaxed) != 0;
  for (Range &r : ranges_) {
    if (r.hash.empty()) continue;
    int rc;
    if (full) {
      rc = refresh(r, true, 0);
    } else {
      rc = refresh(r, false, r.cursor);
      r.cursor = (r.cursor + 1) % r.hash.size();
    }
    if (rc) return rc;
  }
  return SIMP_RT_OK;
}

void ExportWeights::release() {
  for (Range &r : ranges_)
    if (r.dev) (void)hipFree(r.dev);
  ranges_.clear();
}

int KvState::prepare(int64_t pos, const void *caller_k, const void *caller_v, void *dev_k,
                     void *dev_v, size_t row_bytes, size_t pitch_bytes, int64_t layers,
                     hipStream_t st, bool *restart) {
  *restart = !(pos == next_pos && caller_k == k && caller_v == v);
  if (*restart && pos > 0) {
    const size_t w = row_bytes * (size_t)pos;
    SIMP_HIP(hipMemcpy2DAsync(dev_k, pitch_bytes, caller_k, pitch_bytes, w, (size_t)layers,
                              hipMemcpyDefault, st));
    SIMP_HIP(hipMemcpy2DAsync(dev_v, pitch_bytes, caller_v, pitch_bytes, w, (size_t)layers,
                              hipMemcpyDefault, st));
  }
  next_pos = -1;  // set again by done() once the call has succeeded
  k = caller_k;
  v = caller_v;
  return SIMP_RT_OK;
}

}  // namespace simp

extern "C" int32_t simp_rt_export_verify_all(int32_t on) {
  simp::g_verify_all.store(on ? 1 : 0, std::memory_order_relaxed);
  return SIMP_RT_OK;
}
