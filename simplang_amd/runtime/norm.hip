// norm.hip -- wavefront/block-reduction kernels: rmsnorm, softmax, silu, the
// SwiGLU gate and RoPE.  Semantics follow the reference lowering loops (paths
// relative to the SimpLang tree):
//   rmsnorm  ConvertSimpToMemRef.cpp:2192-2233  rms = sqrt(sum x^2 / n + eps),
//            out = (x / rms) * w[w_off + i]  (a division, as in the reference)
//   softmax  ConvertSimpToMemRef.cpp:2264-2316  out = exp(x - max) / sum, offsets on
//            both arrays
//   silu     ConvertSimpToMemRef.cpp:2345-2354  out = x / (1 + exp(-x))
//   swiglu   examples/llama2/stories110M.sl:200-212  out = silu(gate) * up
//   rope     examples/llama2/stories110M.sl:86-112  adjacent pairs, f = theta^-(i%hs/hs)
// The reference sums sequentially; here sums are wave/block trees (fp32), which
// changes rounding only (checked to 1e-4 relative against the oracle).
// rmsnorm and softmax run as one block up to 32767 elements (their cost there
// is the launch) and as two passes over many blocks from 32768 on.
#include <algorithm>

#include "rt_device.h"
#include "rt_internal.h"

namespace simp {
namespace {

// Single-block forms: thread t keeps elements t + k T (k < R) in registers, so
// x (and w) are read once, all before the block reductions (DPP within a wave,
// LDS across waves; loads of w stay in flight across them), and out is
// written once.  Every read precedes the first barrier, so out may alias x.
template <int T, int R>
__global__ void __launch_bounds__(T)
    rmsnorm_k(const float *__restrict__ x, const float *__restrict__ w, float *out, int n,
              float eps) {
  __shared__ float scratch[16];
  float xv[R], wv[R];
#pragma unroll
  for (int k = 0; k < R; k++) {
    const int i = threadIdx.x + k * T;
    xv[k] = i < n ? x[i] : 0.f;
    wv[k] = i < n ? w[i] : 0.f;
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < R; k++) ss = fmaf(xv[k], xv[k], ss);
  ss = block_sum_lds<true>(ss, scratch);
  const float rms = sqrtf(ss / (float)n + eps);
#pragma unroll
  for (int k = 0; k < R; k++) {
    const int i = threadIdx.x + k * T;
    if (i < n) out[i] = (xv[k] / rms) * wv[k];
  }
}

template <int T, int R>
__global__ void __launch_bounds__(T) softmax_k(const float *__restrict__ x, float *out, int n) {
  __shared__ float scratch[16];
  float v[R];
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < R; k++) {
    const int i = threadIdx.x + k * T;
    v[k] = i < n ? x[i] : -INFINITY;
    mx = fmaxf(mx, v[k]);
  }
  mx = block_max_lds<true>(mx, scratch);
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < R; k++) {
    if (threadIdx.x + k * T < n) {
      v[k] = expf(v[k] - mx);
      s += v[k];
    }
  }
  s = block_sum_lds<true>(s, scratch);
#pragma unroll
  for (int k = 0; k < R; k++) {
    const int i = threadIdx.x + k * T;
    if (i < n) out[i] = v[k] / s;
  }
}

// Launches the single-block form whose T x R covers n (n < 32768).
template <template <int, int> class K, typename... Args>
void launch_one_block(int n, hipStream_t st, Args... args) {
  auto go = [&](auto t, auto r) {
    constexpr int T = decltype(t)::value, R = decltype(r)::value;
    hipLaunchKernelGGL((K<T, R>::fn), dim3(1), dim3(T), 0, st, args...);
  };
  using I256 = std::integral_constant<int, 256>;
  using I1024 = std::integral_constant<int, 1024>;
  if (n <= 256) go(I256{}, std::integral_constant<int, 1>{});
  else if (n <= 1024) go(I256{}, std::integral_constant<int, 4>{});
  else if (n <= 4096) go(I256{}, std::integral_constant<int, 16>{});
  else if (n <= 8192) go(I1024{}, std::integral_constant<int, 8>{});
  else if (n <= 16384) go(I1024{}, std::integral_constant<int, 16>{});
  else go(I1024{}, std::integral_constant<int, 32>{});
}
template <int T, int R>
struct RmsnormOne {
  static constexpr auto fn = rmsnorm_k<T, R>;
};
template <int T, int R>
struct SoftmaxOne {
  static constexpr auto fn = softmax_k<T, R>;
};

__global__ void __launch_bounds__(256) silu_k(const float *__restrict__ x, float *__restrict__ out,
                                              int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    out[i] = x[i] / (1.f + expf(-x[i]));
}

__global__ void __launch_bounds__(256)
    swiglu_k(const float *__restrict__ gate, const float *__restrict__ up, float *__restrict__ out,
             int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const float g = gate[i];
    out[i] = (g / (1.f + expf(-g))) * up[i];
  }
}

__global__ void __launch_bounds__(256)
    rope_k(float *__restrict__ q, float *__restrict__ k, int dim, int kv_dim, int hs, int pos,
           float theta) {
  const int i = 2 * (blockIdx.x * 256 + threadIdx.x);
  if (i >= dim) return;
  const float freq = 1.f / powf(theta, (float)(i % hs) / (float)hs);
  const float v = (float)pos * freq;
  const float fcr = cosf(v), fci = sinf(v);
  const float q0 = q[i], q1 = q[i + 1];
  q[i] = q0 * fcr - q1 * fci;
  q[i + 1] = q0 * fci + q1 * fcr;
  if (i < kv_dim) {
    const float k0 = k[i], k1 = k[i + 1];
    k[i] = k0 * fcr - k1 * fci;
    k[i + 1] = k0 * fci + k1 * fcr;
  }
}

// Vectors of kBigNorm elements or more take two passes over many blocks
// (below it one block is faster: the second launch costs more than the
// block's extra latency).  Pass 1: every block reduces its contiguous slice
// (sum of squares; or its maximum and the sum of e^(x - max)) into part[b].
// Pass 2: every block combines the parts in block order (the same order in
// every block, so the result is deterministic) and writes its slice.
constexpr int64_t kBigNorm = 32768;

// Block b's slice [b0, b1) of n elements: multiples of 4 apart, so that with
// 16-byte aligned arrays every slice but the last is whole float4s.
__device__ __forceinline__ void slice_of(int64_t n, int64_t *b0, int64_t *b1) {
  const int64_t per = ((n + gridDim.x - 1) / gridDim.x + 3) & ~(int64_t)3;
  *b0 = min(n, (int64_t)blockIdx.x * per);
  *b1 = min(n, *b0 + per);
}

// f(i, v) over the elements [b0, b1) of the block's threads: float4 loads,
// four in flight per thread, when `vec` (the arrays 16-byte aligned), then the
// slice's last n % 4 elements one by one.
template <typename F>
__device__ __forceinline__ void for_slice4(const float *__restrict__ x, int64_t b0, int64_t b1,
                                           bool vec, F f) {
  int64_t i = b0;
  if (vec) {
    const int64_t e4 = b0 + ((b1 - b0) & ~(int64_t)3);
    const float4 *x4 = (const float4 *)x;
    int64_t j = b0 / 4 + threadIdx.x;
    const int64_t j1 = e4 / 4;
    for (; j + 3 * 256 < j1; j += 4 * 256) {
      float4 v[4];
#pragma unroll
      for (int u = 0; u < 4; u++) v[u] = x4[j + u * 256];
#pragma unroll
      for (int u = 0; u < 4; u++) f(4 * (j + u * 256), v[u]);
    }
    for (; j < j1; j += 256) f(4 * j, x4[j]);
    i = e4;
  }
  for (int64_t k = i + threadIdx.x; k < b1; k += 256) f(-k - 1, make_float4(x[k], 0.f, 0.f, 0.f));
}

__global__ void __launch_bounds__(256)
    sumsq_parts_k(const float *__restrict__ x, int64_t n, float *__restrict__ part, bool vec) {
  __shared__ float scratch[16];
  int64_t b0, b1;
  slice_of(n, &b0, &b1);
  float ss = 0.f;
  for_slice4(x, b0, b1, vec, [&](int64_t i, float4 v) {
    ss = fmaf(v.x, v.x, ss);
    if (i >= 0) {
      ss = fmaf(v.y, v.y, ss);
      ss = fmaf(v.z, v.z, ss);
      ss = fmaf(v.w, v.w, ss);
    }
  });
  ss = block_sum(ss, scratch);
  if (threadIdx.x == 0) part[blockIdx.x] = ss;
}

// The blocks' partials, four per thread requested together (each thread's in
// increasing block order, as a strided loop would add them).
template <typename T, typename F>
__device__ __forceinline__ void for_parts(const T *__restrict__ part, F f) {
  const int G = (int)gridDim.x;
  for (int b0 = threadIdx.x; b0 < G; b0 += 4 * 256) {
    T v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) v[u] = b0 + 256 * u < G ? part[b0 + 256 * u] : T{};
#pragma unroll
    for (int u = 0; u < 4; u++)
      if (b0 + 256 * u < G) f(v[u]);
  }
}

__global__ void __launch_bounds__(256)
    rmsnorm_apply_k(const float *__restrict__ x, const float *__restrict__ w,
                    float *__restrict__ out, int64_t n, float eps, const float *__restrict__ part,
                    bool vec) {
  __shared__ float scratch[16];
  float t = 0.f;
  for_parts(part, [&](float p) { t += p; });
  t = block_sum(t, scratch);
  const float rms = sqrtf(t / (float)n + eps);
  int64_t b0, b1;
  slice_of(n, &b0, &b1);
  for_slice4(x, b0, b1, vec, [&](int64_t i, float4 v) {
    if (i >= 0) {
      const float4 g = *(const float4 *)(w + i);
      *(float4 *)(out + i) = make_float4((v.x / rms) * g.x, (v.y / rms) * g.y, (v.z / rms) * g.z,
                                         (v.w / rms) * g.w);
    } else {
      out[-i - 1] = (v.x / rms) * w[-i - 1];
    }
  });
}

// One read of the slice: every thread keeps a running maximum m and the sum l
// of e^(x - m), rescaling l when m grows (once per float4 at most).
__global__ void __launch_bounds__(256)
    softmax_parts_k(const float *__restrict__ x, int64_t n, float2 *__restrict__ part, bool vec) {
  __shared__ float scratch[16];
  int64_t b0, b1;
  slice_of(n, &b0, &b1);
  float m = -INFINITY, l = 0.f;
  for_slice4(x, b0, b1, vec, [&](int64_t i, float4 v) {
    const float m4 = i >= 0 ? fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w)) : v.x;
    if (m4 > m) {
      l *= expf(m - m4);  // e^-inf = 0 on the first finite value
      m = m4;
    }
    if (m > -INFINITY) {
      l += expf(v.x - m);
      if (i >= 0) l += (expf(v.y - m) + expf(v.z - m)) + expf(v.w - m);
    }
  });
  const float mx = block_max_lds<true>(m, scratch);
  const float t = block_sum_lds<true>(m > -INFINITY ? l * expf(m - mx) : 0.f, scratch);
  if (threadIdx.x == 0) part[blockIdx.x] = make_float2(mx, t);
}

__global__ void __launch_bounds__(256)
    softmax_apply_k(const float *__restrict__ x, float *__restrict__ out, int64_t n,
                    const float2 *__restrict__ part, bool vec) {
  __shared__ float scratch[16];
  float mx = -INFINITY;
  for_parts(part, [&](float2 p) { mx = fmaxf(mx, p.x); });
  mx = block_max(mx, scratch);
  float l = 0.f;
  for_parts(part, [&](float2 p) {
    if (p.x > -INFINITY) l += p.y * expf(p.x - mx);
  });
  l = block_sum(l, scratch);
  int64_t b0, b1;
  slice_of(n, &b0, &b1);
  for_slice4(x, b0, b1, vec, [&](int64_t i, float4 v) {
    if (i >= 0)
      *(float4 *)(out + i) = make_float4(expf(v.x - mx) / l, expf(v.y - mx) / l,
                                         expf(v.z - mx) / l, expf(v.w - mx) / l);
    else
      out[-i - 1] = expf(v.x - mx) / l;
  });
}

__global__ void __launch_bounds__(256) silu_big_k(const float *__restrict__ x,
                                                  float *__restrict__ out, int64_t n) {
  int64_t b0, b1;
  slice_of(n, &b0, &b1);
  for_slice4(x, b0, b1, true, [&](int64_t i, float4 v) {
    if (i >= 0)
      *(float4 *)(out + i) = make_float4(v.x / (1.f + expf(-v.x)), v.y / (1.f + expf(-v.y)),
                                         v.z / (1.f + expf(-v.z)), v.w / (1.f + expf(-v.w)));
    else
      out[-i - 1] = v.x / (1.f + expf(-v.x));
  });
}

// Blocks of the two-pass forms: about 8 slices of 256 x 8 elements per CU.
unsigned big_grid(int64_t n) {
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(cdiv(n, 256 * 8), (int64_t)num_cus() * 4));
}

unsigned grid_for(int64_t n) {
  const int64_t b = cdiv(n, 256);
  const int64_t cap = (int64_t)num_cus() * 8;
  return (unsigned)(b < cap ? (b > 0 ? b : 1) : cap);
}

}  // namespace

int launch_rmsnorm(const float *x, const float *w, float *out, int n, float eps, hipStream_t st) {
  if (n >= kBigNorm) {
    const unsigned g = big_grid(n);
    float *part = nullptr;
    int rc = workspace(st, sizeof(float2) * g, (void **)&part, 4);
    if (rc) return rc;
    const bool vec = (((uintptr_t)x | (uintptr_t)w | (uintptr_t)out) & 15) == 0;
    hipLaunchKernelGGL(sumsq_parts_k, dim3(g), dim3(256), 0, st, x, (int64_t)n, part, vec);
    hipLaunchKernelGGL(rmsnorm_apply_k, dim3(g), dim3(256), 0, st, x, w, out, (int64_t)n, eps,
                       (const float *)part, vec);
  } else {
    launch_one_block<RmsnormOne>(n, st, x, w, out, n, eps);
  }
  SIMP_HIP(hipGetLastError());
  return SIMP_RT_OK;
}

}  // namespace simp

using namespace simp;

extern "C" {

int32_t simp_rt_rmsnorm(const float *in_alloc, const float *in, int64_t in_off, int64_t in_size,
                        int64_t in_stride, const float *w_alloc, const float *w, int64_t w_doff,
                        int64_t w_size, int64_t w_stride, float *out_alloc, float *out,
                        int64_t out_off, int64_t out_size, int64_t out_stride, int64_t size,
                        double epsilon, int64_t weight_offset) {
  (void)in_alloc; (void)w_alloc; (void)out_alloc;
  int rc;
  if ((rc = check_desc1("input", in, in_off, in_size, in_stride))) return rc;
  if ((rc = check_desc1("weight", w, w_doff, w_size, w_stride))) return rc;
  if ((rc = check_desc1("output", out, out_off, out_size, out_stride))) return rc;
  if (size < 0 || weight_offset < 0 || size > in_size || size > out_size ||
      weight_offset + size > w_size)
    return set_error(SIMP_RT_EINVAL, "rmsnorm: size %lld / weight_offset %lld out of range",
                     (long long)size, (long long)weight_offset);
  if (size == 0) return SIMP_RT_OK;
  if (size > INT32_MAX) return set_error(SIMP_RT_EUNSUPPORTED, "rmsnorm: size above 2^31-1");
  Operand oi, ow, oo;
  if ((rc = oi.bind(in + in_off, 4 * (size_t)size, Operand::kIn, "input"))) return rc;
  if ((rc = ow.bind(w + w_doff + weight_offset, 4 * (size_t)size, Operand::kIn, "weight"))) return rc;
  if ((rc = oo.bind(out + out_off, 4 * (size_t)size, Operand::kOut, "output"))) return rc;
  if ((rc = launch_rmsnorm((const float *)oi.dev(), (const float *)ow.dev(), (float *)oo.dev(),
                           (int)size, (float)epsilon, cur_stream())))
    return rc;
  Operand *ops[] = {&oi, &ow, &oo};
  return finish(ops, 3);
}

int32_t simp_rt_softmax(const float *in_alloc, const float *in, int64_t in_doff, int64_t in_size,
                        int64_t in_stride, float *out_alloc, float *out, int64_t out_doff,
                        int64_t out_size, int64_t out_stride, int64_t size, int64_t input_offset,
                        int64_t output_offset) {
  (void)in_alloc; (void)out_alloc;
  int rc;
  if ((rc = check_desc1("input", in, in_doff, in_size, in_stride))) return rc;
  if ((rc = check_desc1("output", out, out_doff, out_size, out_stride))) return rc;
  if (size < 0 || input_offset < 0 || output_offset < 0 || input_offset + size > in_size ||
      output_offset + size > out_size)
    return set_error(SIMP_RT_EINVAL, "softmax: size/offsets out of range");
  if (size == 0) return SIMP_RT_OK;
  if (size > INT32_MAX) return set_error(SIMP_RT_EUNSUPPORTED, "softmax: size above 2^31-1");
  Operand oi, oo;
  if ((rc = oi.bind(in + in_doff + input_offset, 4 * (size_t)size, Operand::kIn, "input"))) return rc;
  if ((rc = oo.bind(out + out_doff + output_offset, 4 * (size_t)size, Operand::kOut, "output"))) return rc;
  hipStream_t st = cur_stream();
  if (size >= kBigNorm) {
    const unsigned g = big_grid(size);
    float2 *part = nullptr;
    if ((rc = workspace(st, sizeof(float2) * g, (void **)&part, 4))) return rc;
    const bool vec = (((uintptr_t)oi.dev() | (uintptr_t)oo.dev()) & 15) == 0;
    hipLaunchKernelGGL(softmax_parts_k, dim3(g), dim3(256), 0, st, (const float *)oi.dev(),
                       (int64_t)size, part, vec);
    hipLaunchKernelGGL(softmax_apply_k, dim3(g), dim3(256), 0, st, (const float *)oi.dev(),
                       (float *)oo.dev(), (int64_t)size, (const float2 *)part, vec);
  } else {
    launch_one_block<SoftmaxOne>((int)size, st, (const float *)oi.dev(), (float *)oo.dev(),
                                 (int)size);
  }
  SIMP_HIP(hipGetLastError());
  Operand *ops[] = {&oi, &oo};
  return finish(ops, 2);
}

int32_t simp_rt_silu(const float *in_alloc, const float *in, int64_t in_off, int64_t in_size,
                     int64_t in_stride, float *out_alloc, float *out, int64_t out_off,
                     int64_t out_size, int64_t out_stride, int64_t size) {
  (void)in_alloc; (void)out_alloc;
  int rc;
  if ((rc = check_desc1("input", in, in_off, in_size, in_stride))) return rc;
  if ((rc = check_desc1("output", out, out_off, out_size, out_stride))) return rc;
  if (size < 0 || size > in_size || size > out_size)
    return set_error(SIMP_RT_EINVAL, "silu: size %lld out of range", (long long)size);
  if (size == 0) return SIMP_RT_OK;
  Operand oi, oo;
  if ((rc = oi.bind(in + in_off, 4 * (size_t)size, Operand::kIn, "input"))) return rc;
  if ((rc = oo.bind(out + out_off, 4 * (size_t)size, Operand::kOut, "output"))) return rc;
  if (size >= kBigNorm && (((uintptr_t)oi.dev() | (uintptr_t)oo.dev()) & 15) == 0)
    hipLaunchKernelGGL(silu_big_k, dim3(big_grid(size)), dim3(256), 0, cur_stream(),
                       (const float *)oi.dev(), (float *)oo.dev(), size);
  else
    hipLaunchKernelGGL(silu_k, dim3(grid_for(size)), dim3(256), 0, cur_stream(),
                       (const float *)oi.dev(), (float *)oo.dev(), size);
  SIMP_HIP(hipGetLastError());
  Operand *ops[] = {&oi, &oo};
  return finish(ops, 2);
}

int32_t simp_rt_swiglu(const float *g_alloc, const float *gate, int64_t g_off, int64_t g_size,
                       int64_t g_stride, const float *u_alloc, const float *up, int64_t u_off,
                       int64_t u_size, int64_t u_stride, float *o_alloc, float *out,
                       int64_t o_off, int64_t o_size, int64_t o_stride, int64_t size) {
  (void)g_alloc; (void)u_alloc; (void)o_alloc;
  int rc;
  if ((rc = check_desc1("gate", gate, g_off, g_size, g_stride))) return rc;
  if ((rc = check_desc1("up", up, u_off, u_size, u_stride))) return rc;
  if ((rc = check_desc1("out", out, o_off, o_size, o_stride))) return rc;
  if (size < 0 || size > g_size || size > u_size || size > o_size)
    return set_error(SIMP_RT_EINVAL, "swiglu: size %lld out of range", (long long)size);
  if (size == 0) return SIMP_RT_OK;
  Operand og, ou, oo;
  if ((rc = og.bind(gate + g_off, 4 * (size_t)size, Operand::kIn, "gate"))) return rc;
  if ((rc = ou.bind(up + u_off, 4 * (size_t)size, Operand::kIn, "up"))) return rc;
  if ((rc = oo.bind(out + o_off, 4 * (size_t)size, Operand::kOut, "out"))) return rc;
  hipLaunchKernelGGL(swiglu_k, dim3(grid_for(size)), dim3(256), 0, cur_stream(),
                     (const float *)og.dev(), (const float *)ou.dev(), (float *)oo.dev(), size);
  SIMP_HIP(hipGetLastError());
  Operand *ops[] = {&og, &ou, &oo};
  return finish(ops, 3);
}

int32_t simp_rt_rope(float *q_alloc, float *q, int64_t q_off, int64_t q_size, int64_t q_stride,
                     float *k_alloc, float *k, int64_t k_off, int64_t k_size, int64_t k_stride,
                     int64_t dim, int64_t kv_dim, int64_t head_size, int64_t pos, double theta) {
  (void)q_alloc; (void)k_alloc;
  int rc;
  if ((rc = check_desc1("q", q, q_off, q_size, q_stride))) return rc;
  if ((rc = check_desc1("k", k, k_off, k_size, k_stride))) return rc;
  if (dim <= 0 || dim % 2 || kv_dim < 0 || kv_dim > dim || head_size <= 0 || pos < 0 ||
      dim > q_size || kv_dim > k_size || dim > INT32_MAX || pos > INT32_MAX)
    return set_error(SIMP_RT_EINVAL, "rope: bad dim/kv_dim/head_size/pos");
  Operand oq, ok;
  if ((rc = oq.bind(q + q_off, 4 * (size_t)dim, Operand::kInOut, "q"))) return rc;
  if ((rc = ok.bind(k + k_off, 4 * (size_t)kv_dim, Operand::kInOut, "k"))) return rc;
  hipLaunchKernelGGL(rope_k, dim3((unsigned)cdiv(dim / 2, 256)), dim3(256), 0, cur_stream(),
                     (float *)oq.dev(), (float *)ok.dev(), (int)dim, (int)kv_dim, (int)head_size,
                     (int)pos, (float)theta);
  SIMP_HIP(hipGetLastError());
  Operand *ops[] = {&oq, &ok};
  return finish(ops, 2);
}

}  // extern "C"
