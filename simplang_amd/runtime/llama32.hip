// llama32.hip -- llama32_forward: the int8 LLaMA-3.2 program
// (examples/llama2/llama32_1b_int8_tensor.sl:16-305, bound by
// examples/llama2/bench_llama32_1b_int8.cpp:36-61,201-230) as a model-level
// export with the compiled program's signature.
//
// The program's arithmetic, with SimpLang's typing (float literals f32,
// integer literals i64): x = (float)x_i8; per layer an RMSNorm, xb*127 clamped
// and truncated to i8, Q/K/V = tensor_matmul_nt (i8 x i8 -> i32), K/V cached as
// (i8)(v / 256), per head fp32 scores / 8, softmax, attn_out = (i32) sum p*v,
// Wo on (i8)clamp(attn_out / 256), x += Wo / 65536, FFN RMSNorm, Gate/Up on the
// re-quantized xb, ffn_hb = (i8)(silu(g/65536) * (u/65536) * 127), x += Down /
// 65536, final RMSNorm and an fp32 classifier.  The RoPE loop of the program
// discards its results (:123-140) and is not run.
//
// Kernels per layer: one int8 GEMV over Wq|Wk|Wv with the attention RMSNorm
// and quantization in its prologue and the K/V cache store in its epilogue,
// attention (one block per head), Wo GEMV adding into x, one paired W1|W3 GEMV
// (FFN RMSNorm + quantization in its prologue) writing ffn_hb, W2 GEMV adding
// into x.
// The int8 GEMVs are HBM-bound: each wave reads whole rows of W_t as 1 KB
// coalesced lines, x sits in registers, v_dot4_i32_i8 accumulates exactly, so
// every integer the program computes is reproduced bit for bit.
//
// State: the KV cache lives on the device (authoritative across calls); each
// call writes the new row of every layer back to the caller's k_cache/v_cache,
// and writes logits, x_fp32, xb_fp32 and attn_out (the last layer's, as the
// program leaves it).  att_scores, att_probs, xb_i8 and ffn_hb are the
// program's per-layer scratch and are not written.
#include <algorithm>
#include <cmath>
#include <limits>
#include <map>
#include <mutex>
#include <vector>

#include "rt_device.h"
#include "rt_internal.h"

namespace simp {
namespace {

enum L32Out { kL32QKV = 0, kL32Resid = 1, kL32Pair = 2 };

// (i8) of an fp32 value as the reference's x86 build lowers fptosi to i8:
// truncate to i32 (0x80000000 for NaN or out of range), keep the low byte.
__device__ __forceinline__ int8_t l32_fptosi_i8(float v) {
  if (!(v > -2147483648.0f && v < 2147483648.0f)) return 0;
  return (int8_t)(uint8_t)(uint32_t)(int32_t)v;
}

// val = v * 127; clamp to [-128, 127]; (i8)val (:96-102, :235-242)
__device__ __forceinline__ int8_t l32_quant127(float v) {
  float val = v * 127.0f;
  val = val > 127.0f ? 127.0f : val;
  val = val < -128.0f ? -128.0f : val;
  return (int8_t)(int32_t)val;
}

__device__ __forceinline__ int32_t dot16(uint4 a, uint4 b, int32_t acc) {
  acc = __builtin_amdgcn_sdot4((int)a.x, (int)b.x, acc, false);
  acc = __builtin_amdgcn_sdot4((int)a.y, (int)b.y, acc, false);
  acc = __builtin_amdgcn_sdot4((int)a.z, (int)b.z, acc, false);
  acc = __builtin_amdgcn_sdot4((int)a.w, (int)b.w, acc, false);
  return acc;
}

// Sum over the wave, every lane gets it: DPP quad and row moves, then the
// rows and halves swapped by v_permlane{16,32}_swap (VALU only; integer sums,
// so the order does not matter).
template <int CTRL>
__device__ __forceinline__ int32_t idpp(int32_t v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ int32_t wave_isum(int32_t v) {
  v += idpp<kDppXor1>(v);
  v += idpp<kDppXor2>(v);
  v += idpp<kDppHalfMirror>(v);
  v += idpp<kDppMirror>(v);
  float a = __int_as_float(v), b = a;
  permlane16_swap(a, b);
  v = __float_as_int(a) + __float_as_int(b);
  a = b = __int_as_float(v);
  permlane32_swap(a, b);
  return __float_as_int(a) + __float_as_int(b);
}

// x = (float)x_i8 (:79-83)
__global__ void __launch_bounds__(256)
    l32_embed_k(const int8_t *__restrict__ xi, float *__restrict__ x, int dim) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < dim) x[i] = (float)xi[i];
}

// RMSNorm (the rmsnorm builtin: (x / sqrt(sum x^2 / n + eps)) * w) of x into xb,
// and, when xq is given, its i8 quantization.  One 1024-thread block.
__global__ void __launch_bounds__(1024)
    l32_norm_k(const float *__restrict__ x, const float *__restrict__ w, float *__restrict__ xb,
               int8_t *__restrict__ xq, int dim, float eps) {
  __shared__ float scratch[16];
  float ss = 0.f;
  for (int i = threadIdx.x; i < dim; i += 1024) ss = fmaf(x[i], x[i], ss);
  ss = block_sum(ss, scratch);
  const float rms = sqrtf(ss / (float)dim + eps);
  for (int i = threadIdx.x; i < dim; i += 1024) {
    const float v = (x[i] / rms) * w[i];
    if (xb) xb[i] = v;
    if (xq) xq[i] = l32_quant127(v);
  }
}

// Rows of up to three int8 matrices W_t[rows, K] against x[K] (i8, K % 16 == 0),
// R rows per wave, C 16-byte chunks per lane (K <= 1024 * C).
//   kL32QKV   rows of s0 -> q[r] (i32); of s1 -> krow[r] = (i8)(acc / 256);
//             of s2 -> vrow[r] = (i8)(acc / 256)           (:104-121, :142-151)
//   kL32Resid rows of s0 -> x[r] += (float)acc / 65536     (:225-229, :275-279)
//   kL32Pair  row r of s0 (W1) and of s1 (W3): hb[r] = (i8)(silu(g / 65536) *
//             (u / 65536) * 127)                            (:245-267)
struct L32Segs {
  const int8_t *w[3];
  int rows[3];
};

//   NORM      the block first forms xq itself from xn: the RMSNorm of xn with
//             weight nw, quantized as l32_quant127 (the l32_norm_k arithmetic;
//             xq is then unused).  The weight loads are issued before the norm,
//             which waits only on xn; xq sits in K bytes of dynamic LDS.
template <int C, int R, int MODE, bool NORM>
__global__ void __launch_bounds__(256)
    l32_gemv_k(L32Segs sg, const int8_t *__restrict__ xq, int K, int32_t *__restrict__ q,
               int8_t *__restrict__ krow, int8_t *__restrict__ vrow, float *__restrict__ x,
               int8_t *__restrict__ hb, const float *__restrict__ xn,
               const float *__restrict__ nw, float eps) {
  constexpr int NM = MODE == kL32Pair ? 2 : 1;  // matrices read per row
  extern __shared__ uint4 xs[];                 // NORM: xq, K bytes
  __shared__ float scratch[16];
  const int lane = threadIdx.x & 63;
  const int total = MODE == kL32QKV ? sg.rows[0] + sg.rows[1] + sg.rows[2] : sg.rows[0];
  const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
  const bool active = row0 < total;  // uniform per wave
  if (!NORM && !active) return;      // (NORM: every wave takes part in the norm)
  const int nch = K >> 4;
  // NORM: element quads 4 (tid + 256 j) of xn and nw (K <= 1024 C)
  float4 xf[NORM ? C : 1], wf[NORM ? C : 1];
  if constexpr (NORM) {
#pragma unroll
    for (int j = 0; j < C; j++) {
      const int i4 = threadIdx.x + 256 * j;
      const bool in = 4 * i4 < K;
      xf[j] = in ? *(const float4 *)(xn + 4 * i4) : make_float4(0.f, 0.f, 0.f, 0.f);
      wf[j] = in ? *(const float4 *)(nw + 4 * i4) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  uint4 xv[C];
  if constexpr (!NORM) {
#pragma unroll
    for (int j = 0; j < C; j++) {
      const int c = lane + 64 * j;
      xv[j] = c < nch ? *(const uint4 *)(xq + 16 * c) : make_uint4(0, 0, 0, 0);
    }
  }
  uint4 wv[NM][R][C];
  if (active) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int row = min(row0 + r, total - 1);
      const int8_t *base[NM];
      if constexpr (MODE == kL32QKV) {
        const int s = row < sg.rows[0] ? 0 : (row < sg.rows[0] + sg.rows[1] ? 1 : 2);
        const int rr = s == 0 ? row : (s == 1 ? row - sg.rows[0] : row - sg.rows[0] - sg.rows[1]);
        base[0] = sg.w[s] + (int64_t)rr * K;
      } else {
#pragma unroll
        for (int mtx = 0; mtx < NM; mtx++) base[mtx] = sg.w[mtx] + (int64_t)row * K;
      }
#pragma unroll
      for (int mtx = 0; mtx < NM; mtx++)
#pragma unroll
        for (int j = 0; j < C; j++) {
          const int c = lane + 64 * j;
          wv[mtx][r][j] = c < nch ? *(const uint4 *)(base[mtx] + 16 * c) : make_uint4(0, 0, 0, 0);
        }
    }
  }
  if constexpr (NORM) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < C; j++) {
      ss = fmaf(xf[j].x, xf[j].x, ss);
      ss = fmaf(xf[j].y, xf[j].y, ss);
      ss = fmaf(xf[j].z, xf[j].z, ss);
      ss = fmaf(xf[j].w, xf[j].w, ss);
    }
    ss = block_sum_lds(ss, scratch);
    const float rms = sqrtf(ss / (float)K + eps);
    uint32_t *xs32 = (uint32_t *)xs;
#pragma unroll
    for (int j = 0; j < C; j++) {
      const int i4 = threadIdx.x + 256 * j;
      if (4 * i4 < K) {
        const uint32_t b0 = (uint8_t)l32_quant127((xf[j].x / rms) * wf[j].x);
        const uint32_t b1 = (uint8_t)l32_quant127((xf[j].y / rms) * wf[j].y);
        const uint32_t b2 = (uint8_t)l32_quant127((xf[j].z / rms) * wf[j].z);
        const uint32_t b3 = (uint8_t)l32_quant127((xf[j].w / rms) * wf[j].w);
        xs32[i4] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
      }
    }
    lds_barrier();
    if (!active) return;
#pragma unroll
    for (int j = 0; j < C; j++) {
      const int c = lane + 64 * j;
      xv[j] = c < nch ? xs[c] : make_uint4(0, 0, 0, 0);
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++) {
    int32_t acc[NM];
#pragma unroll
    for (int mtx = 0; mtx < NM; mtx++) {
      int32_t a = 0;
#pragma unroll
      for (int j = 0; j < C; j++) a = dot16(wv[mtx][r][j], xv[j], a);
      acc[mtx] = wave_isum(a);
    }
    const int row = row0 + r;
    if (lane != 0 || row >= total) continue;
    if constexpr (MODE == kL32QKV) {
      if (row < sg.rows[0]) q[row] = acc[0];
      else if (row < sg.rows[0] + sg.rows[1]) krow[row - sg.rows[0]] = (int8_t)(uint8_t)(uint32_t)(acc[0] / 256);
      else vrow[row - sg.rows[0] - sg.rows[1]] = (int8_t)(uint8_t)(uint32_t)(acc[0] / 256);
    } else if constexpr (MODE == kL32Resid) {
      x[row] = x[row] + (float)acc[0] / 65536.0f;
    } else {
      const float gate_f = (float)acc[0] / 65536.0f;
      const float silu = gate_f / (1.0f + expf(0.0f - gate_f));
      const float up_f = (float)acc[1] / 65536.0f;
      hb[row] = l32_fptosi_i8(silu * up_f * 127.0f);
    }
  }
}

// Attention of one layer, one block of 8 waves per head (:161-216).
//   * Scores: LPP lanes per position (head_size / 16 chunks of 16 bytes,
//     rounded up to a power of two), 16 dims per lane with the program's fp32
//     product then sum (no fused multiply-add) over them, the LPP partial sums
//     added across lanes (DPP), / 8.  q is converted once into registers; the
//     K rows of four passes are loaded before any is summed.
//   * Softmax over pos + 1 scores: wave then block maximum and sum (the
//     waves' values combined in wave order through LDS), p = e / sum.
//   * V sum: head_size / 4 lanes per row (4 dims each, one dword load), row
//     group g of wave w taking positions t = 8 RPW s + RPW w + g; the 8 RPW
//     partial sums of a dim are added in (wave, group) order.
//   * Long contexts: block (h, s) takes positions [CH s, CH s + CH) of head
//     h (grid y = nsplit chunks); with nsplit > 1 it writes its chunk's
//     maximum score, sum of exponentials and normalised V sum to ws[h][s] and
//     l32_attn_combine_k forms the head's output.  One CU per head moved
//     512 KB of K and V at pos 4095 (34 us per launch).
// Only the summation order differs from the program's sequential loops (one
// thread per position and a 16-dim chain per thread, measured 12.9 us per
// launch at the 1B shape's positions 128-191 and 38 us at 4095).
// attn_out = (i32) sum; xq = its i8 quantization (float)attn_out / 256,
// clamped.  Head size and kv_dim multiples of 16, head size <= 256.
// LDS: min(pos + 1, CH) floats (dynamic, at most 47 KB) + 8 KB.
constexpr int kL32AttnWaves = 8;
__global__ void __launch_bounds__(64 * kL32AttnWaves)
    l32_attn_k(const int32_t *__restrict__ Q, const int8_t *__restrict__ kc,
               const int8_t *__restrict__ vc, int32_t *__restrict__ attn_out,
               int8_t *__restrict__ xq, float *__restrict__ ws, int pos, int kv, int hs,
               int n_rep, int chunk) {
  constexpr int NW = kL32AttnWaves, U = 4;
  extern __shared__ float att[];      // the chunk's scores, then probabilities
  __shared__ float red[NW * 256];     // V partial sums: NW * RPW rows of hs (RPW * hs <= 256)
  __shared__ float wv[2][NW];         // per-wave maximum and sum
  const int h = blockIdx.x, kho = (h / n_rep) * hs;
  // this block's positions [t_lo, t_lo + n); att[] is indexed from t_lo
  const int t_lo = blockIdx.y * chunk, n = min(pos + 1 - t_lo, chunk);
  kc += (int64_t)t_lo * kv;
  vc += (int64_t)t_lo * kv;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hc = hs >> 4;  // 16-byte chunks per row
  int lpp = 1;
  while (lpp < hc) lpp <<= 1;  // lanes per position: 1, 2, 4, 8 or 16
  const int ppw = 64 / lpp, ppb = NW * ppw;  // positions per wave and per block pass
  const int c = lane & (lpp - 1);
  const bool cl = c < hc;
  float qv[16];
#pragma unroll
  for (int e = 0; e < 16; e++) qv[e] = cl ? (float)Q[h * hs + 16 * c + e] : 0.f;
  // 1. scores, U passes of loads at a time
  for (int t0 = wave * ppw + lane / lpp; t0 < n; t0 += U * ppb) {
    uint4 kr[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int t = t0 + u * ppb;
      kr[u] = (cl && t < n) ? *(const uint4 *)(kc + (int64_t)t * kv + kho + 16 * c)
                            : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const uint32_t wd[4] = {kr[u].x, kr[u].y, kr[u].z, kr[u].w};
      float sc = 0.f;
#pragma unroll
      for (int e = 0; e < 16; e++)
        sc = __fadd_rn(sc, __fmul_rn(qv[e], (float)(int8_t)(uint8_t)(wd[e >> 2] >> (8 * (e & 3)))));
      // partial sums of the position's lpp lanes (lanes of one 16-lane row)
      if (lpp > 1) sc += dpp_mov<kDppXor1>(sc);
      if (lpp > 2) sc += dpp_mov<kDppXor2>(sc);
      if (lpp > 4) sc += dpp_mov<kDppHalfMirror>(sc);
      if (lpp > 8) sc += dpp_mov<kDppMirror>(sc);
      const int t = t0 + u * ppb;
      if (c == 0 && t < n) att[t] = sc / 8.0f;
    }
  }
  __syncthreads();
  // 2. softmax
  float m = -INFINITY;
  for (int t = tid; t < n; t += 64 * NW) m = fmaxf(m, att[t]);
  m = wave_max_dpp(m);
  if (lane == 0) wv[0][wave] = m;
  __syncthreads();
  m = wv[0][0];
#pragma unroll
  for (int w = 1; w < NW; w++) m = fmaxf(m, wv[0][w]);
  float l = 0.f;
  for (int t = tid; t < n; t += 64 * NW) {
    const float e = expf(att[t] - m);
    att[t] = e;
    l += e;
  }
  l = wave_sum_dpp(l);
  if (lane == 0) wv[1][wave] = l;
  __syncthreads();
  l = 0.f;
#pragma unroll
  for (int w = 0; w < NW; w++) l += wv[1][w];
  for (int t = tid; t < n; t += 64 * NW) att[t] = att[t] / l;
  __syncthreads();
  // 3. V sum
  const int lpr = hs >> 2, rpw = 64 / lpr;  // lanes per V row (4 dims each), rows per wave
  const int dq = lane % lpr, rg = lane / lpr;
  if (rg < rpw) {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    const int step = NW * rpw;
    for (int t0 = wave * rpw + rg; t0 < n; t0 += U * step) {
      uint32_t vr[U];
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int t = t0 + u * step;
        vr[u] = t < n ? *(const uint32_t *)(vc + (int64_t)t * kv + kho + 4 * dq) : 0u;
      }
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int t = t0 + u * step;
        if (t < n) {
          const float p = att[t];
#pragma unroll
          for (int e = 0; e < 4; e++)
            acc[e] = __fadd_rn(acc[e], __fmul_rn(p, (float)(int8_t)(uint8_t)(vr[u] >> (8 * e))));
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 4; e++) red[(wave * rpw + rg) * hs + 4 * dq + e] = acc[e];
  }
  __syncthreads();
  for (int dd = tid; dd < hs; dd += 64 * NW) {
    float v = red[dd];
    const int parts = NW * rpw;
#pragma unroll 8
    for (int pp = 1; pp < parts; pp++) v = __fadd_rn(v, red[pp * hs + dd]);
    if (gridDim.y > 1) {  // the chunk's (max, sum, normalised V sum) for the combine
      float *w = ws + ((int64_t)h * gridDim.y + blockIdx.y) * (hs + 2);
      w[dd] = v;
      if (dd == 0) {
        w[hs] = m;
        w[hs + 1] = l;
      }
      continue;
    }
    const int32_t a = (int32_t)v;
    attn_out[h * hs + dd] = a;
    float s = (float)a * 1.0f / 256.0f;
    s = s > 127.0f ? 127.0f : s;
    s = s < -128.0f ? -128.0f : s;
    xq[h * hs + dd] = (int8_t)(int32_t)s;
  }
}

// Combines the nsplit chunks of l32_attn_k for head blockIdx.x, thread d:
// out = sum_s w_s o_s / sum_s w_s with w_s = e^(m_s - M) l_s, M = max_s m_s
// (o_s the chunk's normalised V sum), then attn_out and xq as l32_attn_k.
// The chunks' (m, l) go through LDS (one load each) and each element requests
// its chunks' o values eight at a time; sums in chunk order.  LDS: nsplit
// float2.
__global__ void __launch_bounds__(256)
    l32_attn_combine_k(const float *__restrict__ ws, int32_t *__restrict__ attn_out,
                       int8_t *__restrict__ xq, int hs, int nsplit) {
  extern __shared__ float2 mls[];
  const int h = blockIdx.x, st = hs + 2;
  const float *w = ws + (int64_t)h * nsplit * st;
  for (int s = threadIdx.x; s < nsplit; s += blockDim.x) mls[s] = make_float2(w[s * st + hs], w[s * st + hs + 1]);
  __syncthreads();
  float M = -INFINITY;
  for (int s = 0; s < nsplit; s++) M = fmaxf(M, mls[s].x);
  for (int dd = threadIdx.x; dd < hs; dd += 256) {
    float num = 0.f, den = 0.f;
    for (int s0 = 0; s0 < nsplit; s0 += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) v[u] = s0 + u < nsplit ? w[(s0 + u) * st + dd] : 0.f;
#pragma unroll
      for (int u = 0; u < 8; u++) {
        if (s0 + u < nsplit) {
          const float f = expf(mls[s0 + u].x - M) * mls[s0 + u].y;
          num = fmaf(f, v[u], num);
          den += f;
        }
      }
    }
    const int32_t a = (int32_t)(num / den);
    attn_out[h * hs + dd] = a;
    float v = (float)a * 1.0f / 256.0f;
    v = v > 127.0f ? 127.0f : v;
    v = v < -128.0f ? -128.0f : v;
    xq[h * hs + dd] = (int8_t)(int32_t)v;
  }
}

// Positions per attention block: longer contexts split over blocks.
constexpr int kL32AttnChunk = 512;

struct L32Model {
  int64_t dim, hid, L, nh, nkv, V, S, hs, kv;
  const float *rms_att, *rms_ffn, *rms_final, *wcls;
  const int8_t *wq, *wk, *wv, *wo, *w1, *w2, *w3;
  float *x = nullptr, *xb = nullptr, *logits = nullptr;
  int8_t *xi = nullptr, *xq = nullptr, *hq = nullptr, *kc = nullptr, *vc = nullptr;
  int32_t *q = nullptr, *attn = nullptr;
  float *attn_ws = nullptr;  // l32_attn_k chunk results: nh * cdiv(S, chunk) * (hs + 2)
  float *first = nullptr;    // pinned: logits[0], the call's return value
  ExportWeights weights;
  KvState kvs;
  uint64_t last_use = 0;
};

void l32_free(L32Model &m) {
  for (void *p : {(void *)m.x, (void *)m.xb, (void *)m.logits, (void *)m.xi, (void *)m.xq,
                  (void *)m.hq, (void *)m.kc, (void *)m.vc, (void *)m.q, (void *)m.attn,
                  (void *)m.attn_ws})
    if (p) (void)hipFree(p);
  m.x = m.xb = m.logits = nullptr;
  m.xi = m.xq = m.hq = m.kc = m.vc = nullptr;
  m.q = m.attn = nullptr;
  m.attn_ws = nullptr;
  if (m.first) (void)hipHostFree(m.first);
  m.first = nullptr;
  m.weights.release();
}

int l32_alloc(L32Model &m) {
  const size_t cache = (size_t)(m.L * m.S * m.kv);
  struct B { void **p; size_t bytes; };
  const B bufs[] = {{(void **)&m.x, 4 * (size_t)m.dim},    {(void **)&m.xb, 4 * (size_t)m.dim},
                    {(void **)&m.logits, 4 * (size_t)m.V}, {(void **)&m.xi, (size_t)m.dim},
                    {(void **)&m.xq, (size_t)m.dim},       {(void **)&m.hq, (size_t)m.hid},
                    {(void **)&m.kc, cache},               {(void **)&m.vc, cache},
                    {(void **)&m.q, 4 * (size_t)m.dim},    {(void **)&m.attn, 4 * (size_t)m.dim},
                    {(void **)&m.attn_ws,
                     4 * (size_t)(m.nh * cdiv(m.S, kL32AttnChunk) * (m.hs + 2))}};
  for (const B &b : bufs) {
    if (hipMalloc(b.p, std::max<size_t>(b.bytes, 16)) != hipSuccess)
      return set_error(SIMP_RT_ENOMEM, "llama32_forward: device buffers");
    SIMP_HIP(hipMemset(*b.p, 0, b.bytes));
  }
  if (hipHostMalloc((void **)&m.first, 64, hipHostMallocDefault) != hipSuccess) {
    m.first = nullptr;
    return set_error(SIMP_RT_ENOMEM, "llama32_forward: pinned return slot");
  }
  return SIMP_RT_OK;
}

// One int8 GEMV launch: C chunks per lane from K, R rows per wave.  With xn
// (and nw) given, the kernel forms xq as the RMSNorm of xn quantized.
template <int MODE, int R>
int l32_gemv_r(const L32Segs &sg, int total, int K, const int8_t *xq, int32_t *q, int8_t *krow,
               int8_t *vrow, float *x, int8_t *hb, hipStream_t st, const float *xn,
               const float *nw, float eps) {
  const int C = (int)cdiv(K / 16, 64);
  const unsigned grid = (unsigned)cdiv(total, 4 * R);
  const size_t lds = xn ? (size_t)K : 0;
#define L32G(CC)                                                                              \
  case CC:                                                                                    \
    if (xn)                                                                                   \
      hipLaunchKernelGGL((l32_gemv_k<CC, R, MODE, true>), dim3(grid), dim3(256), lds, st, sg, \
                         xq, K, q, krow, vrow, x, hb, xn, nw, eps);                           \
    else                                                                                      \
      hipLaunchKernelGGL((l32_gemv_k<CC, R, MODE, false>), dim3(grid), dim3(256), 0, st, sg,  \
                         xq, K, q, krow, vrow, x, hb, xn, nw, eps);                           \
    break;
  switch (C) {
    L32G(1) L32G(2) L32G(4) L32G(8) L32G(16)
    default:
      return set_error(SIMP_RT_EUNSUPPORTED, "llama32_forward: K=%d per matrix row", K);
  }
#undef L32G
  SIMP_HIP(hipGetLastError());
  return SIMP_RT_OK;
}

// Two rows per wave where that gives whole rounds of blocks (a multiple of
// the CU count, or many rounds), else one: a count just past a round leaves
// some CUs a second block (the 1B QKV: 384 blocks of two rows, 768 of one).
template <int MODE>
int l32_gemv(const L32Segs &sg, int total, int K, const int8_t *xq, int32_t *q, int8_t *krow,
             int8_t *vrow, float *x, int8_t *hb, hipStream_t st, const float *xn = nullptr,
             const float *nw = nullptr, float eps = 0.f) {
  const int64_t cus = num_cus(), g2 = cdiv(total, 8);
  if (MODE != kL32Pair && (g2 % cus == 0 || g2 >= 8 * cus))
    return l32_gemv_r<MODE, MODE == kL32Pair ? 1 : 2>(sg, total, K, xq, q, krow, vrow, x, hb, st,
                                                      xn, nw, eps);
  return l32_gemv_r<MODE, 1>(sg, total, K, xq, q, krow, vrow, x, hb, st, xn, nw, eps);
}

int l32_step(L32Model &m, int64_t pos, hipStream_t st) {
  const int dim = (int)m.dim, hid = (int)m.hid, kv = (int)m.kv;
  const float eps = 1e-5f;  // the program's 0.00001 (:93, :232, :287)
  hipLaunchKernelGGL(l32_embed_k, dim3((unsigned)cdiv(dim, 256)), dim3(256), 0, st,
                     (const int8_t *)m.xi, m.x, dim);
  int rc;
  const int nsplit = (int)cdiv(pos + 1, kL32AttnChunk);
  const size_t attn_lds = sizeof(float) * (size_t)std::min<int64_t>(pos + 1, kL32AttnChunk);
  for (int64_t l = 0; l < m.L; l++) {
    int8_t *kc = m.kc + l * m.S * kv, *vc = m.vc + l * m.S * kv;
    L32Segs s{};
    s.w[0] = m.wq + l * m.dim * m.dim;
    s.w[1] = m.wk + l * m.kv * m.dim;
    s.w[2] = m.wv + l * m.kv * m.dim;
    s.rows[0] = dim;
    s.rows[1] = kv;
    s.rows[2] = kv;
    if ((rc = l32_gemv<kL32QKV>(s, dim + 2 * kv, dim, nullptr, m.q, kc + pos * kv,
                                vc + pos * kv, nullptr, nullptr, st, m.x, m.rms_att + l * dim,
                                eps)))
      return rc;
    hipLaunchKernelGGL(l32_attn_k, dim3((unsigned)m.nh, (unsigned)nsplit),
                       dim3(64 * kL32AttnWaves), attn_lds, st, (const int32_t *)m.q,
                       (const int8_t *)kc, (const int8_t *)vc, m.attn, m.xq, m.attn_ws,
                       (int)pos, kv, (int)m.hs, (int)(m.nh / m.nkv), kL32AttnChunk);
    if (nsplit > 1)
      hipLaunchKernelGGL(l32_attn_combine_k, dim3((unsigned)m.nh), dim3(256),
                         sizeof(float2) * (size_t)nsplit, st, (const float *)m.attn_ws, m.attn,
                         m.xq, (int)m.hs, nsplit);
    s = L32Segs{};
    s.w[0] = m.wo + l * m.dim * m.dim;
    s.rows[0] = dim;
    if ((rc = l32_gemv<kL32Resid>(s, dim, dim, m.xq, nullptr, nullptr, nullptr, m.x, nullptr, st)))
      return rc;
    s = L32Segs{};
    s.w[0] = m.w1 + l * m.hid * m.dim;
    s.w[1] = m.w3 + l * m.hid * m.dim;
    s.rows[0] = hid;
    if ((rc = l32_gemv<kL32Pair>(s, hid, dim, nullptr, nullptr, nullptr, nullptr, nullptr, m.hq,
                                 st, m.x, m.rms_ffn + l * dim, eps)))
      return rc;
    s = L32Segs{};
    s.w[0] = m.w2 + l * m.dim * m.hid;
    s.rows[0] = dim;
    if ((rc = l32_gemv<kL32Resid>(s, dim, hid, m.hq, nullptr, nullptr, nullptr, m.x, nullptr, st)))
      return rc;
  }
  hipLaunchKernelGGL(l32_norm_k, dim3(1), dim3(1024), 0, st, (const float *)m.x, m.rms_final,
                     m.xb, (int8_t *)nullptr, dim, eps);
  SIMP_HIP(hipGetLastError());
  return launch_matmul_f32(m.wcls, dim, m.xb, 1, m.logits, 1, (int)m.V, 1, dim, 0.f, st);
}

std::mutex g_l32_mu;
std::map<std::vector<int64_t>, L32Model> g_l32;
uint64_t g_l32_clock = 0;
constexpr size_t kMaxL32Entries = 4;

}  // namespace

void l32_cache_clear() {
  std::lock_guard<std::mutex> lk(g_l32_mu);
  if (!g_l32.empty()) (void)hipDeviceSynchronize();
  for (auto &kv : g_l32) l32_free(kv.second);
  g_l32.clear();
}

}  // namespace simp

using namespace simp;

extern "C" {

#define SIMP_DESC_F32(n) float *n##_alloc, float *n, int64_t n##_off, int64_t n##_size, int64_t n##_stride
#define SIMP_DESC_I8(n) int8_t *n##_alloc, int8_t *n, int64_t n##_off, int64_t n##_size, int64_t n##_stride
#define SIMP_DESC_I32(n) int32_t *n##_alloc, int32_t *n, int64_t n##_off, int64_t n##_size, int64_t n##_stride

float llama32_forward(
    SIMP_DESC_I8(x_i8), SIMP_DESC_F32(rms_att_w), SIMP_DESC_F32(rms_ffn_w),
    SIMP_DESC_F32(rms_final_w), SIMP_DESC_I8(wq_t), SIMP_DESC_I8(wk_t), SIMP_DESC_I8(wv_t),
    SIMP_DESC_I8(wo_t), SIMP_DESC_I8(w1_t), SIMP_DESC_I8(w2_t), SIMP_DESC_I8(w3_t),
    SIMP_DESC_F32(wcls), SIMP_DESC_F32(x_fp32), SIMP_DESC_F32(xb_fp32), SIMP_DESC_F32(logits),
    SIMP_DESC_I8(xb_i8), SIMP_DESC_I8(k_cache), SIMP_DESC_I8(v_cache), SIMP_DESC_F32(att_scores),
    SIMP_DESC_F32(att_probs), SIMP_DESC_I32(attn_out), SIMP_DESC_I8(ffn_hb), int64_t pos,
    int64_t dim, int64_t hidden_dim, int64_t n_layers, int64_t n_heads, int64_t n_kv_heads,
    int64_t vocab_size, int64_t max_seq_len, int64_t head_dim) {
  const float nan = std::numeric_limits<float>::quiet_NaN();
  clear_error();
  (void)xb_i8; (void)att_scores; (void)att_probs; (void)ffn_hb;
  (void)xb_i8_alloc; (void)att_scores_alloc; (void)att_probs_alloc; (void)attn_out_alloc;
  (void)ffn_hb_alloc;
  auto fail = [&](const char *msg) {
    set_error(SIMP_RT_EINVAL, "llama32_forward: %s", msg);
    return nan;
  };
  if (dim <= 0 || hidden_dim <= 0 || n_layers <= 0 || n_heads <= 0 || n_kv_heads <= 0 ||
      vocab_size <= 0 || max_seq_len <= 0 || head_dim <= 0 || n_heads % n_kv_heads ||
      n_heads * head_dim != dim)
    return fail("bad model dimensions (n_heads * head_dim must equal dim)");
  if (dim % 16 || hidden_dim % 16 || head_dim % 16 || head_dim > 256 || dim > 16384 ||
      hidden_dim > 16384 ||
      4 * (head_dim + max_seq_len) > 47 * 1024)
    return fail("dim, hidden_dim and head_dim must be multiples of 16 (dim, hidden_dim <= "
                "16384, head_dim <= 256), head_dim + max_seq_len <= 12032");
  if (pos < 0 || pos >= max_seq_len) return fail("pos out of range");
  const int64_t L = n_layers, D = dim, H = hidden_dim, kv = n_kv_heads * head_dim;
  struct In { const void *p; int64_t off, size, stride, need; size_t esz; const char *name; };
  const In ins[] = {
      {rms_att_w, rms_att_w_off, rms_att_w_size, rms_att_w_stride, L * D, 4, "rms_att_w"},
      {rms_ffn_w, rms_ffn_w_off, rms_ffn_w_size, rms_ffn_w_stride, L * D, 4, "rms_ffn_w"},
      {rms_final_w, rms_final_w_off, rms_final_w_size, rms_final_w_stride, D, 4, "rms_final_w"},
      {wcls, wcls_off, wcls_size, wcls_stride, vocab_size * D, 4, "wcls"},
      {wq_t, wq_t_off, wq_t_size, wq_t_stride, L * D * D, 1, "wq_t"},
      {wk_t, wk_t_off, wk_t_size, wk_t_stride, L * kv * D, 1, "wk_t"},
      {wv_t, wv_t_off, wv_t_size, wv_t_stride, L * kv * D, 1, "wv_t"},
      {wo_t, wo_t_off, wo_t_size, wo_t_stride, L * D * D, 1, "wo_t"},
      {w1_t, w1_t_off, w1_t_size, w1_t_stride, L * H * D, 1, "w1_t"},
      {w2_t, w2_t_off, w2_t_size, w2_t_stride, L * D * H, 1, "w2_t"},
      {w3_t, w3_t_off, w3_t_size, w3_t_stride, L * H * D, 1, "w3_t"},
      {x_i8, x_i8_off, x_i8_size, x_i8_stride, D, 1, "x_i8"},
      {x_fp32, x_fp32_off, x_fp32_size, x_fp32_stride, D, 4, "x_fp32"},
      {xb_fp32, xb_fp32_off, xb_fp32_size, xb_fp32_stride, D, 4, "xb_fp32"},
      {logits, logits_off, logits_size, logits_stride, vocab_size, 4, "logits"},
      {k_cache, k_cache_off, k_cache_size, k_cache_stride, L * max_seq_len * kv, 1, "k_cache"},
      {v_cache, v_cache_off, v_cache_size, v_cache_stride, L * max_seq_len * kv, 1, "v_cache"},
      {attn_out, attn_out_off, attn_out_size, attn_out_stride, D, 4, "attn_out"}};
  for (const In &a : ins) {
    if (check_desc1(a.name, a.p, a.off, a.size, a.stride)) return nan;
    if (a.size < a.need) {
      set_error(SIMP_RT_EINVAL, "llama32_forward: %s has %lld elements, needs %lld", a.name,
                (long long)a.size, (long long)a.need);
      return nan;
    }
  }
  constexpr int NW = 11;  // weight arrays: ins[0..10]
  const void *wp[NW];
  for (int i = 0; i < NW; i++) wp[i] = (const char *)ins[i].p + ins[i].esz * (size_t)ins[i].off;
  std::vector<int64_t> key = {dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size,
                              max_seq_len, head_dim};
  for (int i = 0; i < NW; i++) key.push_back((int64_t)(uintptr_t)wp[i]);
  hipStream_t st = cur_stream();
  // one caller at a time: the engine, its copies and its KV state are shared
  std::lock_guard<std::mutex> lk(g_l32_mu);
  auto it = g_l32.find(key);
  if (it == g_l32.end()) {
    while (g_l32.size() >= kMaxL32Entries) {  // free the least recently used engine
      auto old = g_l32.begin();
      for (auto j = g_l32.begin(); j != g_l32.end(); ++j)
        if (j->second.last_use < old->second.last_use) old = j;
      (void)hipDeviceSynchronize();
      l32_free(old->second);
      g_l32.erase(old);
    }
    it = g_l32.emplace(key, L32Model{}).first;
    L32Model &nm = it->second;
    nm.dim = D; nm.hid = H; nm.L = L; nm.nh = n_heads; nm.nkv = n_kv_heads;
    nm.V = vocab_size; nm.S = max_seq_len; nm.hs = head_dim; nm.kv = kv;
    const void *d[NW];
    const char *err = nullptr;
    bool ok = true;
    for (int i = 0; i < NW && ok; i++)
      ok = nm.weights.bind(wp[i], ins[i].esz * (size_t)ins[i].need, &d[i], ins[i].name) ==
           SIMP_RT_OK;
    if (ok) {
      nm.rms_att = (const float *)d[0]; nm.rms_ffn = (const float *)d[1];
      nm.rms_final = (const float *)d[2]; nm.wcls = (const float *)d[3];
      nm.wq = (const int8_t *)d[4]; nm.wk = (const int8_t *)d[5]; nm.wv = (const int8_t *)d[6];
      nm.wo = (const int8_t *)d[7]; nm.w1 = (const int8_t *)d[8]; nm.w2 = (const int8_t *)d[9];
      nm.w3 = (const int8_t *)d[10];
      for (int i = 4; i < NW && ok; i++)
        if ((uintptr_t)d[i] & 15) {
          ok = false;
          err = "int8 weight arrays must start 16-byte aligned (offset included)";
        }
    }
    if (ok) ok = l32_alloc(nm) == SIMP_RT_OK;
    if (!ok) {
      l32_free(nm);
      g_l32.erase(it);
      return err ? fail(err) : nan;
    }
  }
  L32Model *m = &it->second;
  m->last_use = ++g_l32_clock;
  const size_t pitch = (size_t)(max_seq_len * kv), row = (size_t)kv, at = (size_t)(pos * kv);
  // the program reads the caches' rows [0, pos) and every weight on each call
  bool restart = false;
  if (m->kvs.prepare(pos, k_cache + k_cache_off, v_cache + v_cache_off, m->kc, m->vc, row, pitch,
                     L, st, &restart) ||
      m->weights.verify(restart))
    return nan;
  hipError_t e = hipMemcpyAsync(m->xi, x_i8 + x_i8_off, (size_t)D, hipMemcpyDefault, st);
  if (e != hipSuccess) {
    hip_fail(e, "llama32_forward: input copy");
    return nan;
  }
  if (l32_step(*m, pos, st)) return nan;
  e = hipMemcpyAsync(logits + logits_off, m->logits, 4 * (size_t)vocab_size, hipMemcpyDefault, st);
  if (e == hipSuccess)
    e = hipMemcpyAsync(x_fp32 + x_fp32_off, m->x, 4 * (size_t)D, hipMemcpyDefault, st);
  if (e == hipSuccess)
    e = hipMemcpyAsync(xb_fp32 + xb_fp32_off, m->xb, 4 * (size_t)D, hipMemcpyDefault, st);
  // attn_out as the program leaves it: the last layer's attention
  if (e == hipSuccess)
    e = hipMemcpyAsync(attn_out + attn_out_off, m->attn, 4 * (size_t)D, hipMemcpyDefault, st);
  if (e == hipSuccess)
    e = hipMemcpy2DAsync(k_cache + k_cache_off + at, pitch, m->kc + at, pitch, row, (size_t)L,
                         hipMemcpyDefault, st);
  if (e == hipSuccess)
    e = hipMemcpy2DAsync(v_cache + v_cache_off + at, pitch, m->vc + at, pitch, row, (size_t)L,
                         hipMemcpyDefault, st);
  // logits[0] for the return value, in the same synchronisation
  if (e == hipSuccess) e = hipMemcpyAsync(m->first, m->logits, sizeof(float), hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess) {
    hip_fail(e, "llama32_forward: result copies");
    return nan;
  }
  m->kvs.done(pos);
  return *m->first;
}

#undef SIMP_DESC_F32
#undef SIMP_DESC_I8
#undef SIMP_DESC_I32

}  // extern "C"
