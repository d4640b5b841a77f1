// decode.hip -- single-token LLaMA decode step and greedy generation.
//
// The step is the one of examples/llama2/stories110M.sl:44-247 (fp32 weights)
// and examples/llama2/llama2_quant.sl:57-198 (W4 weights), shape-parametric
// (both reference programs hard-code their dims), with the GQA head map of
// llama2_quant.sl:98, score scale 1/sqrt(head_size) (stories110M.sl:140 writes
// /8.0, which is the same for head_size 64), RoPE as in stories110M.sl:86-112
// (llama2_quant.sl omits it) and greedy strict-'>' argmax
// (examples/llama2/generate_stories110M.cpp:73-83).
//
// Per layer the reference issues ~12 loops/ops; here they are 5 kernels:
//   1 QKV GEMV (Wq|Wk|Wv as one launch) with the attention RMSNorm computed in
//     the prologue of every block (x is dim floats; recomputing it is cheaper
//     than a launch)
//   2 attention, one block per head: RoPE of q and of the head's k, store of
//     k,v into the KV cache at pos, scores, softmax, weighted sum of V
//   3 Wo GEMV accumulating into x (the residual add)
//   4 W1|W3 GEMV with the FFN RMSNorm in the prologue; rows i of W1 and W3 are
//     computed side by side and the epilogue writes g[i] = silu(h1[i]) * h3[i]
//   5 W2 GEMV on g, accumulating into x
// then a final RMSNorm+classifier GEMV and an argmax kernel that also advances
// the step state (token, pos) on the device, so a captured step graph can be
// replayed for every token with no host round trip.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <map>
#include <mutex>
#include <vector>

#include "rt_device.h"
#include "rt_internal.h"

namespace simp {
namespace {

constexpr int kMaxSeg = 3;

// GEMV input prologues: x as given, RMSNorm of x, or x combined from split-
// attention partials (fp32 GEMV; the dot8 W4 kernel has its own CMB form).
enum Prologue { kPlain = 0, kRmsNorm = 1, kCombine = 2 };
// GEMV output modes: store, accumulate into the output (residual add), or
// paired rows: row i of segment 0 (W1) and of segment 1 (W3) are computed
// together and segment 0's output receives silu(h1[i]) * h3[i].
enum OutMode { kStore = 0, kAccum = 1, kPairSwiGLU = 2 };

struct Seg {
  const void *W;    // fp32 rows [rows, K] or packed W4 rows [rows, K/2]
  const float *S;   // W4 scales [rows, K/gs] (unused for fp32)
  float *out;       // [rows]
  int rows;
  int tile0;        // first row tile of this segment (W4 kernel)
  const float *Z = nullptr;  // zeros [rows, K/gs] of the unsigned W4 format
};
struct Segs {
  Seg s[kMaxSeg];
  int n;
};

// Step state on the device: [0] token, [1] pos, [2] n_prompt, [3] n_total.
struct StepState {
  int token, pos, n_prompt, n_total;
};

// Synchronises s on scope exit unless cleared: a call that returns early
// (an error) after queueing copies from its own stack or the caller's arrays
// still lets them finish before those go away.
struct StreamDrain {
  hipStream_t s;
  ~StreamDrain() {
    if (s) (void)hipStreamSynchronize(s);
  }
};

// Split-attention partials that a GEMV combines into its x (launch_attention
// with combine false): n chunks of max_splits per head of hs, each hs floats
// of o, then m and l (a stride of hs + 4 floats).
struct Partials {
  const float *ws;
  int hs, max_splits, n;
};

__device__ __forceinline__ float silu_mul(float h1, float h3) {
  return (h1 / (1.f + expf(-h1))) * h3;
}

// GEMV input staging in two phases, so that the input loads can be issued
// before a kernel's first weight loads (vmcnt retires loads in issue order):
//   load():   x0 (and the norm weight) into registers, KP slots per thread
//   finish(): the prologue math, then the result into LDS (through `put`)
template <int PRO, int KP>
struct XStage {
  float a[KP], b[KP];
  __device__ __forceinline__ void load(const float *__restrict__ x0, const float *__restrict__ nw,
                                       int K) {
#pragma unroll
    for (int k = 0; k < KP; k++) {
      const int i = threadIdx.x + 256 * k;
      a[k] = i < K ? x0[i] : 0.f;
      if constexpr (PRO == kRmsNorm) b[k] = i < K ? nw[i] : 0.f;
    }
  }
  template <class Put>
  __device__ __forceinline__ void finish(int K, float eps, float *scratch, Put put) {
    float rms = 1.f;
    if constexpr (PRO == kRmsNorm) {
      float ss = 0.f;
#pragma unroll
      for (int k = 0; k < KP; k++) ss = fmaf(a[k], a[k], ss);
      ss = block_sum_lds<true>(ss, scratch);  // weight loads issued before stay in flight
      rms = sqrtf(ss / (float)K + eps);
    }
#pragma unroll
    for (int k = 0; k < KP; k++) {
      const int i = threadIdx.x + 256 * k;
      if (i < K) {
        float v = a[k];
        if constexpr (PRO == kRmsNorm) v = (v / rms) * b[k];
        put(i, v);
      }
    }
  }
};

// The kCombine prologue: x[i] from the split-attention partials of i's head,
// in attn_combine_k's arithmetic (M = max_s m_s, L = sum_s e^(m_s - M) l_s,
// x = (sum_s e^(m_s - M) o_s) / L), for at most CR chunks.  load() requests
// every chunk's o of the thread's elements and their heads' (m, l) at once;
// finish() combines in registers.
template <int KP>
struct XStageCmb {
  static constexpr int CR = 8;
  float o[KP][CR];
  float2 ml[KP][CR];
  __device__ __forceinline__ void load(const Partials &cp, int K) {
    const int st = cp.hs + 4;
#pragma unroll
    for (int k = 0; k < KP; k++) {
      const int i = min((int)threadIdx.x + 256 * k, K - 1);
      const int h = i / cp.hs;
      const float *w = cp.ws + (int64_t)h * cp.max_splits * st;
#pragma unroll
      for (int s = 0; s < CR; s++) {
        o[k][s] = s < cp.n ? w[s * st + (i - h * cp.hs)] : 0.f;
        ml[k][s] = s < cp.n ? *(const float2 *)(w + s * st + cp.hs) : make_float2(-INFINITY, 0.f);
      }
    }
  }
  template <class Put>
  __device__ __forceinline__ void finish(const Partials &cp, int K, Put put) {
#pragma unroll
    for (int k = 0; k < KP; k++) {
      const int i = (int)threadIdx.x + 256 * k;
      if (i >= K) continue;
      float M = -INFINITY;
#pragma unroll
      for (int s = 0; s < CR; s++)
        if (s < cp.n) M = fmaxf(M, ml[k][s].x);
      float L = 0.f, v = 0.f;
#pragma unroll
      for (int s = 0; s < CR; s++)
        if (s < cp.n) {
          const float e = expf(ml[k][s].x - M);
          L += e * ml[k][s].y;
          v = fmaf(e, o[k][s], v);
        }
      put(i, v * (1.f / L));
    }
  }
};

__device__ __forceinline__ const Seg &seg_of_row(const Segs &sg, int &row) {
  int i = 0;
  while (i + 1 < sg.n && row >= sg.s[i].rows) {
    row -= sg.s[i].rows;
    i++;
  }
  return sg.s[i];
}

// fp32 multi-matrix GEMV: one wave per row, lanes along K (float4 slots
// j*64 + lane, J per lane), x in LDS.  The wave's first row is loaded before
// the prologue and every next row while the current one is reduced, so the
// prologue and the reductions overlap weight traffic.  J == 0: any K (loop).
// OUT == kPairSwiGLU: "row" i is the pair (W1 row i, W3 row i) of segments 0
// and 1; the wave computes both dot products and stores silu(h1) * h3.
template <int PRO, int OUT, int J, int KP>
__global__ void __launch_bounds__(256)
    dgemv_f32(Segs sg, int total_rows, int K, const float *__restrict__ x0,
              const float *__restrict__ nw, float eps, Partials cp) {
  constexpr int NR = OUT == kPairSwiGLU ? 2 : 1;  // weight rows per output row
  extern __shared__ float xs[];
  __shared__ float scratch[16];
  const int lane = threadIdx.x & 63;
  const int nw_total = gridDim.x * 4;
  const int K4 = K >> 2;
  int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  constexpr int JJ = J > 0 ? J : 1;
  float4 a[NR][JJ];
  auto rowptr = [&](int rr, int e) {
    int row = rr;
    const Seg &sgm = OUT == kPairSwiGLU ? sg.s[e] : seg_of_row(sg, row);
    return (const float4 *)((const float *)sgm.W + (int64_t)row * K);
  };
  auto load = [&](int rr, float4 (&v)[NR][JJ]) {
#pragma unroll
    for (int e = 0; e < NR; e++) {
      const float4 *w = rowptr(rr, e);
#pragma unroll
      for (int j = 0; j < JJ; j++) {
        const int q = lane + 64 * j;
        // streaming loads: the weights are read once per step; the KV cache and
        // activations stay cached (110M: 2570 -> 2930 tok/s)
        v[e][j] = q < K4 ? ntload_f4(w + q) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  };
  if constexpr (PRO == kCombine) {
    XStageCmb<KP> xst;
    xst.load(cp, K);                           // partials first ...
    if (J > 0 && r < total_rows) load(r, a);   // ... then the first row's weights
    xst.finish(cp, K, [&](int i, float v) { xs[i] = v; });
  } else {
    XStage<PRO, KP> xst;
    xst.load(x0, nw, K);                       // input loads first ...
    if (J > 0 && r < total_rows) load(r, a);   // ... then the first row's weights
    xst.finish(K, eps, scratch, [&](int i, float v) { xs[i] = v; });
  }
  lds_barrier();
  for (; r < total_rows; r += nw_total) {
    float s[NR];
#pragma unroll
    for (int e = 0; e < NR; e++) s[e] = 0.f;
    if constexpr (J > 0) {
      float4 b[NR][JJ];
      if (r + nw_total < total_rows) load(r + nw_total, b);
#pragma unroll
      for (int j = 0; j < JJ; j++) {
        const int q = lane + 64 * j;
        if (q < K4) {
          const float4 xv = *(const float4 *)(xs + 4 * q);
#pragma unroll
          for (int e = 0; e < NR; e++) {
            s[e] = fmaf(a[e][j].x, xv.x, s[e]);
            s[e] = fmaf(a[e][j].y, xv.y, s[e]);
            s[e] = fmaf(a[e][j].z, xv.z, s[e]);
            s[e] = fmaf(a[e][j].w, xv.w, s[e]);
          }
        }
      }
#pragma unroll
      for (int e = 0; e < NR; e++)
#pragma unroll
        for (int j = 0; j < JJ; j++) a[e][j] = b[e][j];
    } else {
#pragma unroll
      for (int e = 0; e < NR; e++) {
        const float4 *w = rowptr(r, e);
        for (int q = lane; q < K4; q += 64) {
          const float4 av = w[q];
          const float4 xv = *(const float4 *)(xs + 4 * q);
          s[e] = fmaf(av.x, xv.x, s[e]);
          s[e] = fmaf(av.y, xv.y, s[e]);
          s[e] = fmaf(av.z, xv.z, s[e]);
          s[e] = fmaf(av.w, xv.w, s[e]);
        }
      }
    }
#pragma unroll
    for (int e = 0; e < NR; e++) s[e] = wave_sum_dpp(s[e]);
    if (lane == 0) {
      int row = r;
      const Seg &sgm = OUT == kPairSwiGLU ? sg.s[0] : seg_of_row(sg, row);
      float *o = sgm.out + row;
      if constexpr (OUT == kPairSwiGLU) *o = silu_mul(s[0], s[NR - 1]);
      else *o = OUT == kAccum ? *o + s[0] : s[0];
    }
  }
}

// Sum of NWV per-wave values: pairs of pairs, then the groups of four in order
// (for NWV = 4: (v0 + v1) + (v2 + v3)).
template <int NWV>
__device__ __forceinline__ float sum_waves(const float *v) {
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < NWV; i += 4) t += (v[i] + v[i + 1]) + (v[i + 2] + v[i + 3]);
  return t;
}

// W4 (symmetric, group gs) multi-matrix GEMV: lane -> row (8 rows per block),
// G = 8 NWV chunk groups of 16-byte chunks per block, 8 per wave.  The NWV
// waves partition a row's chunks (wave w takes the chunks c with c % G in
// [8w, 8w + 8)), so each wave stages only its own x chunks in LDS and no block
// barrier precedes the compute: a chunk's work waits only for its own bytes
// (x loads are issued first, then the weights; loads retire in issue order).
// x's float4 slots of chunk j are rotated by j (conflict-free reads), and the
// per-chunk sums of x fold in the -8 of the q+8 nibble flip.
//   PRO kRmsNorm: the wave stages x * norm_weight and its share of sum(x^2);
//     the 1/rms factor multiplies the finished row sums.
//   OUT kPairSwiGLU: lanes r < 4 take row i of segment 0 (W1), lanes r >= 4
//     the same row of segment 1 (W3); segment 0's output gets silu(h1) * h3.
template <int PRO, int OUT, int UB, int NWV = 4>
__global__ void __launch_bounds__(64 * NWV)
    dgemv_w4(Segs sg, int K, int gs, const float *__restrict__ x0, const float *__restrict__ nw,
             float eps) {
  constexpr int RB = 8, G = 64 * NWV / RB, GW = 64 / RB;
  constexpr int CW = GW * UB;         // x chunks staged per wave
  constexpr int XPL = CW * 8 / 64;    // x float4 per lane
  __shared__ float red[NWV][RB];
  __shared__ float ssq[NWV];
  __shared__ __align__(16) float xw[NWV][CW][32];
  __shared__ float xsw[NWV][CW];
  const int nchunk = K >> 5, cpg = gs >> 5, cps = cpg_log2(cpg);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = threadIdx.x % RB, g = threadIdx.x / RB, gl = lane / RB;
  int si = 0, row0, rr;
  if constexpr (OUT == kPairSwiGLU) {
    si = r >> 2;
    row0 = (int)blockIdx.x * (RB / 2);
    rr = r & 3;
  } else {
    while (si + 1 < sg.n && (int)blockIdx.x >= sg.s[si + 1].tile0) si++;
    row0 = ((int)blockIdx.x - sg.s[si].tile0) * RB;
    rr = r;
  }
  const Seg &sgm = sg.s[si];
  const int n = min(row0 + rr, sgm.rows - 1);  // clamped: rows past the end are never stored
  const uint8_t *wrow = (const uint8_t *)sgm.W + (int64_t)n * (K >> 1);
  const float *srow = sgm.S + (int64_t)n * (K / gs);
  // the wave's x chunks: local j = u*GW + jj holds chunk wave*GW + jj + G*u
  float4 xv[XPL], nv[XPL];
#pragma unroll
  for (int i = 0; i < XPL; i++) {
    const int f = lane + 64 * i, j = f >> 3, q = f & 7;
    const int c = min(wave * GW + j % GW + G * (j / GW), nchunk - 1);
    xv[i] = *(const float4 *)(x0 + 32 * c + 4 * q);
    if constexpr (PRO == kRmsNorm) nv[i] = *(const float4 *)(nw + 32 * c + 4 * q);
  }
  uint4 w[UB];
  float sc[UB];
#pragma unroll
  for (int u = 0; u < UB; u++) {
    const int c = min(g + u * G, nchunk - 1);
    w[u] = *(const uint4 *)(wrow + 16 * c);
    sc[u] = srow[chunk_group(c, cpg, cps)];
  }
  // every load above is issued before the x staging below uses any of them
  __builtin_amdgcn_sched_barrier(0);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < XPL; i++) {
    const int f = lane + 64 * i, j = f >> 3, q = f & 7;
    float4 v = xv[i];
    if constexpr (PRO == kRmsNorm) {
      if (wave * GW + j % GW + G * (j / GW) < nchunk) {  // each chunk once per block
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
      }
      v = make_float4(v.x * nv[i].x, v.y * nv[i].y, v.z * nv[i].z, v.w * nv[i].w);
    }
    *(float4 *)(&xw[wave][j][4 * ((q + j) & 7)]) = v;
    float t = (v.x + v.y) + (v.z + v.w);
    t += __shfl_xor(t, 1);
    t += __shfl_xor(t, 2);
    t += __shfl_xor(t, 4);
    if (q == 0) xsw[wave][j] = t;
  }
  if constexpr (PRO == kRmsNorm) {
    ss = wave_sum(ss);
    if (lane == 0) ssq[wave] = ss;
  }
  // the wave's own LDS writes are complete before its lanes read each other's
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();
  float acc = 0.f;
#pragma unroll
  for (int u = 0; u < UB; u++) {
    const int c = g + u * G, j = u * GW + gl;
    if (c < nchunk) {  // uniform across the RB lanes of the group
      uint4 wv = w[u];
      wv.x ^= 0x88888888u; wv.y ^= 0x88888888u; wv.z ^= 0x88888888u; wv.w ^= 0x88888888u;
      float uu[32];
      unpack32(wv, uu);
      float p = 0.f;
#pragma unroll
      for (int q = 0; q < 8; q++) {
        const float4 v = *(const float4 *)(&xw[wave][j][4 * ((q + j) & 7)]);
        p = fmaf(uu[4 * q + 0], v.x, p);
        p = fmaf(uu[4 * q + 1], v.y, p);
        p = fmaf(uu[4 * q + 2], v.z, p);
        p = fmaf(uu[4 * q + 3], v.w, p);
      }
      acc = fmaf(sc[u], fmaf(-8.f, xsw[wave][j], p), acc);  // sum (u-8) x
    }
  }
#pragma unroll
  for (int d = RB; d < 64; d <<= 1) acc += __shfl_xor(acc, d);
  if (lane < RB) red[wave][r] = acc;
  __syncthreads();
  float scale = 1.f;
  if constexpr (PRO == kRmsNorm)
    scale = 1.f / sqrtf(sum_waves<NWV>(ssq) / (float)K + eps);
  auto row_sum = [&](int rr2) {
    float t = 0.f;
#pragma unroll
    for (int v = 0; v < NWV; v += 4)
      t += (red[v][rr2] + red[v + 1][rr2]) + (red[v + 2][rr2] + red[v + 3][rr2]);
    return t * scale;
  };
  if constexpr (OUT == kPairSwiGLU) {
    if (threadIdx.x < RB / 2 && row0 + r < sgm.rows)  // r < 4: segment 0
      sgm.out[row0 + r] = silu_mul(row_sum(r), row_sum(r + RB / 2));
  } else if (threadIdx.x < RB && row0 + r < sgm.rows) {
    float *o = sgm.out + row0 + r;
    const float t = row_sum(r);
    *o = OUT == kAccum ? *o + t : t;
  }
}

// Attention, one 1024-thread block per head (rope == nullptr: no rotation), for
// head sizes attn_split_k does not take.  No cross-block communication: a
// device-scope fence to publish partials between blocks costs an L2 write-back
// on this multi-XCD part, more than the whole head's work.  Latency is the
// cost here, so every cache load that depends
// only on pos is issued first, into registers: the K rows of the first 256
// positions (4 lanes per position, a quarter of the head dimension each, as
// float4) and up to kAttnVE V values per thread (thread (d, p) holds
// positions p, p + P, ...; P = blockDim / head_size).  Then RoPE of q and of
// the head's new k, the KV store at pos (first head of each kv head), scores,
// softmax, and the V sum from registers; positions past the register window
// are loaded in loops.  LDS: 3*256 + seq_len + 1024 floats (dynamic part:
// att[seq_len]).
constexpr int kAttnThreads = 1024;
constexpr int kAttnKF = 7;   // K float4 per lane: head_size <= 112 on the register path
constexpr int kAttnVE = 24;  // V values per thread in registers

__global__ void __launch_bounds__(kAttnThreads)
    attn_k(const float *__restrict__ qkv, float *__restrict__ kc, float *__restrict__ vc,
           float *__restrict__ out, const StepState *__restrict__ st, int dim, int kv_dim,
           int n_heads, int n_kv_heads, int hs, const float2 *__restrict__ rope) {
  __shared__ __align__(16) float qs[256];
  __shared__ __align__(16) float kn[256];
  __shared__ __align__(16) float vn[256];
  __shared__ float red[kAttnThreads];
  __shared__ float scratch[16];
  extern __shared__ float att[];  // [pos + 1]
  const int h = blockIdx.x;
  const int pos = st->pos;
  const int kvh = h * n_kv_heads / n_heads;
  const float *q = qkv + h * hs;
  const float *k = qkv + dim + kvh * hs;
  const float *v = qkv + dim + kv_dim + kvh * hs;
  const float *kbase = kc + kvh * hs;
  const float *vbase = vc + kvh * hs;
  const int hs4 = hs >> 2;
  const int lt = threadIdx.x >> 2, sub = threadIdx.x & 3;
  const int P = blockDim.x / hs;
  const int d = threadIdx.x % hs, p = threadIdx.x / hs;
  const int last = max(pos - 1, 0);  // clamped row index: out-of-range lanes load a valid row
  // 1. cache loads (unconditional, clamped addresses; out-of-range values unused)
  float vv[kAttnVE];
#pragma unroll
  for (int e = 0; e < kAttnVE; e++)
    vv[e] = vbase[(int64_t)min(p + e * P, last) * kv_dim + d];
  const bool kreg = hs4 <= 4 * kAttnKF;
  float4 kr[kAttnKF];
  {
    const float4 *krow = (const float4 *)(kbase + (int64_t)min(lt, last) * kv_dim);
#pragma unroll
    for (int i = 0; i < kAttnKF; i++) kr[i] = krow[min(sub + 4 * i, hs4 - 1)];
  }
  // 2. this token's q, k, v (RoPE on q and k)
  for (int j = 2 * threadIdx.x; j < hs; j += 2 * blockDim.x) {
    const float2 f = rope ? rope[(int64_t)pos * (hs >> 1) + (j >> 1)] : make_float2(1.f, 0.f);
    const float fcr = f.x, fci = f.y;
    qs[j] = q[j] * fcr - q[j + 1] * fci;
    qs[j + 1] = q[j] * fci + q[j + 1] * fcr;
    kn[j] = k[j] * fcr - k[j + 1] * fci;
    kn[j + 1] = k[j] * fci + k[j + 1] * fcr;
    vn[j] = v[j];
    vn[j + 1] = v[j + 1];
  }
  __syncthreads();
  const bool writer = h == 0 || ((h - 1) * n_kv_heads / n_heads) != kvh;
  if (writer) {
    for (int j = threadIdx.x; j < hs; j += blockDim.x) {
      kc[(int64_t)pos * kv_dim + kvh * hs + j] = kn[j];
      vc[(int64_t)pos * kv_dim + kvh * hs + j] = vn[j];
    }
  }
  // 3. scores
  const float inv_scale = 1.f / sqrtf((float)hs);
  const float4 *q4 = (const float4 *)qs;
  for (int tb = 0; tb <= pos; tb += kAttnThreads / 4) {
    const int t = tb + lt;
    float sacc = 0.f;
    if (t <= pos) {
      if (tb == 0 && t < pos && kreg) {
#pragma unroll
        for (int i = 0; i < kAttnKF; i++) {
          const int j = sub + 4 * i;
          if (j < hs4) {
            const float4 a = kr[i], b = q4[j];
            sacc = fmaf(a.x, b.x, sacc);
            sacc = fmaf(a.y, b.y, sacc);
            sacc = fmaf(a.z, b.z, sacc);
            sacc = fmaf(a.w, b.w, sacc);
          }
        }
      } else {
        const float4 *krow = (const float4 *)(t == pos ? kn : kbase + (int64_t)t * kv_dim);
        for (int j = sub; j < hs4; j += 4) {
          const float4 a = krow[j], b = q4[j];
          sacc = fmaf(a.x, b.x, sacc);
          sacc = fmaf(a.y, b.y, sacc);
          sacc = fmaf(a.z, b.z, sacc);
          sacc = fmaf(a.w, b.w, sacc);
        }
      }
    }
    sacc += __shfl_xor(sacc, 1);
    sacc += __shfl_xor(sacc, 2);
    if (sub == 0 && t <= pos) att[t] = sacc * inv_scale;
  }
  __syncthreads();
  // 4. softmax
  float m = -INFINITY;
  for (int t = threadIdx.x; t <= pos; t += blockDim.x) m = fmaxf(m, att[t]);
  m = block_max(m, scratch);
  float l = 0.f;
  for (int t = threadIdx.x; t <= pos; t += blockDim.x) {
    const float e = expf(att[t] - m);
    att[t] = e;
    l += e;
  }
  l = block_sum(l, scratch);
  // 5. V sum: thread (d, p) over positions p, p + P, ...; partitions added through LDS
  if (p < P) {
    float o = 0.f;
#pragma unroll
    for (int e = 0; e < kAttnVE; e++) {
      const int t = p + e * P;
      if (t < pos) o = fmaf(att[t], vv[e], o);
    }
    for (int t = p + kAttnVE * P; t < pos; t += P) o = fmaf(att[t], vbase[(int64_t)t * kv_dim + d], o);
    if (p == pos % P) o = fmaf(att[pos], vn[d], o);
    red[p * hs + d] = o;
  }
  __syncthreads();
  for (int dd = threadIdx.x; dd < hs; dd += blockDim.x) {
    float sacc = 0.f;
    for (int pp = 0; pp < P; pp++) sacc += red[pp * hs + dd];
    out[h * hs + dd] = sacc / l;
  }
}

// Attention split over positions (head_size % 4 == 0, head_size <= 128):
// block (h, s) of NWV waves takes positions [TP s, TP s + TP) of head h,
// TP = 16 NWV, so a long context spreads over up to seq_len / TP CUs per head
// (4 waves and 64 positions: 8 waves and 128 positions measured 8.4 against
// 6.4 us per launch at pos 150, one CU moving twice the rows); the grid has
// exactly the chunks of the step's position range.  Latency is what costs
// here, and the loads' return path of a CU (every lane's bytes, duplicates
// included), so:
//   * lane (half, j) owns float4 j of the head dimension and the wave's
//     positions tw + 2e + half (e < 8): it loads q, this token's k and v and
//     the RoPE row once, and 16 cache rows (K, V) of 16 bytes.  An earlier
//     layout with 4 lanes per position loaded q, k and the RoPE row in every
//     position's lanes, 49 KB per wave against 20 KB here, and its launch
//     took 1.3 us longer (6.4 against 5.1 us in a 3B-shaped layer graph);
//   * every load that does not depend on pos is issued first, the RoPE row
//     after pos;
//   * rows at or past pos are loaded (clamped to the cache) and never used:
//     position pos takes this token's k, v, which the first head of each kv
//     head stores into the cache at pos;
//   * the 8 partial dot products of a lane are summed over the 32 lanes of its
//     half by a transposed butterfly (rows of 16 swapped, DPP row rotations
//     and mirrors), which leaves position (half, e)'s score in lanes
//     32 half + 4 e .. + 3; a softmax over the wave's 16 positions (m_w, l_w)
//     and the V sum o_w (probabilities broadcast by v_readlane, the halves
//     added by v_permlane32_swap) stay in the VALU;
//   * one barrier, then the NWV (m_w, l_w, o_w) are combined into the
//     chunk's (m, l, o).
// A single chunk (pos < TP) writes out = o / l directly; otherwise (o, m, l)
// go to ws[h][s] and attn_combine_k forms
//   out = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s,  M = max_s m_s,
// which equals the one-pass softmax-weighted sum up to rounding.  (Combining in
// the last chunk's block instead, after a count of the others in a global
// counter, measured ~4 us slower than the separate kernel: the agent-scope
// round trips cost more than a launch.)
constexpr int kAttnNWV = 4, kAttnTP = 16 * kAttnNWV;
template <int NWV>
__global__ void __launch_bounds__(64 * NWV)
    attn_split_k(const float *__restrict__ qkv, float *__restrict__ kc, float *__restrict__ vc,
                 float *__restrict__ out, float *__restrict__ ws,
                 const StepState *__restrict__ st, int dim, int kv_dim, int n_heads,
                 int n_kv_heads, int hs, const float2 *__restrict__ rope, int max_splits,
                 int nsplit, int seq_len) {
  constexpr int WP = 16;          // positions per wave
  constexpr int E = WP / 2;       // positions per lane
  constexpr int TP = WP * NWV;
  __shared__ __align__(16) float4 wo[NWV][32];
  __shared__ float wml[NWV][2];
  const int h = blockIdx.x, s = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, j = lane & 31;
  const int t0 = s * TP, tw = t0 + WP * wave;  // first position of the wave
  const int kvh = h * n_kv_heads / n_heads;
  const int hs4 = hs >> 2, kv4 = kv_dim >> 2;
  const int jj = min(j, hs4 - 1);
  const float4 *kbase = (const float4 *)(kc + kvh * hs), *vbase = (const float4 *)(vc + kvh * hs);
  // 1. loads, all before pos
  float4 kr[E], vv[E];
#pragma unroll
  for (int e = 0; e < E; e++)
    kr[e] = kbase[(int64_t)min(tw + 2 * e + half, seq_len - 1) * kv4 + jj];
  float4 qv = ((const float4 *)(qkv + h * hs))[jj];
  float4 kn = ((const float4 *)(qkv + dim + kvh * hs))[jj];
  const float4 vn = ((const float4 *)(qkv + dim + kv_dim + kvh * hs))[jj];
#pragma unroll
  for (int e = 0; e < E; e++)
    vv[e] = vbase[(int64_t)min(tw + 2 * e + half, seq_len - 1) * kv4 + jj];
  const int pos = st->pos;
  // (cos, sin) of the two pairs of float4 j at pos
  const float4 rf = rope ? ((const float4 *)(rope + (int64_t)pos * (hs >> 1)))[jj]
                         : make_float4(1.f, 0.f, 1.f, 0.f);
  // 2. RoPE of q and of this token's k (pairs (x, y) and (z, w) of a float4)
  auto rot = [](float4 a, float4 f) {
    return make_float4(a.x * f.x - a.y * f.y, a.x * f.y + a.y * f.x, a.z * f.z - a.w * f.w,
                       a.z * f.w + a.w * f.z);
  };
  qv = rot(qv, rf);
  kn = rot(kn, rf);
  // the first head of each kv head stores k, v at pos (chunk holding pos)
  const bool writer = (h == 0 || ((h - 1) * n_kv_heads / n_heads) != kvh) && pos >= t0 &&
                      pos < t0 + TP && wave == 0;
  if (writer && half == 0 && j < hs4) {
    ((float4 *)(kc + (int64_t)pos * kv_dim + kvh * hs))[j] = kn;
    ((float4 *)(vc + (int64_t)pos * kv_dim + kvh * hs))[j] = vn;
  }
  // 3. scores: this lane's part of the dot product for each of its positions,
  // then a reduce-scatter over the 32 lanes of the half
  float v[E];
#pragma unroll
  for (int e = 0; e < E; e++) {
    const float4 a = tw + 2 * e + half == pos ? kn : kr[e];
    float d = a.x * qv.x;
    d = fmaf(a.y, qv.y, d);
    d = fmaf(a.z, qv.z, d);
    d = fmaf(a.w, qv.w, d);
    v[e] = j < hs4 ? d : 0.f;
  }
  const bool b4 = lane & 16, b3 = lane & 8, b2 = lane & 4;
  float w4[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {  // lanes 16 apart: bit 4 clear keeps index i, set i + 4
    float a = v[i], b = v[i + 4];
    permlane16_swap(a, b);
    w4[i] = a + b;
  }
  float w2[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {  // lanes 8 apart: bit 3 clear keeps i, set i + 2
    const float a = b3 ? w4[i + 2] : w4[i], b = b3 ? w4[i] : w4[i + 2];
    w2[i] = a + dpp_mov<kDppRor8>(b);
  }
  float sc;
  {  // lanes l and l ^ 7 (bit 2 differs): bit 2 clear keeps 0, set 1
    const float a = b2 ? w2[1] : w2[0], b = b2 ? w2[0] : w2[1];
    sc = a + dpp_mov<kDppHalfMirror>(b);
  }
  sc += dpp_mov<kDppXor1>(sc);  // the 4 lanes l ^ {0, 1, 2, 3}: all 32 lanes added
  sc += dpp_mov<kDppXor2>(sc);
  // lanes 32 half + 4 e .. + 3 hold position tw + 2 e + half, e = 4 b4 + 2 b3 + b2
  const int pl = tw + 2 * ((b4 ? 4 : 0) + (b3 ? 2 : 0) + (b2 ? 1 : 0)) + half;
  sc = pl <= pos ? sc * (1.f / sqrtf((float)hs)) : -INFINITY;
  // 4. softmax over the wave's positions (each replicated in 4 lanes)
  const float m = wave_max_dpp(sc);
  const float pe = pl <= pos ? expf(sc - m) : 0.f;  // pl <= pos: m is finite
  const float l = wave_sum_dpp((lane & 3) == 0 ? pe : 0.f);
  // 5. V sum: lane (half, j) over its positions, probabilities from lanes
  // 32 half + 4 e; the two halves added
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int e = 0; e < E; e++) {
    const float p0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pe), 4 * e));
    const float p1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pe), 32 + 4 * e));
    const float pt = half ? p1 : p0;
    const int p = tw + 2 * e + half;
    // rows past pos are selected out, not weighted by 0: the cache beyond
    // the written positions holds whatever the memory held (0 * NaN = NaN)
    const float4 x = p == pos ? vn : p < pos ? vv[e] : make_float4(0.f, 0.f, 0.f, 0.f);
    o.x = fmaf(pt, x.x, o.x);
    o.y = fmaf(pt, x.y, o.y);
    o.z = fmaf(pt, x.z, o.z);
    o.w = fmaf(pt, x.w, o.w);
  }
  {
    float a = o.x, b = o.x;
    permlane32_swap(a, b);
    o.x = a + b;
    a = b = o.y;
    permlane32_swap(a, b);
    o.y = a + b;
    a = b = o.z;
    permlane32_swap(a, b);
    o.z = a + b;
    a = b = o.w;
    permlane32_swap(a, b);
    o.w = a + b;
  }
  if (lane < hs4) wo[wave][lane] = o;
  if (lane == 0) {
    wml[wave][0] = m;
    wml[wave][1] = l;
  }
  __syncthreads();
  // 6. the NWV waves of the chunk (a wave wholly past pos has m = -inf, l = 0)
  if ((int)threadIdx.x < hs4) {
    float M = wml[0][0];
#pragma unroll
    for (int w = 1; w < NWV; w++) M = fmaxf(M, wml[w][0]);
    float L = 0.f;
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int w = 0; w < NWV; w++) {
      const float f = wml[w][1] > 0.f ? expf(wml[w][0] - M) : 0.f;
      L = fmaf(f, wml[w][1], L);
      const float4 x = wo[w][threadIdx.x];
      O.x = fmaf(f, x.x, O.x);
      O.y = fmaf(f, x.y, O.y);
      O.z = fmaf(f, x.z, O.z);
      O.w = fmaf(f, x.w, O.w);
    }
    if (nsplit == 1) {
      const float il = 1.f / L;
      ((float4 *)(out + h * hs))[threadIdx.x] = make_float4(O.x * il, O.y * il, O.z * il, O.w * il);
    } else {
      float *w = ws + ((int64_t)h * max_splits + s) * (hs + 4);
      ((float4 *)w)[threadIdx.x] = O;
      if (threadIdx.x == 0) {
        w[hs] = M;
        w[hs + 1] = L;
      }
    }
  }
}

// Combines the nsplit (> 1) chunks of attn_split_k: the chunks' (m, l) go
// through LDS (one load each), and each output element requests its chunks'
// o values eight at a time; sums in chunk order.  LDS: nsplit float2.
__global__ void __launch_bounds__(128)
    attn_combine_k(const float *__restrict__ ws, float *__restrict__ out, int hs, int max_splits,
                   int nsplit) {
  extern __shared__ float2 mls[];
  const int h = blockIdx.x, st = hs + 4;
  const float *w = ws + (int64_t)h * max_splits * st;
  for (int s = threadIdx.x; s < nsplit; s += blockDim.x) mls[s] = *(const float2 *)(w + s * st + hs);
  __syncthreads();
  float M = -INFINITY;
  for (int s = 0; s < nsplit; s++) M = fmaxf(M, mls[s].x);
  float L = 0.f;
  for (int s = 0; s < nsplit; s++) L += expf(mls[s].x - M) * mls[s].y;
  const float il = 1.f / L;
  for (int d = threadIdx.x; d < hs; d += blockDim.x) {
    float o = 0.f;
    for (int s0 = 0; s0 < nsplit; s0 += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) v[u] = s0 + u < nsplit ? w[(s0 + u) * st + d] : 0.f;
#pragma unroll
      for (int u = 0; u < 8; u++)
        if (s0 + u < nsplit) o = fmaf(expf(mls[s0 + u].x - M), v[u], o);
    }
    out[h * hs + d] = o * il;
  }
}

// How a step computes attention, chosen on the host from pos; the graph of a
// step is captured once per key:
//   key 0      one 1024-thread block per head (attn_k)
//   key n > 0  attn_split_k over the n chunks of 64 positions that cover
//              [0, pos] (the same n for every pos in [64(n-1), 64n)), then,
//              for n > 1, attn_combine_k
// Workspace floats of the split attention (0: the split kernel is not used).
int64_t attn_ws_floats(int64_t n_heads, int64_t seq_len, int hs) {
  if (hs % 4 != 0 || hs > 128) return 0;
  return n_heads * cdiv(seq_len, kAttnTP) * (hs + 4);
}

// The key for a step at pos: the split kernel alone while one chunk covers the
// context, then split + combine (the split kernel needs head_size % 4 == 0 and
// <= 128; otherwise the one-block kernel).  With the split kernel's
// lane-per-float4 layout this holds for 12 heads of 64 as well: the 110M
// decode (positions 0..287) ran 3021-3031 tok/s against 2974 with the
// one-block kernel up to pos 480, where the earlier split kernel crossed over.
int attn_key(int64_t pos, bool have_ws, int64_t n_heads) {
  (void)n_heads;
  if (!have_ws) return 0;
  return (int)(pos / kAttnTP + 1);
}

// One decode step's attention for one layer (cache rows [seq_len, kv_dim]).
// combine false: with more than one chunk the partials stay in ws for the
// consumer (the Wo GEMV) to combine; out is not written.
int launch_attention(int key, const float *qkv, float *kc, float *vc, float *out, float *ws,
                     const StepState *state, int dim, int kv_dim, int n_heads, int n_kv_heads,
                     int hs, const float2 *rope, int64_t seq_len, hipStream_t st,
                     bool combine = true) {
  if (key == 0) {
    hipLaunchKernelGGL(attn_k, dim3((unsigned)n_heads), dim3(kAttnThreads),
                       sizeof(float) * (size_t)seq_len, st, qkv, kc, vc, out, state, dim, kv_dim,
                       n_heads, n_kv_heads, hs, rope);
  } else {
    const int splits = (int)cdiv(seq_len, kAttnTP);
    if (key > splits) return set_error(SIMP_RT_EINVAL, "attention: %d chunks of %d", key, splits);
    hipLaunchKernelGGL(attn_split_k<kAttnNWV>, dim3((unsigned)n_heads, (unsigned)key),
                       dim3(64 * kAttnNWV), 0, st, qkv, kc, vc, out, ws, state, dim, kv_dim,
                       n_heads, n_kv_heads, hs, rope, splits, key, (int)seq_len);
    if (key > 1 && combine)
      hipLaunchKernelGGL(attn_combine_k, dim3((unsigned)n_heads), dim3(128),
                         sizeof(float2) * (size_t)key, st, (const float *)ws, out, hs, splits, key);
  }
  SIMP_HIP(hipGetLastError());
  return SIMP_RT_OK;
}

// RoPE factors (cos, sin)(pos * freq_j), freq_j = 1 / theta^(j / head_size)
// for even j, as stories110M.sl:86-112 computes them at every step; tabulated
// once per model with the same fp32 expressions, so the values are identical.
__global__ void __launch_bounds__(256)
    rope_table_k(float2 *__restrict__ tab, int seq_len, int hs, float theta) {
  const int half = hs >> 1;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)seq_len * half) return;
  const int pos = (int)(i / half), j = 2 * (int)(i - (int64_t)pos * half);
  const float freq = 1.f / powf(theta, (float)j / (float)hs);
  const float a = (float)pos * freq;
  tab[i] = make_float2(cosf(a), sinf(a));
}

// x = emb[token]. A token outside [0, vocab) (no path writes one: the host
// checks prompts and argmax_advance_k returns an index below vocab) gives a
// NaN row instead of a read outside emb.
__global__ void __launch_bounds__(256)
    embed_k(const float *__restrict__ emb, float *__restrict__ x, const StepState *__restrict__ st,
            int dim, int vocab) {
  const int64_t tok = st->token;
  const bool ok = tok >= 0 && tok < vocab;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < dim; i += gridDim.x * 256)
    x[i] = ok ? emb[tok * dim + i] : __builtin_nanf("");
}

// Greedy argmax and step advance:
//   out_tokens[pos+1] = next = (pos+1 < n_prompt) ? prompt[pos+1] : argmax(logits)
// argmax is sample_argmax of generate_stories110M.cpp:73-83: a scan seeded
// with logits[0] that moves on a strict '>'. NaN compares false, so the scan
// returns 0 when logits[0] is NaN, and otherwise the first index of the
// largest non-NaN value (0 when nothing exceeds logits[0], e.g. all -inf).
// The parallel form: per-thread strict-'>' scans from -inf (NaN never taken),
// ties to the lower index across threads, then 0 when logits[0] is NaN or no
// thread found a value above -inf (the maximum is then logits[0] = -inf).
// The step state, logits[0] and the prompt token of pos + 1 are requested
// before the scan (they are what the last thread's decision waits on), and the
// cross-lane steps are DPP and permlane moves.
__device__ __forceinline__ void argmax_pair(float &best, int &idx, float ov, int oi) {
  if (ov > best || (ov == best && oi < idx)) {
    best = ov;
    idx = oi;
  }
}
template <int CTRL>
__device__ __forceinline__ void argmax_dpp(float &best, int &idx) {
  const float ov = dpp_mov<CTRL>(best);
  const int oi = __builtin_amdgcn_mov_dpp(idx, CTRL, 0xF, 0xF, false);
  argmax_pair(best, idx, ov, oi);
}
__global__ void __launch_bounds__(1024)
    argmax_advance_k(const float *__restrict__ logits, int vocab, StepState *st,
                     const int *__restrict__ prompt, int *__restrict__ out_tokens) {
  __shared__ float bv[16];
  __shared__ int bi[16];
  const int pos0 = st->pos, n_prompt = st->n_prompt, n_total = st->n_total;
  const float l0 = logits[0];
  const int p = pos0 + 1;
  const int ptok = p < n_prompt ? prompt[p] : 0;
  float best = -INFINITY;
  int idx = 0x7fffffff;
  // each thread scans its elements in increasing index order (strict '>' keeps
  // the first maximum); eight float4 loads are issued before they are compared
  const int n4 = ((uintptr_t)logits & 15) == 0 ? vocab >> 2 : 0;
  const float4 *l4 = (const float4 *)logits;
  for (int i0 = threadIdx.x; i0 < n4; i0 += 8 * blockDim.x) {
    float4 v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int i = i0 + u * blockDim.x;
      v[u] = i < n4 ? l4[i] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    }
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int b = 4 * (i0 + u * blockDim.x);
      if (v[u].x > best) { best = v[u].x; idx = b; }
      if (v[u].y > best) { best = v[u].y; idx = b + 1; }
      if (v[u].z > best) { best = v[u].z; idx = b + 2; }
      if (v[u].w > best) { best = v[u].w; idx = b + 3; }
    }
  }
  for (int i = 4 * n4 + threadIdx.x; i < vocab; i += blockDim.x) {
    const float v = logits[i];
    if (v > best) { best = v; idx = i; }  // strictly greater: first max per thread
  }
  // across the wave (each step pairs every lane with one partner, and the
  // pair rule is symmetric, so both end with the same (best, idx))
  argmax_dpp<kDppXor1>(best, idx);
  argmax_dpp<kDppXor2>(best, idx);
  argmax_dpp<kDppHalfMirror>(best, idx);
  argmax_dpp<kDppMirror>(best, idx);
  // rows of 16, then halves of 32: each swap leaves this lane's pair and its
  // partner's in (a, b) in some order
  auto swap_step = [&](auto swapfn) {
    float a = best, b = best, ai = __int_as_float(idx), bi2 = ai;
    swapfn(a, b);
    swapfn(ai, bi2);
    int ni = __float_as_int(ai);
    argmax_pair(a, ni, b, __float_as_int(bi2));
    best = a;
    idx = ni;
  };
  swap_step([](float &a, float &b) { permlane16_swap(a, b); });
  swap_step([](float &a, float &b) { permlane32_swap(a, b); });
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) { bv[wave] = best; bi[wave] = idx; }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b0 = bv[0];
    int i0 = bi[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) argmax_pair(b0, i0, bv[w], bi[w]);
    if (l0 != l0 || i0 >= vocab) i0 = 0;
    const int next = (p < n_prompt) ? ptok : i0;
    if (p < n_total) out_tokens[p] = next;
    st->token = next;
    st->pos = p;
  }
}

}  // namespace

struct LlamaModel {
  simp_rt_llama_config cfg;
  simp_rt_llama_weights w;
  int kv_dim, hs;
  int device;
  hipStream_t stream = nullptr;
  // device buffers
  float *x = nullptr, *xb = nullptr, *qkv = nullptr, *h13 = nullptr, *logits = nullptr;
  float *kcache = nullptr, *vcache = nullptr;
  float2 *rope = nullptr;  // [seq_len][head_size / 2] (cos, sin); null when theta <= 0
  float *attn_ws = nullptr;  // split-attention partials; null: one block per head
  StepState *state = nullptr;
  int *prompt = nullptr, *tokens = nullptr;
  // one captured step per attention key (attn_key)
  std::map<int, std::pair<hipGraph_t, hipGraphExec_t>> graphs;
};

namespace {

// Weight format and launch context of a step's GEMVs.  kFmtW4U: the
// reference W4 format (unsigned nibbles, scale and zero per group), on the
// dot8 kernel only.
constexpr int kFmtW4U = 100;
struct GemvCtx {
  int fmt;  // SIMP_RT_W_F32, SIMP_RT_W_W4S or kFmtW4U
  int gs;
  float eps;
  hipStream_t st;
};


// Whether the Wo GEMV of a step with attention key `attn` takes the partials
// (the other GEMVs read the combine kernel's output).  Every Wo block reads
// all chunks of every head:
//   * W4 (the dot8 kernel): the fold stops paying past four chunks (positions
//     >= 256); measured on the 3B W4 decode at three chunks, Wo 5.0 -> 6.9 us
//     against the 4.0 us combine kernel it replaces.  It also needs what the
//     kernel's prologue assumes: one thread per head (at most 256 heads, the
//     smallest block) and whole float4 groups per head.
//   * fp32 (dgemv_f32's kCombine prologue): dim <= 1024 (four elements per
//     thread) and up to eight chunks (positions < 512).  110M decode: 3110
//     tok/s against 3010-3031 with the combine kernel (and 2934 with a
//     prologue that read the heads' (m, l) chunk by chunk after the weights).
// Any other step takes the separate attn_combine_k launch.
bool fold_combine(int fmt, int gs, int attn, int K, int hs, const float *x0) {
  if (attn <= 1 || hs <= 0 || hs % 4 != 0 || K % hs != 0) return false;
  if (fmt == SIMP_RT_W_F32) return attn <= 8 && K <= 1024;
  return attn <= 4 && K / hs <= 256 && w4d8_supported(K, gs, x0, nullptr);
}

// out_mode kPairSwiGLU: segments 0 and 1 are W1 and W3 (same rows), the
// output is segment 0's.  cp: x combined from attention partials (only where
// fold_combine holds).
int gemv(const GemvCtx &c, Segs sg, int K, int pro, int out_mode, const float *x0, const float *nw,
         const Partials *cp = nullptr) {
  if (cp && (c.fmt == SIMP_RT_W_F32 ? K > 1024 : !w4d8_supported(K, c.gs, x0, nullptr)))
    return set_error(SIMP_RT_EINVAL,
                     "step GEMV: attention partials need the dot8 kernel or fp32 with K <= 1024");
  const Partials pc = cp ? *cp : Partials{nullptr, 1, 1, 0};
  const float eps = c.eps;
  hipStream_t st = c.st;
  const bool pair = out_mode == kPairSwiGLU;
  if (c.fmt == SIMP_RT_W_F32) {
    int total = 0;
    if (pair) total = sg.s[0].rows;
    else for (int i = 0; i < sg.n; i++) total += sg.s[i].rows;
    const unsigned grid = (unsigned)std::min<int64_t>(cdiv(total, 4), (int64_t)num_cus() * 8);
    const size_t shm = sizeof(float) * (size_t)K;
    const int J = (int)cdiv(K / 4, 64);
#define DGJ(P, O, JV, KPV) hipLaunchKernelGGL((dgemv_f32<P, O, JV, KPV>), dim3(grid), dim3(256), shm, st, sg, total, K, x0, nw, eps, pc)
// (paired rows hold two rows of weights per wave: the 16-slot variant is left
// to the loop form there)
#define DG(P, O)                                              \
  do {                                                        \
    if (J <= 4) DGJ(P, O, 4, 4);                              \
    else if (J <= 8) DGJ(P, O, 8, 8);                         \
    else if (J <= 16 && O != kPairSwiGLU) DGJ(P, O, 16, 16);  \
    else DGJ(P, O, 0, 36);                                    \
  } while (0)
    if (cp) DGJ(kCombine, kAccum, 4, 4);  // K <= 1024: J <= 4
    else if (pro == kRmsNorm) { if (pair) DG(kRmsNorm, kPairSwiGLU); else DG(kRmsNorm, kStore); }
    else { if (out_mode == kAccum) DG(kPlain, kAccum); else DG(kPlain, kStore); }
#undef DG
#undef DGJ
  } else if (w4d8_supported(K, c.gs, x0, pro == kRmsNorm ? nw : nullptr)) {
    // exact integer chunk products on v_dot8_i32_i4 (w4d8.hip)
    W4D8Args a{};
    for (int i = 0; i < sg.n; i++)
      a.s[i] = W4D8Seg{(const uint8_t *)sg.s[i].W, sg.s[i].S, sg.s[i].out, K / 2, K / c.gs,
                       sg.s[i].rows, c.fmt == kFmtW4U ? sg.s[i].Z : nullptr};
    a.n = sg.n;
    a.K = K;
    a.gs = c.gs;
    a.x0 = x0;
    a.nw = pro == kRmsNorm ? nw : nullptr;
    a.eps = eps;
    a.out_mode = out_mode;
    if (cp) {
      a.cws = cp->ws;
      a.chs = cp->hs;
      a.cmax = cp->max_splits;
      a.cn = cp->n;
    }
    return launch_w4d8(a, st);
  } else if (c.fmt == kFmtW4U) {
    return set_error(SIMP_RT_EUNSUPPORTED, "step GEMV: reference W4 format needs the dot8 kernel (K=%d)", K);
  } else {
    int tiles = 0;
    if (pair) {
      tiles = (int)cdiv(sg.s[0].rows, 4);
    } else {
      for (int i = 0; i < sg.n; i++) {
        sg.s[i].tile0 = tiles;
        tiles += (int)cdiv(sg.s[i].rows, 8);
      }
    }
    const int gs = c.gs;
    const int nchunk = K / 32;
    // 8 waves per block for rows of more than 64 chunks over fewer than 8
    // blocks per CU: half the serial unpack/FMA work per wave
    const bool wide = nchunk > 64 && tiles < 8 * num_cus();
#define DWU(P, O, U) hipLaunchKernelGGL((dgemv_w4<P, O, U>), dim3(tiles), dim3(256), 0, st, sg, K, gs, x0, nw, eps)
#define DWU8(P, O, U) hipLaunchKernelGGL((dgemv_w4<P, O, U, 8>), dim3(tiles), dim3(512), 0, st, sg, K, gs, x0, nw, eps)
#define DW(P, O)                      \
  do {                                \
    if (wide && nchunk <= 128) DWU8(P, O, 2); \
    else if (wide) DWU8(P, O, 5);     \
    else if (nchunk <= 32) DWU(P, O, 1);   \
    else if (nchunk <= 64) DWU(P, O, 2); \
    else if (nchunk <= 128) DWU(P, O, 4); \
    else if (nchunk <= 256) DWU(P, O, 8); \
    else DWU(P, O, 9);                \
  } while (0)
    if (pro == kRmsNorm) { if (pair) DW(kRmsNorm, kPairSwiGLU); else DW(kRmsNorm, kStore); }
    else { if (out_mode == kAccum) DW(kPlain, kAccum); else DW(kPlain, kStore); }
#undef DW
#undef DWU
#undef DWU8
  }
  SIMP_HIP(hipGetLastError());
  return SIMP_RT_OK;
}

int gemv(LlamaModel &m, Segs sg, int K, int pro, int out_mode, const float *x0, const float *nw,
         const Partials *cp = nullptr) {
  return gemv(GemvCtx{m.cfg.weight_format, m.cfg.group_size, m.cfg.eps, m.stream}, sg, K, pro,
              out_mode, x0, nw, cp);
}

Seg seg_f32(const float *W, float *out, int rows) { return Seg{W, nullptr, out, rows, 0}; }
Seg seg_w4(const uint8_t *W, const float *S, float *out, int rows) { return Seg{W, S, out, rows, 0}; }

// Enqueues one decode step (token and pos read from the device state).
// attn: the attention key of the step's position (attn_key).
int enqueue_step(LlamaModel &m, int attn) {
  const auto &c = m.cfg;
  const int dim = (int)c.dim, hid = (int)c.hidden_dim, kv = m.kv_dim, hs = m.hs;
  const int L = (int)c.n_layers, gs = c.group_size;
  const bool w4 = c.weight_format == SIMP_RT_W_W4S;
  hipStream_t st = m.stream;
  int rc;
  hipLaunchKernelGGL(embed_k, dim3((unsigned)cdiv(dim, 256)), dim3(256), 0, st,
                     m.w.token_embedding, m.x, m.state, dim, (int)c.vocab_size);
  SIMP_HIP(hipGetLastError());
  float *q = m.qkv, *k = m.qkv + dim, *v = m.qkv + dim + kv;
  float *g = m.h13;  // silu(h1) * h3
  for (int l = 0; l < L; l++) {
    const int64_t lq = (int64_t)l * dim * dim, lk = (int64_t)l * kv * dim;
    const int64_t lf = (int64_t)l * hid * dim;
    Segs s{};
    // 1. QKV with the attention RMSNorm
    if (w4) {
      s.s[0] = seg_w4(m.w.q_wq + lq / 2, m.w.s_wq + lq / gs, q, dim);
      s.s[1] = seg_w4(m.w.q_wk + lk / 2, m.w.s_wk + lk / gs, k, kv);
      s.s[2] = seg_w4(m.w.q_wv + lk / 2, m.w.s_wv + lk / gs, v, kv);
    } else {
      s.s[0] = seg_f32(m.w.wq + lq, q, dim);
      s.s[1] = seg_f32(m.w.wk + lk, k, kv);
      s.s[2] = seg_f32(m.w.wv + lk, v, kv);
    }
    s.n = 3;
    if ((rc = gemv(m, s, dim, kRmsNorm, kStore, m.x, m.w.rms_att + (int64_t)l * dim))) return rc;
    // 2. attention (RoPE, cache store at pos, softmax, V sum), one block per
    // head or per chunk of positions; with chunks, the Wo GEMV on the dot8
    // kernel combines them in its prologue
    float *kc = m.kcache + (int64_t)l * c.seq_len * kv, *vc = m.vcache + (int64_t)l * c.seq_len * kv;
    const bool fold = fold_combine(c.weight_format, gs, attn, dim, hs, m.xb);
    if ((rc = launch_attention(attn, m.qkv, kc, vc, m.xb, m.attn_ws, m.state, dim, kv,
                               (int)c.n_heads, (int)c.n_kv_heads, hs, (const float2 *)m.rope,
                               c.seq_len, st, !fold)))
      return rc;
    const Partials parts{m.attn_ws, hs, (int)cdiv(c.seq_len, kAttnTP), attn};
    // 3. Wo, accumulated into x (residual)
    s = Segs{};
    s.s[0] = w4 ? seg_w4(m.w.q_wo + lq / 2, m.w.s_wo + lq / gs, m.x, dim) : seg_f32(m.w.wo + lq, m.x, dim);
    s.n = 1;
    if ((rc = gemv(m, s, dim, kPlain, kAccum, m.xb, nullptr, fold ? &parts : nullptr))) return rc;
    // 4. W1 | W3 with the FFN RMSNorm, rows paired: g = silu(h1) * h3
    s = Segs{};
    if (w4) {
      s.s[0] = seg_w4(m.w.q_w1 + lf / 2, m.w.s_w1 + lf / gs, g, hid);
      s.s[1] = seg_w4(m.w.q_w3 + lf / 2, m.w.s_w3 + lf / gs, nullptr, hid);
    } else {
      s.s[0] = seg_f32(m.w.w1 + lf, g, hid);
      s.s[1] = seg_f32(m.w.w3 + lf, nullptr, hid);
    }
    s.n = 2;
    if ((rc = gemv(m, s, dim, kRmsNorm, kPairSwiGLU, m.x, m.w.rms_ffn + (int64_t)l * dim))) return rc;
    // 5. W2 on g, accumulated into x
    s = Segs{};
    s.s[0] = w4 ? seg_w4(m.w.q_w2 + lf / 2, m.w.s_w2 + lf / gs, m.x, dim) : seg_f32(m.w.w2 + lf, m.x, dim);
    s.n = 1;
    if ((rc = gemv(m, s, hid, kPlain, kAccum, g, nullptr))) return rc;
  }
  // final RMSNorm + classifier
  Segs s{};
  s.s[0] = w4 ? seg_w4(m.w.q_wcls, m.w.s_wcls, m.logits, (int)c.vocab_size)
              : seg_f32(m.w.wcls, m.logits, (int)c.vocab_size);
  s.n = 1;
  if ((rc = gemv(m, s, dim, kRmsNorm, kStore, m.x, m.w.rms_final))) return rc;
  hipLaunchKernelGGL(argmax_advance_k, dim3(1), dim3(1024), 0, st, m.logits, (int)c.vocab_size,
                     m.state, m.prompt, m.tokens);
  SIMP_HIP(hipGetLastError());
  return SIMP_RT_OK;
}

// Captures the step graph of attention key `mode` (once per key) on a
// capture stream; the engine's stream is synchronised first.
int capture_step(LlamaModel &m, int mode) {
  if (m.graphs.count(mode)) return SIMP_RT_OK;
  SIMP_HIP(hipStreamSynchronize(m.stream));
  hipStream_t cap;
  SIMP_HIP(hipStreamCreateWithFlags(&cap, hipStreamNonBlocking));
  hipStream_t saved = m.stream;
  m.stream = cap;
  SIMP_HIP(hipStreamBeginCapture(cap, hipStreamCaptureModeThreadLocal));
  const int rc = enqueue_step(m, mode);
  hipGraph_t g = nullptr;
  const hipError_t e = hipStreamEndCapture(cap, &g);
  m.stream = saved;
  (void)hipStreamDestroy(cap);
  if (rc) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
  hipGraphExec_t ge = nullptr;
  const hipError_t ie = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
  if (ie != hipSuccess) {
    (void)hipGraphDestroy(g);
    return hip_fail(ie, "hipGraphInstantiate");
  }
  m.graphs[mode] = {g, ge};
  return SIMP_RT_OK;
}

int check_cfg(const simp_rt_llama_config &c) {
  if (c.dim <= 0 || c.hidden_dim <= 0 || c.n_layers <= 0 || c.n_heads <= 0 ||
      c.n_kv_heads <= 0 || c.vocab_size <= 0 || c.seq_len <= 0)
    return set_error(SIMP_RT_EINVAL, "llama: non-positive dimension in config");
  if (c.dim % c.n_heads || c.n_heads % c.n_kv_heads || (c.dim / c.n_heads) % 2)
    return set_error(SIMP_RT_EINVAL, "llama: dim must split into even-sized heads, n_heads into kv heads");
  if (c.dim % 4 || c.hidden_dim % 4)
    return set_error(SIMP_RT_EINVAL, "llama: dim and hidden_dim must be multiples of 4");
  if (c.weight_format == SIMP_RT_W_W4S) {
    const int gs = c.group_size;
    const int64_t kv = c.dim * c.n_kv_heads / c.n_heads;
    if (gs <= 0 || gs % 32 || c.dim % gs || c.hidden_dim % gs)
      return set_error(SIMP_RT_EINVAL, "llama W4: group_size must be a multiple of 32 dividing dim and hidden_dim");
    (void)kv;
  } else if (c.weight_format != SIMP_RT_W_F32) {
    return set_error(SIMP_RT_EINVAL, "llama: unknown weight_format %d", c.weight_format);
  }
  const int64_t hs = c.dim / c.n_heads;
  if (hs > 256 || hs % 4)
    return set_error(SIMP_RT_EUNSUPPORTED, "llama: head_size must be a multiple of 4, at most 256");
  if (sizeof(float) * (size_t)(c.seq_len + 3 * 256 + 1024 + 16) > 64 * 1024)
    return set_error(SIMP_RT_EUNSUPPORTED, "llama: seq_len %lld too long for the attention kernel",
                     (long long)c.seq_len);
  if (std::max(c.dim, c.hidden_dim) > 256 * 36)
    return set_error(SIMP_RT_EUNSUPPORTED, "llama: dim and hidden_dim must be at most 9216");
  return SIMP_RT_OK;
}

}  // namespace
}  // namespace simp

using namespace simp;

extern "C" {

int32_t simp_rt_llama_create(const simp_rt_llama_config *cfg, const simp_rt_llama_weights *w,
                             simp_rt_llama **out) {
  if (!cfg || !w || !out) return set_error(SIMP_RT_EINVAL, "llama_create: null argument");
  *out = nullptr;
  int rc;
  if ((rc = check_cfg(*cfg))) return rc;
  const bool w4 = cfg->weight_format == SIMP_RT_W_W4S;
  const void *need[] = {w->token_embedding, w->rms_att, w->rms_ffn, w->rms_final,
                        w4 ? (const void *)w->q_wq : (const void *)w->wq,
                        w4 ? (const void *)w->q_wk : (const void *)w->wk,
                        w4 ? (const void *)w->q_wv : (const void *)w->wv,
                        w4 ? (const void *)w->q_wo : (const void *)w->wo,
                        w4 ? (const void *)w->q_w1 : (const void *)w->w1,
                        w4 ? (const void *)w->q_w2 : (const void *)w->w2,
                        w4 ? (const void *)w->q_w3 : (const void *)w->w3,
                        w4 ? (const void *)w->q_wcls : (const void *)w->wcls};
  for (const void *p : need)
    if (!p) return set_error(SIMP_RT_EINVAL, "llama_create: missing weight pointer");
  if (w4 && (!w->s_wq || !w->s_wk || !w->s_wv || !w->s_wo || !w->s_w1 || !w->s_w2 || !w->s_w3 ||
             !w->s_wcls))
    return set_error(SIMP_RT_EINVAL, "llama_create: missing W4 scales pointer");
  // every weight must already be device-resident (device memory or a registered range)
  const int64_t dim = cfg->dim, hid = cfg->hidden_dim, L = cfg->n_layers, V = cfg->vocab_size;
  const int64_t kvd = dim * cfg->n_kv_heads / cfg->n_heads;
  simp_rt_llama_weights dw = *w;
  struct Need { const void **p; size_t bytes; const char *name; };
  std::vector<Need> needs = {
      {(const void **)&dw.token_embedding, 4 * (size_t)(V * dim), "token_embedding"},
      {(const void **)&dw.rms_att, 4 * (size_t)(L * dim), "rms_att"},
      {(const void **)&dw.rms_ffn, 4 * (size_t)(L * dim), "rms_ffn"},
      {(const void **)&dw.rms_final, 4 * (size_t)dim, "rms_final"}};
  const int64_t mats[8][2] = {{dim, dim}, {kvd, dim}, {kvd, dim}, {dim, dim},
                              {hid, dim}, {dim, hid}, {hid, dim}, {V, dim}};
  const char *names[8] = {"wq", "wk", "wv", "wo", "w1", "w2", "w3", "wcls"};
  const void **fp[8] = {(const void **)&dw.wq, (const void **)&dw.wk, (const void **)&dw.wv,
                        (const void **)&dw.wo, (const void **)&dw.w1, (const void **)&dw.w2,
                        (const void **)&dw.w3, (const void **)&dw.wcls};
  const void **qp[8] = {(const void **)&dw.q_wq, (const void **)&dw.q_wk, (const void **)&dw.q_wv,
                        (const void **)&dw.q_wo, (const void **)&dw.q_w1, (const void **)&dw.q_w2,
                        (const void **)&dw.q_w3, (const void **)&dw.q_wcls};
  const void **sp[8] = {(const void **)&dw.s_wq, (const void **)&dw.s_wk, (const void **)&dw.s_wv,
                        (const void **)&dw.s_wo, (const void **)&dw.s_w1, (const void **)&dw.s_w2,
                        (const void **)&dw.s_w3, (const void **)&dw.s_wcls};
  for (int i = 0; i < 8; i++) {
    const int64_t cnt = mats[i][0] * mats[i][1] * (i == 7 ? 1 : L);
    if (w4) {
      needs.push_back({qp[i], (size_t)(cnt / 2), names[i]});
      needs.push_back({sp[i], 4 * (size_t)(cnt / cfg->group_size), names[i]});
    } else {
      needs.push_back({fp[i], 4 * (size_t)cnt, names[i]});
    }
  }
  for (auto &nd : needs)
    if ((rc = device_view(*nd.p, nd.bytes, nd.p, nd.name))) return rc;
  auto *m = new LlamaModel();
  m->cfg = *cfg;
  m->w = dw;
  m->kv_dim = (int)(cfg->dim * cfg->n_kv_heads / cfg->n_heads);
  m->hs = (int)(cfg->dim / cfg->n_heads);
  m->device = ensure_device();
  m->stream = cur_stream();
  auto alloc = [&](void **p, size_t bytes) -> int {
    hipError_t e = hipMalloc(p, std::max<size_t>(bytes, 16));
    if (e != hipSuccess) return set_error(SIMP_RT_ENOMEM, "llama_create: %s", hipGetErrorString(e));
    return SIMP_RT_OK;
  };
  const size_t kvb = sizeof(float) * (size_t)(cfg->n_layers * cfg->seq_len * m->kv_dim);
  if ((rc = alloc((void **)&m->x, 4 * cfg->dim)) || (rc = alloc((void **)&m->xb, 4 * cfg->dim)) ||
      (rc = alloc((void **)&m->qkv, 4 * (cfg->dim + 2 * m->kv_dim))) ||
      (rc = alloc((void **)&m->h13, 8 * cfg->hidden_dim)) ||
      (rc = alloc((void **)&m->logits, 4 * cfg->vocab_size)) ||
      (rc = alloc((void **)&m->kcache, kvb)) || (rc = alloc((void **)&m->vcache, kvb)) ||
      (rc = alloc((void **)&m->state, sizeof(StepState))) ||
      (rc = alloc((void **)&m->prompt, 4 * cfg->seq_len)) ||
      (rc = alloc((void **)&m->tokens, 4 * cfg->seq_len))) {
    simp_rt_llama_destroy((simp_rt_llama *)m);
    return rc;
  }
  if (const int64_t wsf = attn_ws_floats(cfg->n_heads, cfg->seq_len, m->hs)) {
    if ((rc = alloc((void **)&m->attn_ws, sizeof(float) * (size_t)wsf))) {
      simp_rt_llama_destroy((simp_rt_llama *)m);
      return rc;
    }
    if (hipMemset(m->attn_ws, 0, sizeof(float) * (size_t)wsf) != hipSuccess) {
      simp_rt_llama_destroy((simp_rt_llama *)m);
      return set_error(SIMP_RT_EHIP, "llama_create: attention workspace");
    }
  }
  if (cfg->rope_theta > 0.f) {
    const int64_t n = cfg->seq_len * (m->hs / 2);
    if ((rc = alloc((void **)&m->rope, sizeof(float2) * (size_t)n))) {
      simp_rt_llama_destroy((simp_rt_llama *)m);
      return rc;
    }
    hipLaunchKernelGGL(rope_table_k, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, m->stream, m->rope,
                       (int)cfg->seq_len, m->hs, cfg->rope_theta);
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(m->stream) != hipSuccess) {
      simp_rt_llama_destroy((simp_rt_llama *)m);
      return set_error(SIMP_RT_EHIP, "llama_create: RoPE table");
    }
  }
  *out = (simp_rt_llama *)m;
  return SIMP_RT_OK;
}

int32_t simp_rt_llama_destroy(simp_rt_llama *h) {
  auto *m = (LlamaModel *)h;
  if (!m) return SIMP_RT_OK;
  (void)hipStreamSynchronize(m->stream);
  for (auto &kv : m->graphs) {
    if (kv.second.second) (void)hipGraphExecDestroy(kv.second.second);
    if (kv.second.first) (void)hipGraphDestroy(kv.second.first);
  }
  for (void *p : {(void *)m->x, (void *)m->xb, (void *)m->qkv, (void *)m->h13, (void *)m->logits,
                  (void *)m->kcache, (void *)m->vcache, (void *)m->rope, (void *)m->attn_ws,
                  (void *)m->state,
                  (void *)m->prompt, (void *)m->tokens})
    if (p) (void)hipFree(p);
  delete m;
  return SIMP_RT_OK;
}

int32_t simp_rt_llama_forward(simp_rt_llama *h, int64_t token, int64_t pos, float *logits) {
  auto *m = (LlamaModel *)h;
  if (!m) return set_error(SIMP_RT_EINVAL, "llama_forward: null model");
  if (token < 0 || token >= m->cfg.vocab_size || pos < 0 || pos >= m->cfg.seq_len)
    return set_error(SIMP_RT_EINVAL, "llama_forward: token %lld / pos %lld out of range",
                     (long long)token, (long long)pos);
  m->stream = cur_stream();
  StepState s{(int)token, (int)pos, 0, 0};
  SIMP_HIP(hipMemcpyAsync(m->state, &s, sizeof s, hipMemcpyHostToDevice, m->stream));
  StreamDrain drain{m->stream};  // s is read by the copy until the stream drains
  int rc = enqueue_step(*m, attn_key(pos, m->attn_ws != nullptr, m->cfg.n_heads));
  if (rc) return rc;
  if (logits) {
    Operand ol;
    if ((rc = ol.bind(logits, 4 * (size_t)m->cfg.vocab_size, Operand::kOut, "logits"))) return rc;
    SIMP_HIP(hipMemcpyAsync(ol.dev(), m->logits, 4 * (size_t)m->cfg.vocab_size,
                            hipMemcpyDeviceToDevice, m->stream));
    Operand *ops[] = {&ol};
    if ((rc = finish(ops, 1))) return rc;
  }
  drain.s = nullptr;
  SIMP_HIP(hipStreamSynchronize(m->stream));
  return SIMP_RT_OK;
}

int32_t simp_rt_llama_generate(simp_rt_llama *h, const int32_t *prompt, int64_t n_prompt,
                               int64_t n_new, int32_t *out_tokens, int32_t use_graph) {
  auto *m = (LlamaModel *)h;
  if (!m || !prompt || !out_tokens) return set_error(SIMP_RT_EINVAL, "llama_generate: null argument");
  if (n_prompt <= 0 || n_new < 0 || n_prompt + n_new > m->cfg.seq_len)
    return set_error(SIMP_RT_EINVAL, "llama_generate: n_prompt %lld + n_new %lld exceeds seq_len %lld",
                     (long long)n_prompt, (long long)n_new, (long long)m->cfg.seq_len);
  for (int64_t i = 0; i < n_prompt; i++)
    if (prompt[i] < 0 || prompt[i] >= m->cfg.vocab_size)
      return set_error(SIMP_RT_EINVAL, "llama_generate: prompt token %lld out of range", (long long)i);
  m->stream = cur_stream();
  hipStream_t st = m->stream;
  const int64_t total = n_prompt + n_new;
  SIMP_HIP(hipMemcpyAsync(m->prompt, prompt, 4 * (size_t)n_prompt, hipMemcpyHostToDevice, st));
  SIMP_HIP(hipMemcpyAsync(m->tokens, prompt, 4 * (size_t)n_prompt, hipMemcpyHostToDevice, st));
  StepState s{prompt[0], 0, (int)n_prompt, (int)total};
  SIMP_HIP(hipMemcpyAsync(m->state, &s, sizeof s, hipMemcpyHostToDevice, st));
  StreamDrain drain{st};  // s and the caller's arrays are read until the stream drains
  int rc;
  const int64_t steps = total - 1;  // the last sampled token needs no forward pass
  // step i runs at pos i
  auto mode_of = [&](int64_t i) { return attn_key(i, m->attn_ws != nullptr, m->cfg.n_heads); };
  if (use_graph) {
    for (int64_t i = 0; i < steps; i++)  // capture every key the run needs up front
      if ((rc = capture_step(*m, mode_of(i)))) return rc;
    for (int64_t i = 0; i < steps; i++)
      SIMP_HIP(hipGraphLaunch(m->graphs[mode_of(i)].second, st));
  } else {
    for (int64_t i = 0; i < steps; i++)
      if ((rc = enqueue_step(*m, mode_of(i)))) return rc;
  }
  SIMP_HIP(hipMemcpyAsync(out_tokens, m->tokens, 4 * (size_t)total, hipMemcpyDeviceToHost, st));
  drain.s = nullptr;
  SIMP_HIP(hipStreamSynchronize(st));
  return SIMP_RT_OK;
}

}  // extern "C"

// ------------------------------------------------- model-level drop-in exports
// stories110M_forward with the signature of the compiled program
// (examples/llama2/stories110M.sl:5-44 as bound by
// examples/llama2/generate_stories110M.cpp:15-21,136): every array is a rank-1
// memref descriptor, the call computes one token and returns logits[0].
namespace simp {
namespace {

// One engine instance per (weights, config) seen by a model-level export:
// the engine, the device copies of host weights and the KV continuity state
// (export_state.hip).  At most kMaxEntries engines are kept; the least recently
// used one is freed to make room (a host that frees its model and loads
// another at new addresses leaves an entry that is never called again).
// What a model-level export hands back per call: logits and the K/V rows of
// the step's position in every layer.  Destinations in host memory are filled
// through one pinned buffer -- device -> pinned copies on the stream, host
// memcpy once it has synchronised -- since a 2-D copy into pageable memory is
// staged row by row.  The same buffer holds the step state the call uploads.
class StepIO {
 public:
  void release() {
    if (buf_) (void)hipHostFree(buf_);
    buf_ = nullptr;
    cap_ = 0;
  }
  // token and pos into the device state, asynchronously on st
  int upload_state(int64_t token, int64_t pos, StepState *dev, hipStream_t st) {
    int rc;
    if ((rc = reserve(0))) return rc;
    auto *hs = (StepState *)buf_;
    *hs = StepState{(int)token, (int)pos, 0, 0};
    SIMP_HIP(hipMemcpyAsync(dev, hs, sizeof(StepState), hipMemcpyHostToDevice, st));
    return SIMP_RT_OK;
  }
  // Copies lg_bytes of logits and L rows of `row` bytes (`pitch` apart) of K
  // and V to the caller's arrays, then synchronises st; *first gets logits[0]
  // (from the same device logits, through the pinned buffer, so the call's
  // return value needs no copy of its own).
  int copy_back(void *lg_dst, const void *lg_src, size_t lg_bytes, char *k_dst, char *v_dst,
                const char *k_src, const char *v_src, size_t row, size_t pitch, int64_t L,
                hipStream_t st, float *first) {
    const void *dv;
    const size_t span = (size_t)(L - 1) * pitch + row;
    const bool lg_host = !try_device_view(lg_dst, lg_bytes, &dv);
    const bool kv_host = !try_device_view(k_dst, span, &dv) || !try_device_view(v_dst, span, &dv);
    const size_t o_lg = kHead, o_k = o_lg + (lg_host ? align(lg_bytes) : 0);
    const size_t o_v = o_k + (kv_host ? align((size_t)L * row) : 0);
    const size_t need = o_v + (kv_host ? (size_t)L * row : 0);
    int rc;
    if ((rc = reserve(need))) return rc;
    if (lg_host) SIMP_HIP(hipMemcpyAsync(buf_ + o_lg, lg_src, lg_bytes, hipMemcpyDeviceToHost, st));
    else SIMP_HIP(hipMemcpyAsync(lg_dst, lg_src, lg_bytes, hipMemcpyDefault, st));
    if (kv_host) {
      SIMP_HIP(hipMemcpy2DAsync(buf_ + o_k, row, k_src, pitch, row, (size_t)L, hipMemcpyDeviceToHost, st));
      SIMP_HIP(hipMemcpy2DAsync(buf_ + o_v, row, v_src, pitch, row, (size_t)L, hipMemcpyDeviceToHost, st));
    } else {
      SIMP_HIP(hipMemcpy2DAsync(k_dst, pitch, k_src, pitch, row, (size_t)L, hipMemcpyDefault, st));
      SIMP_HIP(hipMemcpy2DAsync(v_dst, pitch, v_src, pitch, row, (size_t)L, hipMemcpyDefault, st));
    }
    if (!lg_host) SIMP_HIP(hipMemcpyAsync(buf_ + kFirst, lg_src, sizeof(float), hipMemcpyDeviceToHost, st));
    SIMP_HIP(hipStreamSynchronize(st));
    std::memcpy(first, lg_host ? buf_ + o_lg : buf_ + kFirst, sizeof(float));
    if (lg_host) std::memcpy(lg_dst, buf_ + o_lg, lg_bytes);
    if (kv_host)
      for (int64_t l = 0; l < L; l++) {
        std::memcpy(k_dst + l * pitch, buf_ + o_k + l * row, row);
        std::memcpy(v_dst + l * pitch, buf_ + o_v + l * row, row);
      }
    return SIMP_RT_OK;
  }

 private:
  static constexpr size_t kHead = 256;   // the state slot and logits[0]
  static constexpr size_t kFirst = 64;   // logits[0] within the head
  static size_t align(size_t n) { return (n + 255) & ~(size_t)255; }
  int reserve(size_t n) {
    n = std::max(n, kHead);
    if (n <= cap_) return SIMP_RT_OK;
    release();
    if (hipHostMalloc((void **)&buf_, n, hipHostMallocDefault) != hipSuccess) {
      buf_ = nullptr;
      return set_error(SIMP_RT_ENOMEM, "model export: %zu bytes of pinned staging", n);
    }
    cap_ = n;
    return SIMP_RT_OK;
  }
  char *buf_ = nullptr;
  size_t cap_ = 0;
};

struct ForwardEntry {
  simp_rt_llama *model = nullptr;
  ExportWeights weights;
  KvState kv;
  StepIO io;
  uint64_t last_use = 0;
};
constexpr size_t kMaxEntries = 4;
std::mutex g_fwd_mu;
std::map<std::vector<int64_t>, ForwardEntry> g_fwd;
uint64_t g_fwd_clock = 0;

void forward_entry_free(ForwardEntry &e) {
  if (e.model) simp_rt_llama_destroy(e.model);
  e.model = nullptr;
  e.weights.release();
  e.io.release();
}

}  // namespace

// Frees the least recently used entry of `map` while it holds `cap` or more.
template <class Map, class Free>
void evict_lru(Map &map, size_t cap, Free free_entry) {
  while (map.size() >= cap) {
    auto old = map.begin();
    for (auto it = map.begin(); it != map.end(); ++it)
      if (it->second.last_use < old->second.last_use) old = it;
    (void)hipDeviceSynchronize();
    free_entry(old->second);
    map.erase(old);
  }
}

}  // namespace simp

extern "C" {

#define SIMP_DESC_F32(n) float *n##_alloc, float *n, int64_t n##_off, int64_t n##_size, int64_t n##_stride

float stories110M_forward(
    SIMP_DESC_F32(token_embedding_table), SIMP_DESC_F32(rms_att_w), SIMP_DESC_F32(wq),
    SIMP_DESC_F32(wk), SIMP_DESC_F32(wv), SIMP_DESC_F32(wo), SIMP_DESC_F32(rms_ffn_w),
    SIMP_DESC_F32(w1), SIMP_DESC_F32(w2), SIMP_DESC_F32(w3), SIMP_DESC_F32(rms_final_w),
    SIMP_DESC_F32(wcls), SIMP_DESC_F32(x), SIMP_DESC_F32(xb), SIMP_DESC_F32(xb2), SIMP_DESC_F32(hb),
    SIMP_DESC_F32(hb_silu), SIMP_DESC_F32(q), SIMP_DESC_F32(k), SIMP_DESC_F32(v),
    SIMP_DESC_F32(att), SIMP_DESC_F32(att_soft), SIMP_DESC_F32(logits), SIMP_DESC_F32(key_cache),
    SIMP_DESC_F32(value_cache), int64_t token, int64_t pos, int64_t dim, int64_t hidden_dim,
    int64_t n_layers, int64_t n_heads, int64_t n_kv_heads, int64_t vocab_size, int64_t seq_len) {
  const float nan = std::numeric_limits<float>::quiet_NaN();
  clear_error();
  // the scratch activations of the program (x ... att_soft) are not used: the
  // engine keeps its own device buffers and leaves the caller's unchanged
  (void)x; (void)xb; (void)xb2; (void)hb; (void)hb_silu; (void)q; (void)k; (void)v; (void)att;
  (void)att_soft;
  simp_rt_llama_config cfg{};
  cfg.dim = dim;
  cfg.hidden_dim = hidden_dim;
  cfg.n_layers = n_layers;
  cfg.n_heads = n_heads;
  cfg.n_kv_heads = n_kv_heads;
  cfg.vocab_size = vocab_size;
  cfg.seq_len = seq_len;
  cfg.eps = 1e-5f;         // stories110M.sl:61,185,235
  cfg.rope_theta = 10000.f;  // stories110M.sl:86-112
  cfg.weight_format = SIMP_RT_W_F32;
  cfg.group_size = 32;
  if (check_cfg(cfg)) return nan;
  const int64_t L = n_layers, D = dim, H = hidden_dim, V = vocab_size;
  const int64_t kvd = D * n_kv_heads / n_heads;
  struct In { const float *p; int64_t off, size, stride, need; const char *name; };
  const In ins[] = {
      {token_embedding_table, token_embedding_table_off, token_embedding_table_size,
       token_embedding_table_stride, V * D, "token_embedding_table"},
      {rms_att_w, rms_att_w_off, rms_att_w_size, rms_att_w_stride, L * D, "rms_att_w"},
      {wq, wq_off, wq_size, wq_stride, L * D * D, "wq"},
      {wk, wk_off, wk_size, wk_stride, L * kvd * D, "wk"},
      {wv, wv_off, wv_size, wv_stride, L * kvd * D, "wv"},
      {wo, wo_off, wo_size, wo_stride, L * D * D, "wo"},
      {rms_ffn_w, rms_ffn_w_off, rms_ffn_w_size, rms_ffn_w_stride, L * D, "rms_ffn_w"},
      {w1, w1_off, w1_size, w1_stride, L * H * D, "w1"},
      {w2, w2_off, w2_size, w2_stride, L * D * H, "w2"},
      {w3, w3_off, w3_size, w3_stride, L * H * D, "w3"},
      {rms_final_w, rms_final_w_off, rms_final_w_size, rms_final_w_stride, D, "rms_final_w"},
      {wcls, wcls_off, wcls_size, wcls_stride, V * D, "wcls"},
      {logits, logits_off, logits_size, logits_stride, V, "logits"},
      {key_cache, key_cache_off, key_cache_size, key_cache_stride, L * seq_len * kvd, "key_cache"},
      {value_cache, value_cache_off, value_cache_size, value_cache_stride, L * seq_len * kvd,
       "value_cache"}};
  for (const In &a : ins) {
    if (check_desc1(a.name, a.p, a.off, a.size, a.stride)) return nan;
    if (a.size < a.need) {
      set_error(SIMP_RT_EINVAL, "stories110M_forward: %s has %lld elements, needs %lld", a.name,
                (long long)a.size, (long long)a.need);
      return nan;
    }
  }
  if (token < 0 || token >= V || pos < 0 || pos >= seq_len) {
    set_error(SIMP_RT_EINVAL, "stories110M_forward: token %lld / pos %lld out of range",
              (long long)token, (long long)pos);
    return nan;
  }
  const float *wp[12];
  for (int i = 0; i < 12; i++) wp[i] = ins[i].p + ins[i].off;
  std::vector<int64_t> key = {dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len};
  for (int i = 0; i < 12; i++) key.push_back((int64_t)(uintptr_t)wp[i]);
  // One caller at a time per process: the entry's engine, copies and KV state
  // are shared by every thread that passes these arrays.
  std::lock_guard<std::mutex> lk(g_fwd_mu);
  auto it = g_fwd.find(key);
  if (it == g_fwd.end()) {
    evict_lru(g_fwd, kMaxEntries, forward_entry_free);
    it = g_fwd.emplace(key, ForwardEntry{}).first;
    ForwardEntry &e = it->second;
    const void *d[12];
    for (int i = 0; i < 12; i++)
      if (e.weights.bind(wp[i], 4 * (size_t)ins[i].need, &d[i], ins[i].name)) {
        forward_entry_free(e);
        g_fwd.erase(it);
        return nan;
      }
    simp_rt_llama_weights w{};
    w.token_embedding = (const float *)d[0];
    w.rms_att = (const float *)d[1];
    w.wq = (const float *)d[2];
    w.wk = (const float *)d[3];
    w.wv = (const float *)d[4];
    w.wo = (const float *)d[5];
    w.rms_ffn = (const float *)d[6];
    w.w1 = (const float *)d[7];
    w.w2 = (const float *)d[8];
    w.w3 = (const float *)d[9];
    w.rms_final = (const float *)d[10];
    w.wcls = (const float *)d[11];
    if (simp_rt_llama_create(&cfg, &w, &e.model)) {
      e.model = nullptr;
      forward_entry_free(e);
      g_fwd.erase(it);
      return nan;
    }
  }
  ForwardEntry &ent = it->second;
  ent.last_use = ++g_fwd_clock;
  auto *m = (LlamaModel *)ent.model;
  m->stream = cur_stream();
  const size_t pitch = 4 * (size_t)(seq_len * kvd), row = 4 * (size_t)kvd;
  const size_t at = (size_t)(pos * kvd);
  // the program reads the caches' rows [0, pos) and every weight on each call
  bool restart = false;
  if (ent.kv.prepare(pos, key_cache + key_cache_off, value_cache + value_cache_off, m->kcache,
                     m->vcache, row, pitch, L, m->stream, &restart) ||
      ent.weights.verify(restart))
    return nan;
  float *lg = logits + logits_off;
  // the step as its captured graph (token and pos through the device state),
  // then the logits and the step's K and V rows at pos back into the caller's
  // arrays ([n_layers, seq_len, kv_dim], stories110M.sl:115-121)
  const int mode = attn_key(pos, m->attn_ws != nullptr, m->cfg.n_heads);
  if (capture_step(*m, mode) || ent.io.upload_state(token, pos, m->state, m->stream)) return nan;
  if (hipGraphLaunch(m->graphs[mode].second, m->stream) != hipSuccess) {
    hip_fail(hipGetLastError(), "stories110M_forward: hipGraphLaunch");
    return nan;
  }
  float l0 = nan;
  if (ent.io.copy_back(lg, m->logits, 4 * (size_t)vocab_size, (char *)(key_cache + key_cache_off + at),
                       (char *)(value_cache + value_cache_off + at), (const char *)(m->kcache + at),
                       (const char *)(m->vcache + at), row, pitch, L, m->stream, &l0))
    return nan;
  ent.kv.done(pos);
  return l0;
}

#undef SIMP_DESC_F32


}  // extern "C"

// llama2_quant_forward (examples/llama2/llama2_quant.sl:7-56 as bound by
// examples/llama2/bench_llama_quant.cpp:15-24,320): the reference W4 program.
// Its seven layer matrices are in the reference format (one flat nibble array,
// u4 with a scale and zero per flat group of group_size, per-matrix element
// offsets advanced per layer), the classifier is fp32 and there is no RoPE.
// Dims come from the arguments (the program hard-codes 1536/6144/128).
// Where the offsets, group size and dims allow (quant_fusable), the step is
// the engine's fused form -- RMSNorm in the QKV and W1|W3 GEMV prologues, Wq|Wk|Wv
// and W1|W3 as one launch each, residual adds and SwiGLU in the epilogues --
// on the dot8 GEMV with the format's unsigned nibbles and zeros, captured
// once per attention key as a graph and replayed per call; otherwise it runs
// as a sequence of the library's kernels (quant_step).
namespace simp {
namespace {

__global__ void __launch_bounds__(256) add_inplace_k(float *__restrict__ x, const float *__restrict__ y, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) x[i] = x[i] + y[i];
}

// hb = silu(hb) * hb2  (llama2_quant.sl:163-169)
__global__ void __launch_bounds__(256) swiglu_inplace_k(float *__restrict__ hb, const float *__restrict__ hb2, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) {
    const float g = hb[i];
    hb[i] = (g / (1.f + expf(-g))) * hb2[i];
  }
}

struct QuantModel {
  int64_t dim, hid, L, nh, nkv, V, seq, gs, off[7];
  int kv_dim, hs;
  const float *emb, *rms_att, *rms_ffn, *rms_final, *wcls, *scales, *zeros;
  const uint8_t *qw;
  float *x = nullptr, *xb = nullptr, *xb2 = nullptr, *qkv = nullptr, *hb = nullptr, *hb2 = nullptr,
        *logits = nullptr, *kc = nullptr, *vc = nullptr, *attn_ws = nullptr;
  StepState *state = nullptr;
  ExportWeights weights;
  KvState kv;
  uint64_t last_use = 0;
  bool fused = false;
  std::map<int, std::pair<hipGraph_t, hipGraphExec_t>> graphs;  // per attention key
  StepIO io;
};

void quant_free(QuantModel &m) {
  for (auto &g : m.graphs) {
    if (g.second.second) (void)hipGraphExecDestroy(g.second.second);
    if (g.second.first) (void)hipGraphDestroy(g.second.first);
  }
  m.graphs.clear();
  for (void *p : {(void *)m.x, (void *)m.xb, (void *)m.xb2, (void *)m.qkv, (void *)m.hb,
                  (void *)m.hb2, (void *)m.logits, (void *)m.kc, (void *)m.vc, (void *)m.attn_ws,
                  (void *)m.state})
    if (p) (void)hipFree(p);
  m.x = m.xb = m.xb2 = m.qkv = m.hb = m.hb2 = m.logits = m.kc = m.vc = m.attn_ws = nullptr;
  m.state = nullptr;
  m.weights.release();
  m.io.release();
}

int quant_alloc(QuantModel &m) {
  const size_t kv = (size_t)(m.L * m.seq * m.kv_dim);
  struct B { float **p; size_t n; };
  const B bufs[] = {{&m.x, (size_t)m.dim}, {&m.xb, (size_t)m.dim}, {&m.xb2, (size_t)m.dim},
                    {&m.qkv, (size_t)(m.dim + 2 * m.kv_dim)}, {&m.hb, (size_t)m.hid},
                    {&m.hb2, (size_t)m.hid}, {&m.logits, (size_t)m.V}, {&m.kc, kv}, {&m.vc, kv}};
  for (const B &b : bufs) {
    if (hipMalloc((void **)b.p, 4 * b.n) != hipSuccess)
      return set_error(SIMP_RT_ENOMEM, "llama2_quant_forward: device buffers");
    SIMP_HIP(hipMemset(*b.p, 0, 4 * b.n));
  }
  if (hipMalloc((void **)&m.state, sizeof(StepState)) != hipSuccess)
    return set_error(SIMP_RT_ENOMEM, "llama2_quant_forward: device buffers");
  if (const int64_t wsf = attn_ws_floats(m.nh, m.seq, m.hs)) {
    if (hipMalloc((void **)&m.attn_ws, sizeof(float) * (size_t)wsf) != hipSuccess)
      return set_error(SIMP_RT_ENOMEM, "llama2_quant_forward: device buffers");
    SIMP_HIP(hipMemset(m.attn_ws, 0, sizeof(float) * (size_t)wsf));
  }
  return SIMP_RT_OK;
}

int quant_step(QuantModel &m, int64_t token, int64_t pos, hipStream_t st) {
  const int dim = (int)m.dim, hid = (int)m.hid, kvd = m.kv_dim, gs = (int)m.gs;
  const float eps = 1e-5f;  // llama2_quant.sl:73,146,184
  int rc;
  // from the pinned staging buffer: the copy may still be pending on return
  if ((rc = m.io.upload_state(token, pos, m.state, st))) return rc;
  SIMP_HIP(hipMemcpyAsync(m.x, m.emb + token * m.dim, 4 * (size_t)dim, hipMemcpyDeviceToDevice, st));
  const unsigned gd = (unsigned)cdiv(dim, 256), gh = (unsigned)cdiv(hid, 256);
  for (int64_t l = 0; l < m.L; l++) {
    if ((rc = launch_rmsnorm(m.x, m.rms_att + l * dim, m.xb, dim, eps, st))) return rc;
    if ((rc = launch_w4u(m.qw, m.scales, m.zeros, m.xb, m.qkv, dim, dim, gs, m.off[0] + l * m.dim * m.dim, st))) return rc;
    if ((rc = launch_w4u(m.qw, m.scales, m.zeros, m.xb, m.qkv + dim, kvd, dim, gs, m.off[1] + l * m.dim * kvd, st))) return rc;
    if ((rc = launch_w4u(m.qw, m.scales, m.zeros, m.xb, m.qkv + dim + kvd, kvd, dim, gs, m.off[2] + l * m.dim * kvd, st))) return rc;
    float *kc = m.kc + l * m.seq * kvd, *vc = m.vc + l * m.seq * kvd;
    if ((rc = launch_attention(attn_key(pos, m.attn_ws != nullptr, m.nh), m.qkv, kc, vc, m.xb2,
                               m.attn_ws, m.state, dim, kvd, (int)m.nh,
                               (int)m.nkv, m.hs, nullptr, m.seq, st)))  // llama2_quant.sl: no RoPE
      return rc;
    if ((rc = launch_w4u(m.qw, m.scales, m.zeros, m.xb2, m.xb, dim, dim, gs, m.off[3] + l * m.dim * m.dim, st))) return rc;
    hipLaunchKernelGGL(add_inplace_k, dim3(gd), dim3(256), 0, st, m.x, (const float *)m.xb, dim);
    if ((rc = launch_rmsnorm(m.x, m.rms_ffn + l * dim, m.xb, dim, eps, st))) return rc;
    if ((rc = launch_w4u(m.qw, m.scales, m.zeros, m.xb, m.hb, hid, dim, gs, m.off[4] + l * m.hid * m.dim, st))) return rc;
    if ((rc = launch_w4u(m.qw, m.scales, m.zeros, m.xb, m.hb2, hid, dim, gs, m.off[6] + l * m.hid * m.dim, st))) return rc;
    hipLaunchKernelGGL(swiglu_inplace_k, dim3(gh), dim3(256), 0, st, m.hb, (const float *)m.hb2, hid);
    if ((rc = launch_w4u(m.qw, m.scales, m.zeros, m.hb, m.xb, dim, hid, gs, m.off[5] + l * m.dim * m.hid, st))) return rc;
    hipLaunchKernelGGL(add_inplace_k, dim3(gd), dim3(256), 0, st, m.x, (const float *)m.xb, dim);
    SIMP_HIP(hipGetLastError());
  }
  if ((rc = launch_rmsnorm(m.x, m.rms_final, m.xb, dim, eps, st))) return rc;
  return launch_matmul_f32(m.wcls, dim, m.xb, 1, m.logits, 1, (int)m.V, 1, dim, 0.f, st);
}

// Whether the fused step applies: groups that start at row starts (offsets
// and dims multiples of gs, gs a multiple of 32), rows the dot8 kernel takes
// (K / 32 <= 640), 16-byte aligned operands, a classifier row the fp32 GEMV
// holds in LDS.
bool quant_fusable(const QuantModel &m) {
  const int64_t gs = m.gs;
  if (gs % 32 || m.dim % gs || m.hid % gs || m.dim > 9216 || m.hid / 32 > 640) return false;
  for (int i = 0; i < 7; i++)
    if (m.off[i] % gs || m.off[i] % 32) return false;
  for (const void *p : {(const void *)m.qw, (const void *)m.rms_att, (const void *)m.rms_ffn,
                        (const void *)m.rms_final, (const void *)m.wcls})
    if ((uintptr_t)p & 15) return false;
  return true;
}

// One fused step on st (token and pos read from the device state): the
// kernels of enqueue_step on the reference W4 format, no RoPE, fp32
// classifier, logits left in m.logits.
int quant_enqueue_fused(QuantModel &m, int attn, hipStream_t st) {
  const int dim = (int)m.dim, hid = (int)m.hid, kvd = m.kv_dim, gs = (int)m.gs;
  const float eps = 1e-5f;  // llama2_quant.sl:73,146,184
  const GemvCtx cq{kFmtW4U, gs, eps, st};
  hipLaunchKernelGGL(embed_k, dim3((unsigned)cdiv(dim, 256)), dim3(256), 0, st, m.emb, m.x, m.state, dim,
                     (int)m.V);
  SIMP_HIP(hipGetLastError());
  // matrix i of layer l: element offset off[i] + l * per (a multiple of gs)
  auto seg = [&](int i, int64_t l, int64_t per, float *out, int rows) {
    const int64_t e = m.off[i] + l * per;
    Seg s{m.qw + e / 2, m.scales + e / gs, out, rows, 0};
    s.Z = m.zeros + e / gs;
    return s;
  };
  const int64_t D = m.dim, H = m.hid, KV = kvd;
  float *q = m.qkv, *k = m.qkv + dim, *v = m.qkv + dim + kvd;
  int rc;
  for (int64_t l = 0; l < m.L; l++) {
    Segs s{};
    s.s[0] = seg(0, l, D * D, q, dim);
    s.s[1] = seg(1, l, D * KV, k, kvd);
    s.s[2] = seg(2, l, D * KV, v, kvd);
    s.n = 3;
    if ((rc = gemv(cq, s, dim, kRmsNorm, kStore, m.x, m.rms_att + l * dim))) return rc;
    float *kc = m.kc + l * m.seq * kvd, *vc = m.vc + l * m.seq * kvd;
    const bool fold = fold_combine(kFmtW4U, gs, attn, dim, (int)m.hs, m.xb2);
    if ((rc = launch_attention(attn, m.qkv, kc, vc, m.xb2, m.attn_ws, m.state, dim, kvd, (int)m.nh,
                               (int)m.nkv, m.hs, nullptr, m.seq, st, !fold)))  // llama2_quant.sl: no RoPE
      return rc;
    const Partials parts{m.attn_ws, m.hs, (int)cdiv(m.seq, kAttnTP), attn};
    s = Segs{};
    s.s[0] = seg(3, l, D * D, m.x, dim);  // x += Wo xb2
    s.n = 1;
    if ((rc = gemv(cq, s, dim, kPlain, kAccum, m.xb2, nullptr, fold ? &parts : nullptr))) return rc;
    s = Segs{};
    s.s[0] = seg(4, l, H * D, m.hb, hid);  // hb = silu(W1 xb) * (W3 xb)
    s.s[1] = seg(6, l, H * D, nullptr, hid);
    s.n = 2;
    if ((rc = gemv(cq, s, dim, kRmsNorm, kPairSwiGLU, m.x, m.rms_ffn + l * dim))) return rc;
    s = Segs{};
    s.s[0] = seg(5, l, D * H, m.x, dim);  // x += W2 hb
    s.n = 1;
    if ((rc = gemv(cq, s, hid, kPlain, kAccum, m.hb, nullptr))) return rc;
  }
  Segs s{};
  s.s[0] = seg_f32(m.wcls, m.logits, (int)m.V);
  s.n = 1;
  return gemv(GemvCtx{SIMP_RT_W_F32, gs, eps, st}, s, dim, kRmsNorm, kStore, m.x, m.rms_final);
}

// One token: the fused step as a captured graph (once per attention key),
// else the kernel sequence.
int quant_forward_device(QuantModel &m, int64_t token, int64_t pos, hipStream_t st) {
  if (!m.fused) return quant_step(m, token, pos, st);
  int rc;
  if ((rc = m.io.upload_state(token, pos, m.state, st))) return rc;
  const int key = attn_key(pos, m.attn_ws != nullptr, m.nh);
  auto it = m.graphs.find(key);
  if (it == m.graphs.end()) {
    SIMP_HIP(hipStreamSynchronize(st));
    hipStream_t cap;
    SIMP_HIP(hipStreamCreateWithFlags(&cap, hipStreamNonBlocking));
    SIMP_HIP(hipStreamBeginCapture(cap, hipStreamCaptureModeThreadLocal));
    rc = quant_enqueue_fused(m, key, cap);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(cap, &g);
    (void)hipStreamDestroy(cap);
    if (rc) {
      if (g) (void)hipGraphDestroy(g);
      return rc;
    }
    if (e != hipSuccess) return hip_fail(e, "llama2_quant_forward: hipStreamEndCapture");
    hipGraphExec_t ge = nullptr;
    const hipError_t ie = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    if (ie != hipSuccess) {
      (void)hipGraphDestroy(g);
      return hip_fail(ie, "llama2_quant_forward: hipGraphInstantiate");
    }
    it = m.graphs.emplace(key, std::make_pair(g, ge)).first;
  }
  SIMP_HIP(hipGraphLaunch(it->second.second, st));
  return SIMP_RT_OK;
}

std::map<std::vector<int64_t>, QuantModel> g_qfwd;

}  // namespace
}  // namespace simp

extern "C" {

#define SIMP_DESC_F32(n) float *n##_alloc, float *n, int64_t n##_off, int64_t n##_size, int64_t n##_stride
#define SIMP_DESC_I8(n) int8_t *n##_alloc, int8_t *n, int64_t n##_off, int64_t n##_size, int64_t n##_stride

float llama2_quant_forward(
    SIMP_DESC_F32(token_emb), SIMP_DESC_F32(rms_att_w), SIMP_DESC_F32(rms_ffn_w),
    SIMP_DESC_F32(rms_final_w), SIMP_DESC_F32(wcls), SIMP_DESC_I8(qweights), SIMP_DESC_F32(scales),
    SIMP_DESC_F32(zeros), SIMP_DESC_F32(x), SIMP_DESC_F32(xb), SIMP_DESC_F32(xb2), SIMP_DESC_F32(q),
    SIMP_DESC_F32(k), SIMP_DESC_F32(v), SIMP_DESC_F32(att), SIMP_DESC_F32(att_soft),
    SIMP_DESC_F32(hb), SIMP_DESC_F32(hb_silu), SIMP_DESC_F32(hb2), SIMP_DESC_F32(logits),
    SIMP_DESC_F32(key_cache), SIMP_DESC_F32(value_cache), int64_t token, int64_t pos,
    int64_t dim, int64_t hidden_dim, int64_t n_layers, int64_t n_heads, int64_t n_kv_heads,
    int64_t vocab_size, int64_t seq_len, int64_t group_size, int64_t wq_off, int64_t wk_off,
    int64_t wv_off, int64_t wo_off, int64_t w1_off, int64_t w2_off, int64_t w3_off) {
  const float nan = std::numeric_limits<float>::quiet_NaN();
  clear_error();
  (void)x; (void)xb; (void)xb2; (void)q; (void)k; (void)v; (void)att; (void)att_soft; (void)hb;
  (void)hb_silu; (void)hb2;
  auto fail = [&](const char *msg) {
    set_error(SIMP_RT_EINVAL, "llama2_quant_forward: %s", msg);
    return nan;
  };
  if (dim <= 0 || hidden_dim <= 0 || n_layers <= 0 || n_heads <= 0 || n_kv_heads <= 0 ||
      vocab_size <= 0 || seq_len <= 0 || dim % n_heads || n_heads % n_kv_heads)
    return fail("bad model dimensions");
  const int64_t hs = dim / n_heads, kvd = dim * n_kv_heads / n_heads;
  if (hs % 4 || hs > 256 || 4 * seq_len > 64 * 1024 || dim > INT32_MAX || hidden_dim > INT32_MAX)
    return fail("head_size must be a multiple of 4 and <= 256, seq_len <= 16384");
  if (group_size <= 0) return fail("group_size must be positive");
  if (token < 0 || token >= vocab_size || pos < 0 || pos >= seq_len)
    return fail("token or pos out of range");
  const int64_t L = n_layers, D = dim, H = hidden_dim;
  const int64_t offs[7] = {wq_off, wk_off, wv_off, wo_off, w1_off, w2_off, w3_off};
  const int64_t per[7] = {D * D, D * kvd, D * kvd, D * D, H * D, D * H, H * D};  // per-layer elements
  int64_t end = 0;
  for (int i = 0; i < 7; i++) {
    if (offs[i] < 0) return fail("negative weight offset");
    end = std::max(end, offs[i] + L * per[i]);
  }
  struct In { const void *p; int64_t off, size, stride, need; const char *name; };
  const In ins[] = {
      {token_emb, token_emb_off, token_emb_size, token_emb_stride, vocab_size * D, "token_emb"},
      {rms_att_w, rms_att_w_off, rms_att_w_size, rms_att_w_stride, L * D, "rms_att_w"},
      {rms_ffn_w, rms_ffn_w_off, rms_ffn_w_size, rms_ffn_w_stride, L * D, "rms_ffn_w"},
      {rms_final_w, rms_final_w_off, rms_final_w_size, rms_final_w_stride, D, "rms_final_w"},
      {wcls, wcls_off, wcls_size, wcls_stride, vocab_size * D, "wcls"},
      {qweights, qweights_off, qweights_size, qweights_stride, (end + 1) / 2, "qweights"},
      {scales, scales_off, scales_size, scales_stride, cdiv(end, group_size), "scales"},
      {zeros, zeros_off, zeros_size, zeros_stride, cdiv(end, group_size), "zeros"},
      {logits, logits_off, logits_size, logits_stride, vocab_size, "logits"},
      {key_cache, key_cache_off, key_cache_size, key_cache_stride, L * seq_len * kvd, "key_cache"},
      {value_cache, value_cache_off, value_cache_size, value_cache_stride, L * seq_len * kvd,
       "value_cache"}};
  for (const In &a : ins) {
    if (check_desc1(a.name, a.p, a.off, a.size, a.stride)) return nan;
    if (a.size < a.need) {
      set_error(SIMP_RT_EINVAL, "llama2_quant_forward: %s has %lld elements, needs %lld", a.name,
                (long long)a.size, (long long)a.need);
      return nan;
    }
  }
  const size_t esz[8] = {4, 4, 4, 4, 4, 1, 4, 4};
  const void *wp[8];
  for (int i = 0; i < 8; i++) wp[i] = (const char *)ins[i].p + esz[i] * (size_t)ins[i].off;
  std::vector<int64_t> key = {dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len,
                              group_size};
  for (int i = 0; i < 7; i++) key.push_back(offs[i]);
  for (int i = 0; i < 8; i++) key.push_back((int64_t)(uintptr_t)wp[i]);
  hipStream_t st = cur_stream();
  std::lock_guard<std::mutex> lk(g_fwd_mu);
  auto it = g_qfwd.find(key);
  if (it == g_qfwd.end()) {
    evict_lru(g_qfwd, kMaxEntries, quant_free);
    it = g_qfwd.emplace(key, QuantModel{}).first;
    QuantModel &nm = it->second;
    nm.dim = dim; nm.hid = hidden_dim; nm.L = L; nm.nh = n_heads; nm.nkv = n_kv_heads;
    nm.V = vocab_size; nm.seq = seq_len; nm.gs = group_size;
    for (int i = 0; i < 7; i++) nm.off[i] = offs[i];
    nm.kv_dim = (int)kvd;
    nm.hs = (int)hs;
    const void *d[8];
    bool ok = true;
    for (int i = 0; i < 8 && ok; i++)
      ok = nm.weights.bind(wp[i], esz[i] * (size_t)ins[i].need, &d[i], ins[i].name) == SIMP_RT_OK;
    if (ok) {
      nm.emb = (const float *)d[0]; nm.rms_att = (const float *)d[1]; nm.rms_ffn = (const float *)d[2];
      nm.rms_final = (const float *)d[3]; nm.wcls = (const float *)d[4];
      nm.qw = (const uint8_t *)d[5]; nm.scales = (const float *)d[6]; nm.zeros = (const float *)d[7];
      ok = quant_alloc(nm) == SIMP_RT_OK;
      nm.fused = quant_fusable(nm);
    }
    if (!ok) {
      quant_free(nm);
      g_qfwd.erase(it);
      return nan;
    }
  }
  QuantModel *m = &it->second;
  m->last_use = ++g_fwd_clock;
  const size_t pitch = 4 * (size_t)(seq_len * kvd), row = 4 * (size_t)kvd;
  const size_t at = (size_t)(pos * kvd);
  bool restart = false;
  if (m->kv.prepare(pos, key_cache + key_cache_off, value_cache + value_cache_off, m->kc, m->vc,
                    row, pitch, L, st, &restart) ||
      m->weights.verify(restart))
    return nan;
  if (quant_forward_device(*m, token, pos, st)) return nan;
  float *lg = logits + logits_off;
  float l0 = nan;
  if (m->io.copy_back(lg, m->logits, 4 * (size_t)vocab_size, (char *)(key_cache + key_cache_off + at),
                      (char *)(value_cache + value_cache_off + at), (const char *)(m->kc + at),
                      (const char *)(m->vc + at), row, pitch, L, st, &l0))
    return nan;
  m->kv.done(pos);
  return l0;
}

#undef SIMP_DESC_F32
#undef SIMP_DESC_I8

}  // extern "C"

extern "C" {

int32_t simp_rt_forward_cache_clear(void) {
  std::lock_guard<std::mutex> lk(g_fwd_mu);
  for (auto &kv : g_fwd) forward_entry_free(kv.second);
  g_fwd.clear();
  for (auto &kv : g_qfwd) {
    (void)hipDeviceSynchronize();
    quant_free(kv.second);
  }
  g_qfwd.clear();
  l32_cache_clear();
  return SIMP_RT_OK;
}

}  // extern "C"
