// w4.hip -- W4 (4-bit weight) GEMV / skinny GEMM, HBM-bound.
//
// Two packed formats, both "low nibble = even index, two weights per byte":
//   reference  (matmul_quant, MatMulQuantOpLowering, ConvertSimpToMemRef.cpp:3853-4013):
//              unsigned q in [0,15], w = q*scale + zero, groups are flat runs of
//              `gs` weights of the concatenated weight array starting at `offset`.
//              The reference reads scales at (i*cols)/gs + g, ignoring `offset`,
//              and always walks 8 tiles of 16 (gs must be 128); both are fixed
//              here: the group index is (offset + i*cols)/gs + g and any gs that
//              is a multiple of 32 works.
//   symmetric  (the int4 convention of ConvertSimpToMemRef.cpp:3016-3037): signed
//              q in [-8,7], one fp32 scale per group of `gs` along K, W[N,K] with
//              rows of K/2 bytes, scales[N,K/gs], x[M,K] -> out[M,N].
//
// Kernel shape: 16 lanes cooperate on one weight row, each lane taking 16-byte
// chunks (32 weights) of the row in turn, so a wave streams 4 rows x 256
// contiguous bytes per load.  Per chunk the 8 dwords are split into even/odd
// nibble bytes (and/shift) and converted with v_cvt_f32_ubyte{0..3}: 1.4 VALU
// ops per weight for decode, then one FMA per weight and row of x.  Signed
// nibbles are first flipped to q+8 (xor 0x88888888) and the -8*sum(x) term is
// folded in once per chunk from per-chunk sums of x computed in the block
// prologue (LDS), so no per-weight sign handling is needed.  Per-chunk partial
// dot products are scaled by the group's scale (and zero) and summed in fp32;
// the 16 lane partials are combined with a butterfly over the lane group.
#include <type_traits>

#include "rt_device.h"
#include "rt_internal.h"

namespace simp {
namespace {

// Calls f(std::integral_constant<int, I>()) for I = B .. E-1 (fully unrolled).
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>());
    static_for<B + 1, E>(f);
  }
}

constexpr int kRowsPerBlock = 16;  // 16 lanes per row, 256 threads
constexpr int kLanesPerRow = 16;

// Sum over the 16 lanes of a row group.
__device__ __forceinline__ float group16_sum(float v) {
  v += __shfl_xor(v, 8);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 1);
  return v;
}

// Per-chunk sums of x (xs[m*nchunk + c] = sum_{j<32} x[m, 32c + j]) into LDS.
template <int MT>
__device__ __forceinline__ void chunk_sums(const float *__restrict__ X, int64_t ldx, int M, int nchunk,
                                           float *xs) {
  for (int i = threadIdx.x; i < M * nchunk; i += blockDim.x) {
    const int m = i / nchunk, c = i - m * nchunk;
    const float4 *p = (const float4 *)(X + (int64_t)m * ldx + 32 * c);
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const float4 v = p[q];
      s += (v.x + v.y) + (v.z + v.w);
    }
    xs[i] = s;
  }
  lds_barrier();
}

// Symmetric signed W4, one scale per `gs` weights along K.  MT = max rows of x.
// Lane -> row mapping: a block owns RB weight rows; thread t takes row t % RB
// and the chunks c = g, g+G, g+2G, ... of it, g = t / RB, G = 256 / RB, so a
// wave's load covers RB rows x 64/RB consecutive chunks.  The RB lanes of a
// group need the same x chunk.  XL: x is staged once per block in LDS, each
// chunk's eight float4 slots rotated by the chunk index so the 64/RB chunks
// read by one instruction fall in distinct banks, and the per-chunk sums of x
// (the -8 offset of the flipped nibbles) are taken from LDS.  !XL (x too large
// for LDS): x is read from global memory as broadcasts and the chunk sums are
// split over the RB lanes sharing a chunk.  UB weight chunks are loaded before
// any is used.  The G partial sums of a row are reduced with shuffles inside a
// wave, then through LDS across the 4 waves.
template <int MT, int RB, int UB, bool XL>
__global__ void __launch_bounds__(256)
    w4s_gemv(const uint8_t *__restrict__ W, int64_t ldw, const float *__restrict__ S, int64_t lds,
             const float *__restrict__ X, int64_t ldx, float *__restrict__ O, int64_t ldo, int M,
             int N, int K, int gs) {
  constexpr int G = 256 / RB, XPER = 32 / RB;
  static_assert(32 % RB == 0 && RB <= 32, "RB");
  __shared__ float red[4][MT][RB];
  extern __shared__ float smem[];  // XL: xl[M][K] then xs[M][K/32]
  const int nchunk = K >> 5;
  float *xl = smem, *xs = smem + (XL ? M * K : 0);
  const int r = threadIdx.x % RB, g = threadIdx.x / RB;
  const int n = min(blockIdx.x * RB + r, N - 1);  // clamped: rows past N compute, never store
  const uint8_t *wrow = W + (int64_t)n * ldw;
  const float *srow = S + (int64_t)n * lds;
  const int cpg = gs >> 5, cps = cpg_log2(cpg);
  uint4 w[UB];
  float sc[UB];
  auto load_batch = [&](int c0) {
#pragma unroll
    for (int u = 0; u < UB; u++) {
      const int c = min(c0 + u * G, nchunk - 1);
      w[u] = *(const uint4 *)(wrow + 16 * c);
      sc[u] = srow[chunk_group(c, cpg, cps)];
    }
  };
  // the first weight batch is requested before x is staged; the staging
  // barriers are LDS-only, so these loads stay in flight through them
  load_batch(g);
  if constexpr (XL) {
    for (int i = threadIdx.x; i < M * (K >> 2); i += 256) {
      const int m = i / (K >> 2), f = i - m * (K >> 2);
      const int c = f >> 3, q = f & 7;
      *(float4 *)(xl + m * K + 32 * c + 4 * ((q + c) & 7)) =
          *(const float4 *)(X + (int64_t)m * ldx + 4 * f);
    }
    lds_barrier();
    for (int i = threadIdx.x; i < M * nchunk; i += 256) {
      const int m = i / nchunk, c = i - m * nchunk;
      float t = 0.f;
#pragma unroll
      for (int q = 0; q < 8; q++) {
        const float4 v = *(const float4 *)(xl + m * K + 32 * c + 4 * q);
        t += (v.x + v.y) + (v.z + v.w);
      }
      xs[i] = t;
    }
    lds_barrier();
  }
  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; m++) acc[m] = 0.f;
  for (int c0 = g; c0 < nchunk; c0 += G * UB) {
    if (c0 != g) load_batch(c0);
#pragma unroll
    for (int u = 0; u < UB; u++) {
      const int c = c0 + u * G;
      if (c < nchunk) {  // uniform across the RB lanes of the group
        uint4 wv = w[u];
        wv.x ^= 0x88888888u; wv.y ^= 0x88888888u; wv.z ^= 0x88888888u; wv.w ^= 0x88888888u;
        float uu[32];
        unpack32(wv, uu);
#pragma unroll
        for (int m = 0; m < MT; m++) {
          if (m < M) {
            float p = 0.f;
#pragma unroll
            for (int q = 0; q < 8; q++) {
              const float4 v = XL ? *(const float4 *)(xl + m * K + 32 * c + 4 * ((q + c) & 7))
                                  : *(const float4 *)(X + (int64_t)m * ldx + 32 * c + 4 * q);
              p = fmaf(uu[4 * q + 0], v.x, p);
              p = fmaf(uu[4 * q + 1], v.y, p);
              p = fmaf(uu[4 * q + 2], v.z, p);
              p = fmaf(uu[4 * q + 3], v.w, p);
            }
            float xsum;
            if constexpr (XL) {
              xsum = xs[m * nchunk + c];
            } else {
              const float *xc = X + (int64_t)m * ldx + 32 * c;
              xsum = 0.f;
#pragma unroll
              for (int e = 0; e < XPER; e++) xsum += xc[r * XPER + e];
#pragma unroll
              for (int d = 1; d < RB; d <<= 1) xsum += __shfl_xor(xsum, d);
            }
            acc[m] = fmaf(sc[u], fmaf(-8.f, xsum, p), acc[m]);  // sum (u-8) x
          }
        }
      }
    }
  }
  // reduce the 64/RB groups of this wave, then the 4 waves
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int m = 0; m < MT; m++) {
    float v = acc[m];
#pragma unroll
    for (int d = RB; d < 64; d <<= 1) v += __shfl_xor(v, d);
    if ((threadIdx.x & 63) < RB) red[wave][m][r] = v;
  }
  __syncthreads();
  if (threadIdx.x < RB && blockIdx.x * RB + (int)threadIdx.x < N) {
#pragma unroll
    for (int m = 0; m < MT; m++)
      if (m < M)
        O[(int64_t)m * ldo + blockIdx.x * RB + r] = (red[0][m][r] + red[1][m][r]) + (red[2][m][r] + red[3][m][r]);
  }
}

// Symmetric W4 with one x vector (the decode shape).  Same lane -> row mapping
// as w4s_gemv (RB = 8 rows per block, chunk groups g = t / 8, chunks g + 32u),
// but no block-wide barrier before the compute: a block barrier makes every
// wave wait for all of its outstanding weight loads (the fence drains vmcnt),
// which serialises the unpack/FMA work behind the last byte of the transfer.
// Instead each wave stages into its own LDS region just the x chunks its lanes
// use, with the x loads issued before the weight loads (loads retire in issue
// order), and each chunk's work then waits only for that chunk's bytes.
// Requires 32 * UB >= K / 32.
template <int UB>
__global__ void __launch_bounds__(256)
    w4s_gemv1(const uint8_t *__restrict__ W, int64_t ldw, const float *__restrict__ S, int64_t lds,
              const float *__restrict__ X, float *__restrict__ O, int N, int K, int gs) {
  constexpr int RB = 8, G = 256 / RB, GW = 64 / RB;  // chunk groups per block / per wave
  constexpr int CW = GW * UB;                         // x chunks staged per wave
  constexpr int XPL = CW * 8 / 64;                    // x float4 per lane
  __shared__ float red[4][RB];
  __shared__ __align__(16) float xw[4][CW][32];
  __shared__ float xsw[4][CW];
  const int nchunk = K >> 5, cpg = gs >> 5, cps = cpg_log2(cpg);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = threadIdx.x % RB, g = threadIdx.x / RB, gl = lane / RB;
  const int n = min((int)blockIdx.x * RB + r, N - 1);  // clamped: rows past N never stored
  const uint8_t *wrow = W + (int64_t)n * ldw;
  const float *srow = S + (int64_t)n * lds;
  // x of the wave's chunks: local j = u*GW + gl' holds chunk wave*GW + gl' + G*u
  float4 xv[XPL];
#pragma unroll
  for (int i = 0; i < XPL; i++) {
    const int f = lane + 64 * i, j = f >> 3, q = f & 7;
    const int c = min(wave * GW + j % GW + G * (j / GW), nchunk - 1);
    xv[i] = *(const float4 *)(X + 32 * c + 4 * q);
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
  // stage x (float4 slots of chunk j rotated by j: the GW chunks one read touches
  // fall in distinct banks) and the per-chunk sums of x
#pragma unroll
  for (int i = 0; i < XPL; i++) {
    const int f = lane + 64 * i, j = f >> 3, q = f & 7;
    *(float4 *)(&xw[wave][j][4 * ((q + j) & 7)]) = xv[i];
    float t = (xv[i].x + xv[i].y) + (xv[i].z + xv[i].w);
    t += __shfl_xor(t, 1);
    t += __shfl_xor(t, 2);
    t += __shfl_xor(t, 4);
    if (q == 0) xsw[wave][j] = t;
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
  if (threadIdx.x < RB && (int)blockIdx.x * RB + (int)threadIdx.x < N)
    O[blockIdx.x * RB + r] = (red[0][r] + red[1][r]) + (red[2][r] + red[3][r]);
}

// Symmetric W4, group size 32, 2 <= M <= 16 x vectors, on fp32 MFMA
// (v_mfma_f32_16x16x4_f32): C[m][n] = sum_g s[n][g] * sum_{k in g} x[m][k] q[n][k].
//   * Block = 4 waves, one tile of 16 weight rows each (64 rows), and one part
//     of at most kW4mMaxG groups of K (gridDim.y parts).  With more than one
//     part each block writes its partial tile to P[part][M][N] and
//     w4s_sum_parts adds the parts in order.
//   * Every load of the block is issued up front: x of the part (staged in LDS
//     as [k/4][m] float4, so a read of 16 rows x 16 B per lane group covers 256
//     contiguous bytes), then each lane's weight chunks (lane (n = l%16, kq =
//     l/16) takes groups 4s + kq of row n) and their scales.  Loads retire in
//     issue order, so step s computes as soon as its own chunks are in.
//   * Per step of 4 groups the wave moves its 16 rows x 64 B of chunks through
//     a small LDS tile (row n's chunk kq in slot kq ^ (n/4), so the dword reads
//     of one group hit 64 banks): lane (n, kq) then holds dword kq of every
//     group, i.e. k = 8 kq + j of MFMA j, matching x[m][32g + 8kq + j].
//   * Per group: eight MFMAs of K = 4 accumulate D = x q (exact nibble values,
//     fp32 x and accumulation), then acc += s * D.
constexpr int kW4mRows = 64;  // weight rows per block
constexpr int kW4mMaxG = 12;  // K groups per block part at most (x of a part: 24 KB of LDS)

// MS = steps of 4 groups per part (4 MS >= the part's groups); every step
// runs, groups past the part multiply zero x.  Straight-line steps keep each
// step's chunks in registers (two blocks per CU by LDS: up to 256 VGPRs).
template <int MS>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
    w4s_mfma(const uint8_t *__restrict__ W, int64_t ldw, const float *__restrict__ S, int64_t lds,
             const float *__restrict__ X, int64_t ldx, float *__restrict__ O, int64_t ldo,
             float *__restrict__ P, int M, int N, int K) {
  typedef float v4f __attribute__((ext_vector_type(4)));
  constexpr int XPT = MS * 4 * 8 * 16 / 256;  // x float4 per thread
  __shared__ __align__(16) float4 xl[MS * 4 * 8][16];  // [k/4 within the part][m]
  __shared__ __align__(16) uint32_t wt[4][2][16 * 16];   // [wave][buf][row*16 + slot*4 + dword]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 15, kq = lane >> 4;
  const int ng = K >> 5;
  const int part = blockIdx.y, nparts = gridDim.y;
  const int g0 = part * ng / nparts, g1 = (part + 1) * ng / nparts;  // g1 - g0 <= 4 MS
  const int nk4 = 8 * (g1 - g0);                                     // float4 of x per row
  const int n = min((int)blockIdx.x * kW4mRows + 16 * wave + ln, N - 1);  // rows past N: never stored
  // 1. x of the part: thread t -> (m = t % 16, k/4 = t / 16 + 16 i); rows m >= M stay zero
  const int xm = tid & 15, xc = tid >> 4;
  const float *xrow = X + (int64_t)min(xm, M - 1) * ldx + 32 * g0;
  float4 xv[XPT];
#pragma unroll
  for (int i = 0; i < XPT; i++) {
    const int c = xc + 16 * i;
    xv[i] = (xm < M && c < nk4) ? *(const float4 *)(xrow + 4 * c) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  // 2. this lane's weight chunks and scales (clamped; groups past g1 are not used)
  const uint8_t *wrow = W + (int64_t)n * ldw;
  const float *srow = S + (int64_t)n * lds;
  // (named registers, not arrays: an array here is moved to LDS by the
  // compiler's alloca promotion, which serializes the loads)
  static_assert(MS <= 6, "at most six steps per part");
  uint4 wv0, wv1, wv2, wv3, wv4, wv5;
  float sv0, sv1, sv2, sv3, sv4, sv5;
  auto wv = [&](auto ST) -> uint4 & {
    constexpr int i = decltype(ST)::value;
    if constexpr (i == 0) return wv0; else if constexpr (i == 1) return wv1;
    else if constexpr (i == 2) return wv2; else if constexpr (i == 3) return wv3;
    else if constexpr (i == 4) return wv4; else return wv5;
  };
  auto sv = [&](auto ST) -> float & {
    constexpr int i = decltype(ST)::value;
    if constexpr (i == 0) return sv0; else if constexpr (i == 1) return sv1;
    else if constexpr (i == 2) return sv2; else if constexpr (i == 3) return sv3;
    else if constexpr (i == 4) return sv4; else return sv5;
  };
  static_for<0, MS>([&](auto ST) {
    const int g = min(g0 + 4 * decltype(ST)::value + kq, ng - 1);
    wv(ST) = *(const uint4 *)(wrow + 16 * g);
    sv(ST) = srow[g];
  });
  __builtin_amdgcn_sched_barrier(0);  // all loads issued before the staging below waits
#pragma unroll
  for (int i = 0; i < XPT; i++) xl[xc + 16 * i][xm] = xv[i];  // zero past the part
  lds_barrier();
  v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
  const int swz = ln >> 2;
  static_for<0, MS>([&](auto ST) {  // unrolled: each step's chunk stays in its register
    constexpr int st = decltype(ST)::value;
    *(uint4 *)&wt[wave][st & 1][ln * 16 + ((kq ^ swz) << 2)] = wv(ST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave's tile is written
    __builtin_amdgcn_wave_barrier();
    // the step's four groups as four independent MFMA chains (a dependent
    // 16x16x4 f32 MFMA waits ~40 cycles for its predecessor; four chains keep
    // the pipe busy)
    float xs[4][8];
    uint32_t d[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int gl = 4 * st + j;  // group within the part
      const float4 xa = xl[8 * gl + 2 * kq][ln], xb = xl[8 * gl + 2 * kq + 1][ln];
      xs[j][0] = xa.x; xs[j][1] = xa.y; xs[j][2] = xa.z; xs[j][3] = xa.w;
      xs[j][4] = xb.x; xs[j][5] = xb.y; xs[j][6] = xb.z; xs[j][7] = xb.w;
      d[j] = wt[wave][st & 1][ln * 16 + ((j ^ swz) << 2) + kq];
    }
    v4f D[4];
#pragma unroll
    for (int j = 0; j < 4; j++) D[j] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 8; e++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float q = (float)(((int)(d[j] << (28 - 4 * e))) >> 28);  // signed nibble e
        D[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(xs[j][e], q, D[j], 0, 0, 0);
      }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float sc = __shfl(sv(ST), ln + 16 * j);  // scale of (row ln, group g0 + 4 st + j)
      acc = acc + sc * D[j];
    }
  });
  // acc[r] = C[m = 4 kq + r][this wave's row ln] over this block's part of K
  const int nn = (int)blockIdx.x * kW4mRows + 16 * wave + ln;
  if (nn < N) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int m = 4 * kq + r;
      if (m < M) {
        if (nparts == 1) O[(int64_t)m * ldo + nn] = acc[r];
        else P[((int64_t)part * M + m) * N + nn] = acc[r];
      }
    }
  }
}

// out[m][n] = sum over parts p (in order) of P[p][m][n].
__global__ void __launch_bounds__(256)
    w4s_sum_parts(const float *__restrict__ P, int nparts, float *__restrict__ O, int64_t ldo, int M,
                  int N) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)M * N) return;
  float t = 0.f;
  for (int p = 0; p < nparts; p++) t += P[(int64_t)p * M * N + i];
  const int m = (int)(i / N), n = (int)(i - (int64_t)m * N);
  O[(int64_t)m * ldo + n] = t;
}

// Reference W4 (unsigned + zero, flat groups), one x vector.  Row i's nibbles
// start at element offset off + i*cols (a multiple of 32 here).
__global__ void __launch_bounds__(256)
    w4u_gemv(const uint8_t *__restrict__ Q, const float *__restrict__ S, const float *__restrict__ Z,
             const float *__restrict__ X, float *__restrict__ O, int rows, int cols, int gs,
             int64_t off) {
  extern __shared__ float xs[];
  const int nchunk = cols >> 5;
  chunk_sums<1>(X, 0, 1, nchunk, xs);
  const int seg = threadIdx.x & (kLanesPerRow - 1);
  const int i = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 4);
  if (i >= rows) return;
  const int64_t base = off + (int64_t)i * cols;  // element index of the row start
  const uint8_t *qrow = Q + (base >> 1);
  const int64_t g0 = base / gs;
  const int cpg = gs >> 5, cps = cpg_log2(cpg);
  float acc = 0.f;
  for (int c = seg; c < nchunk; c += kLanesPerRow) {
    const uint4 w = *(const uint4 *)(qrow + 16 * c);
    const int64_t g = g0 + chunk_group(c, cpg, cps);
    const float s = S[g], z = Z[g];
    float u[32];
    unpack32(w, u);
    const float4 *xp = (const float4 *)(X + 32 * c);
    float p = 0.f;
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const float4 v = xp[q];
      p = fmaf(u[4 * q + 0], v.x, p);
      p = fmaf(u[4 * q + 1], v.y, p);
      p = fmaf(u[4 * q + 2], v.z, p);
      p = fmaf(u[4 * q + 3], v.w, p);
    }
    acc = fmaf(s, p, fmaf(z, xs[c], acc));  // sum (u*s + z) x
  }
  const float v = group16_sum(acc);
  if (seg == 0) O[i] = v;
}

// Any-shape fallbacks (one thread per output; correctness path).
__global__ void __launch_bounds__(256)
    w4s_generic(const uint8_t *__restrict__ W, int64_t ldw, const float *__restrict__ S, int64_t lds,
                const float *__restrict__ X, int64_t ldx, float *__restrict__ O, int64_t ldo, int M,
                int N, int K, int gs) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)M * N) return;
  const int m = (int)(idx / N), n = (int)(idx - (int64_t)m * N);
  float acc = 0.f;
  for (int k = 0; k < K; k++) {
    const uint8_t b = W[(int64_t)n * ldw + (k >> 1)];
    int q = (k & 1) ? (b >> 4) : (b & 15);
    q = q >= 8 ? q - 16 : q;
    acc = fmaf((float)q * S[(int64_t)n * lds + k / gs], X[(int64_t)m * ldx + k], acc);
  }
  O[(int64_t)m * ldo + n] = acc;
}

__global__ void __launch_bounds__(256)
    w4u_generic(const uint8_t *__restrict__ Q, const float *__restrict__ S, const float *__restrict__ Z,
                const float *__restrict__ X, float *__restrict__ O, int rows, int cols, int gs,
                int64_t off) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= rows) return;
  float acc = 0.f;
  const int64_t base = off + (int64_t)i * cols;
  for (int k = 0; k < cols; k++) {
    const int64_t e = base + k;
    const uint8_t b = Q[e >> 1];
    const int q = (e & 1) ? (b >> 4) : (b & 15);
    const int64_t g = e / gs;
    acc = fmaf((float)q * S[g] + Z[g], X[k], acc);
  }
  O[i] = acc;
}

}  // namespace

// Launches the symmetric W4 GEMV on device pointers (shared with the decode step).
int launch_w4s(const uint8_t *W, int64_t ldw, const float *S, int64_t lds, const float *X,
               int64_t ldx, float *O, int64_t ldo, int M, int N, int K, int gs, hipStream_t st) {
  if (M == 0 || N == 0) return SIMP_RT_OK;
  const bool fast = K % 32 == 0 && gs % 32 == 0 && K % gs == 0 && ldw % 16 == 0 &&
                    ((uintptr_t)W & 15) == 0 && ldx % 4 == 0 && ((uintptr_t)X & 15) == 0 &&
                    M <= 16;
  if (!fast) {
    const int64_t tot = (int64_t)M * N;
    hipLaunchKernelGGL(w4s_generic, dim3((unsigned)cdiv(tot, 256)), dim3(256), 0, st, W, ldw, S,
                       lds, X, ldx, O, ldo, M, N, K, gs);
  } else if (M >= 2 && gs == 32) {
    // several x vectors, groups of 32: fp32 MFMA.  The K parts make about two
    // blocks per CU; with more than one part the partial tiles go through a
    // workspace and a second, ordered sum.
    const int nb = (int)cdiv(N, kW4mRows), ng = K / 32;
    const int occ = nb >= num_cus() ? 1 : (int)cdiv(2 * num_cus(), nb);
    const int parts = (int)std::min<int64_t>(ng, std::max<int64_t>(cdiv(ng, kW4mMaxG), occ));
    float *P = nullptr;
    if (parts > 1) {
      int rc = workspace(st, sizeof(float) * (size_t)parts * M * N, (void **)&P, 2);
      if (rc) return rc;
    }
    const int ms = (int)cdiv(cdiv(ng, parts), 4);  // steps for the largest part
    KernelTimer kt(st, "w4s_mfma");
#define W4M(MSV) hipLaunchKernelGGL((w4s_mfma<MSV>), dim3((unsigned)nb, (unsigned)parts), dim3(256), 0, st, \
                                    W, ldw, S, lds, X, ldx, O, ldo, P, M, N, K)
    if (ms <= 2) W4M(2);
    else W4M(3);
#undef W4M
    if (parts > 1)
      hipLaunchKernelGGL(w4s_sum_parts, dim3((unsigned)cdiv((int64_t)M * N, 256)), dim3(256), 0, st, P,
                         parts, O, ldo, M, N);
  } else if (M == 1 && K / 32 <= 32 * 16) {
    // one x vector: the barrier-free kernel, UB chunks per lane with 32*UB >= K/32
    const int nchunk = K / 32;
    const dim3 grid((unsigned)cdiv(N, 8));
    KernelTimer kt(st, "w4s_gemv");
#define W4S1(U) hipLaunchKernelGGL((w4s_gemv1<U>), grid, dim3(256), 0, st, W, ldw, S, lds, X, O, N, K, gs)
    if (nchunk <= 64) W4S1(2);
    else if (nchunk <= 128) W4S1(4);
    else if (nchunk <= 256) W4S1(8);
    else if (nchunk <= 384) W4S1(12);
    else W4S1(16);
#undef W4S1
  } else {
    // 8 rows per block keeps >= 400 blocks at N = 3200; x in LDS when it fits.
    constexpr int RB = 8;
    const dim3 grid((unsigned)cdiv(N, RB));
    const size_t xl_bytes = sizeof(float) * ((size_t)M * K + (size_t)M * (K / 32));
    const bool xl = xl_bytes <= 64 * 1024;
    const bool ub4 = K / 32 <= 4 * (256 / RB);
    const size_t shm = xl ? xl_bytes : 0;
    KernelTimer kt(st, "w4s_gemv");
#define W4S_LAUNCH(MTV)                                                                         \
  do {                                                                                          \
    if (xl && ub4)                                                                              \
      hipLaunchKernelGGL((w4s_gemv<MTV, RB, 4, true>), grid, dim3(256), shm, st, W, ldw, S, lds, X, \
                         ldx, O, ldo, M, N, K, gs);                                             \
    else if (xl)                                                                                \
      hipLaunchKernelGGL((w4s_gemv<MTV, RB, 8, true>), grid, dim3(256), shm, st, W, ldw, S, lds, X, \
                         ldx, O, ldo, M, N, K, gs);                                             \
    else                                                                                        \
      hipLaunchKernelGGL((w4s_gemv<MTV, RB, 8, false>), grid, dim3(256), 0, st, W, ldw, S, lds, X, \
                         ldx, O, ldo, M, N, K, gs);                                             \
  } while (0)
    if (M == 1) W4S_LAUNCH(1);
    else if (M <= 4) W4S_LAUNCH(4);
    else if (M <= 8) W4S_LAUNCH(8);
    else W4S_LAUNCH(16);
#undef W4S_LAUNCH
  }
  SIMP_HIP(hipGetLastError());
  return SIMP_RT_OK;
}

int launch_w4u(const uint8_t *Q, const float *S, const float *Z, const float *X, float *O, int rows,
               int cols, int gs, int64_t off, hipStream_t st) {
  if (rows == 0) return SIMP_RT_OK;
  const bool fast = cols % 32 == 0 && gs % 32 == 0 && off % 32 == 0 && off % gs == 0 &&
                    cols % gs == 0 &&
                    ((uintptr_t)Q & 15) == 0 && ((uintptr_t)X & 15) == 0;
  if (!fast) {
    hipLaunchKernelGGL(w4u_generic, dim3((unsigned)cdiv(rows, 256)), dim3(256), 0, st, Q, S, Z, X, O,
                       rows, cols, gs, off);
  } else {
    KernelTimer kt(st, "w4u_gemv");
    hipLaunchKernelGGL(w4u_gemv, dim3((unsigned)cdiv(rows, kRowsPerBlock)), dim3(256),
                       sizeof(float) * (size_t)(cols / 32), st, Q, S, Z, X, O, rows, cols, gs, off);
  }
  SIMP_HIP(hipGetLastError());
  return SIMP_RT_OK;
}

}  // namespace simp

using namespace simp;

extern "C" {

int32_t simp_rt_matmul_quant(
    const int8_t *qw_alloc, const int8_t *qw, int64_t qw_off, int64_t qw_size, int64_t qw_stride,
    const float *s_alloc, const float *s, int64_t s_off, int64_t s_size, int64_t s_stride,
    const float *z_alloc, const float *z, int64_t z_off, int64_t z_size, int64_t z_stride,
    const float *in_alloc, const float *in, int64_t in_off, int64_t in_size, int64_t in_stride,
    float *out_alloc, float *out, int64_t out_off, int64_t out_size, int64_t out_stride,
    int64_t rows, int64_t cols, int64_t group_size, int64_t offset) {
  (void)qw_alloc; (void)s_alloc; (void)z_alloc; (void)in_alloc; (void)out_alloc;
  int rc;
  if ((rc = check_desc1("qweights", qw, qw_off, qw_size, qw_stride))) return rc;
  if ((rc = check_desc1("scales", s, s_off, s_size, s_stride))) return rc;
  if ((rc = check_desc1("zeros", z, z_off, z_size, z_stride))) return rc;
  if ((rc = check_desc1("input", in, in_off, in_size, in_stride))) return rc;
  if ((rc = check_desc1("output", out, out_off, out_size, out_stride))) return rc;
  if (rows < 0 || cols < 0 || offset < 0 || group_size <= 0)
    return set_error(SIMP_RT_EINVAL, "matmul_quant: bad rows/cols/group_size/offset");
  if (rows == 0) return SIMP_RT_OK;
  const int64_t last = offset + rows * cols;  // one past the last weight
  const int64_t ngroups = (last + group_size - 1) / group_size;
  if ((last + 1) / 2 > qw_size || ngroups > s_size || ngroups > z_size || cols > in_size ||
      rows > out_size)
    return set_error(SIMP_RT_EINVAL,
                     "matmul_quant: arrays too small for rows=%lld cols=%lld gs=%lld offset=%lld",
                     (long long)rows, (long long)cols, (long long)group_size, (long long)offset);
  if (rows > INT32_MAX || cols > INT32_MAX)
    return set_error(SIMP_RT_EUNSUPPORTED, "matmul_quant: dimension above 2^31-1");
  Operand oq, os, oz, oi, oo;
  if ((rc = oq.bind(qw + qw_off, (size_t)qw_size, Operand::kIn, "qweights"))) return rc;
  if ((rc = os.bind(s + s_off, sizeof(float) * (size_t)s_size, Operand::kIn, "scales"))) return rc;
  if ((rc = oz.bind(z + z_off, sizeof(float) * (size_t)z_size, Operand::kIn, "zeros"))) return rc;
  if ((rc = oi.bind(in + in_off, sizeof(float) * (size_t)cols, Operand::kIn, "input"))) return rc;
  if ((rc = oo.bind(out + out_off, sizeof(float) * (size_t)rows, Operand::kOut, "output"))) return rc;
  if ((rc = launch_w4u((const uint8_t *)oq.dev(), (const float *)os.dev(), (const float *)oz.dev(),
                       (const float *)oi.dev(), (float *)oo.dev(), (int)rows, (int)cols,
                       (int)group_size, offset, cur_stream())))
    return rc;
  Operand *ops[] = {&oq, &os, &oz, &oi, &oo};
  return finish(ops, 5);
}

int32_t simp_rt_matmul_w4s(
    const uint8_t *w_alloc, const uint8_t *w, int64_t w_off, int64_t w_s0, int64_t w_s1, int64_t w_st0, int64_t w_st1,
    const float *s_alloc, const float *s, int64_t s_off, int64_t s_s0, int64_t s_s1, int64_t s_st0, int64_t s_st1,
    const float *x_alloc, const float *x, int64_t x_off, int64_t x_s0, int64_t x_s1, int64_t x_st0, int64_t x_st1,
    float *o_alloc, float *o, int64_t o_off, int64_t o_s0, int64_t o_s1, int64_t o_st0, int64_t o_st1,
    int64_t group_size) {
  (void)w_alloc; (void)s_alloc; (void)x_alloc; (void)o_alloc;
  int rc;
  if ((rc = check_desc2("W", w, w_off, w_s0, w_s1, w_st0, w_st1))) return rc;
  if ((rc = check_desc2("scales", s, s_off, s_s0, s_s1, s_st0, s_st1))) return rc;
  if ((rc = check_desc2("x", x, x_off, x_s0, x_s1, x_st0, x_st1))) return rc;
  if ((rc = check_desc2("out", o, o_off, o_s0, o_s1, o_st0, o_st1))) return rc;
  const int64_t N = w_s0, M = x_s0, K = x_s1;
  if (group_size <= 0 || K % 2 != 0 || K % group_size != 0)
    return set_error(SIMP_RT_EINVAL, "matmul_w4s: K=%lld must be even and a multiple of gs=%lld",
                     (long long)K, (long long)group_size);
  if (w_s1 != K / 2 || s_s0 != N || s_s1 != K / group_size || o_s0 != M || o_s1 != N)
    return set_error(SIMP_RT_EINVAL,
                     "matmul_w4s: shape mismatch W[%lld,%lld] scales[%lld,%lld] x[%lld,%lld] "
                     "out[%lld,%lld] gs=%lld",
                     (long long)w_s0, (long long)w_s1, (long long)s_s0, (long long)s_s1,
                     (long long)x_s0, (long long)x_s1, (long long)o_s0, (long long)o_s1,
                     (long long)group_size);
  if (N > INT32_MAX || K > INT32_MAX || M > INT32_MAX)
    return set_error(SIMP_RT_EUNSUPPORTED, "matmul_w4s: dimension above 2^31-1");
  Operand ow, os, ox, oo;
  const size_t wb = (N && K) ? (size_t)((N - 1) * w_st0 + K / 2) : 0;
  const size_t sb = (N && K) ? sizeof(float) * (size_t)((N - 1) * s_st0 + K / group_size) : 0;
  const size_t xb = (M && K) ? sizeof(float) * (size_t)((M - 1) * x_st0 + K) : 0;
  const size_t ob = (M && N) ? sizeof(float) * (size_t)((M - 1) * o_st0 + N) : 0;
  if ((rc = ow.bind(w + w_off, wb, Operand::kIn, "W"))) return rc;
  if ((rc = os.bind(s + s_off, sb, Operand::kIn, "scales"))) return rc;
  if ((rc = ox.bind(x + x_off, xb, Operand::kIn, "x"))) return rc;
  if ((rc = oo.bind(o + o_off, ob, Operand::kOut, "out"))) return rc;
  if ((rc = launch_w4s((const uint8_t *)ow.dev(), w_st0, (const float *)os.dev(), s_st0,
                       (const float *)ox.dev(), x_st0, (float *)oo.dev(), o_st0, (int)M, (int)N,
                       (int)K, (int)group_size, cur_stream())))
    return rc;
  Operand *ops[] = {&ow, &os, &ox, &oo};
  return finish(ops, 4);
}

}  // extern "C"
