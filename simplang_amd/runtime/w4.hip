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
// Several x vectors (2 <= M <= 16, groups of 32) run on f16 MFMA instead
// (w4s_h16): nibbles as exact f16 subnormals, x split exactly into f16 hi+lo.
#include "rt_device.h"
#include "rt_internal.h"

namespace simp {
namespace {

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
// as w4s_gemv (RB = 8 rows per block, chunk groups g = t / 8, chunks g + Gu),
// but no block-wide barrier before the compute: a block barrier makes every
// wave wait for all of its outstanding weight loads (the fence drains vmcnt),
// which serialises the unpack/FMA work behind the last byte of the transfer.
// Instead each wave stages into its own LDS region just the x chunks its lanes
// use, with the x loads issued before the weight loads (loads retire in issue
// order), and each chunk's work then waits only for that chunk's bytes.
// NWV waves per block (G = 8 NWV chunk groups): 8 for long rows over few
// blocks, which halves each wave's serial unpack/FMA work.
// Requires G * UB >= K / 32.
template <int UB, int NWV>
__global__ void __launch_bounds__(64 * NWV)
    w4s_gemv1(const uint8_t *__restrict__ W, int64_t ldw, const float *__restrict__ S, int64_t lds,
              const float *__restrict__ X, float *__restrict__ O, int N, int K, int gs) {
  constexpr int RB = 8, G = 64 * NWV / RB, GW = 64 / RB;  // chunk groups per block / per wave
  constexpr int CW = GW * UB;                              // x chunks staged per wave
  constexpr int XPL = CW * 8 / 64;                         // x float4 per lane
  __shared__ float red[NWV][RB];
  __shared__ __align__(16) float xw[NWV][CW][32];
  __shared__ float xsw[NWV][CW];
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
  if (threadIdx.x < RB && (int)blockIdx.x * RB + (int)threadIdx.x < N) {
    // the waves' partial sums in pairs, then the pairs in order
    float t = 0.f;
#pragma unroll
    for (int v = 0; v < NWV; v += 4)
      t += (red[v][r] + red[v + 1][r]) + (red[v + 2][r] + red[v + 3][r]);
    O[blockIdx.x * RB + r] = t;
  }
}

// ------------------------------------------- 2 <= M <= 16: f16 MFMA path
// Symmetric W4, groups of 32, on v_mfma_f32_16x16x32_f16 (D[16 x 16] +=
// A[16 x 32] B[32 x 16]): B = 16 weight rows x one group, A = x rows.
//   * Exact operands.  A nibble u = q + 8 enters as the f16 subnormal with bit
//     pattern u (value u * 2^-24, exact; the MFMA keeps f16 subnormals), built
//     by byte permutes of the nibble halves with zero high bytes.  x row m
//     enters as two A rows, hi = f16(x * 2^-e_m) and lo = f16(x * 2^-e_m - hi),
//     22 significant bits; e_m keeps the wave's largest |x| of row m below
//     2^14, so f16 cannot overflow.  Products are exact in fp32, so the result
//     differs from the fp32 VALU path only by accumulation order and the
//     22-bit x.  Per group: acc += s * (2^(24 + e_m) * (D_hi + D_lo) - 8 * sum x).
//   * Layout.  Lane (n = l%16, q = l/16) loads the 16 bytes of group g0 + q of
//     weight row n (four lanes read 64 contiguous bytes of each of 16 rows);
//     a 4 x 4 dword transpose across the lane groups (v_permlane32_swap then
//     v_permlane16_swap) gives lane (n, q) dword q of each of the four groups,
//     i.e. k = 8q..8q+7 of MFMA j, as the B layout wants.
//   * Block = 4 waves on the same 16 rows, each a slice of GQ groups of K; x
//     of the slice is staged per wave in LDS as f16 hi/lo (no block barrier
//     before the MFMAs), the four slices are added through LDS at the end.
//     Blocks of one row tile cover K in gridDim.y parts; with more than one
//     part the partial tiles go through P[part][M][N] and w4s_sum_parts.
//   * MT = 8-row tiles of x (1: M <= 8, 2: M <= 16), MS = steps of 4 groups
//     per wave (GQ = 4 MS).
typedef _Float16 w4h8 __attribute__((ext_vector_type(8)));
typedef float w4f4 __attribute__((ext_vector_type(4)));

// Eight nibbles (element order, low nibble = even element) as eight f16
// subnormals with the nibble as bit pattern.
__device__ __forceinline__ w4h8 nib8_f16(uint32_t t) {
  const uint32_t lo = t & 0x0F0F0F0Fu, hi = (t >> 4) & 0x0F0F0F0Fu;
  uint32_t d[4];
  d[0] = __builtin_amdgcn_perm(hi, lo, 0x0C040C00u);
  d[1] = __builtin_amdgcn_perm(hi, lo, 0x0C050C01u);
  d[2] = __builtin_amdgcn_perm(hi, lo, 0x0C060C02u);
  d[3] = __builtin_amdgcn_perm(hi, lo, 0x0C070C03u);
  w4h8 r;
  __builtin_memcpy(&r, d, 16);
  return r;
}

// Lane (n, q) holds w[0..3] = dwords of group q; afterwards w[j] = dword q of
// group j (4 x 4 transpose across the lane groups q = lane / 16).
__device__ __forceinline__ void xpose4x4(uint32_t (&w)[4]) {
  const auto a = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
  w[0] = a[0];
  w[2] = a[1];
  w[1] = b[0];
  w[3] = b[1];
  const auto c = __builtin_amdgcn_permlane16_swap(w[0], w[1], false, false);
  const auto e = __builtin_amdgcn_permlane16_swap(w[2], w[3], false, false);
  w[0] = c[0];
  w[1] = c[1];
  w[2] = e[0];
  w[3] = e[1];
}

template <int MT, int RT>
__global__ void __launch_bounds__(256)
    w4s_h16(const uint8_t *__restrict__ W, int64_t ldw, const float *__restrict__ S, int64_t lds,
            const float *__restrict__ X, int64_t ldx, float *__restrict__ O, int64_t ldo,
            float *__restrict__ P, int M, int N, int K, int chunks) {
  constexpr int GQ = 8, MS = 2, XR = 8 * MT, KS = 32 * GQ;  // groups / k of a chunk, x rows
  constexpr int XE = XR / 4;  // x float4 per thread: float4 i of thread t is row wave + 4 i
  __shared__ __align__(16) _Float16 xh[XR][KS];
  __shared__ __align__(16) _Float16 xl[XR][KS];
  __shared__ float xs[XR][GQ];
  __shared__ float fm[XR];
  const int G = K >> 5;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n16 = lane & 15, q = lane >> 4;
  const int row0 = ((int)blockIdx.x * 4 + wave) * RT * 16;
  const int ar = n16 >> 1;  // x row (within an 8-row tile) of this lane's A fragment
  float acc[RT][MT][2];
#pragma unroll
  for (int rt = 0; rt < RT; rt++)
#pragma unroll
    for (int t = 0; t < MT; t++) acc[rt][t][0] = acc[rt][t][1] = 0.f;
  for (int c = 0; c < chunks; c++) {
    const int gbeg = ((int)blockIdx.y * chunks + c) * GQ, gend = min(G, gbeg + GQ);
    if (gbeg >= G) break;  // uniform per block
    // every load of the chunk first: weights and scales, then x
    uint4 wv[RT][MS];
    float sc[RT][MS][4];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
      const int n = min(row0 + 16 * rt + n16, N - 1);
      const uint8_t *wrow = W + (int64_t)n * ldw;
      const float *srow = S + (int64_t)n * lds;
#pragma unroll
      for (int st = 0; st < MS; st++) {
        wv[rt][st] = *(const uint4 *)(wrow + 16 * min(gbeg + 4 * st + q, G - 1));
#pragma unroll
        for (int j = 0; j < 4; j++) sc[rt][st][j] = srow[min(gbeg + 4 * st + j, G - 1)];
      }
    }
    float4 xr[XE];
#pragma unroll
    for (int i = 0; i < XE; i++) {
      const int m = wave + 4 * i, k = 32 * gbeg + 4 * lane;
      xr[i] = (m < M && k < K) ? *(const float4 *)(X + (int64_t)m * ldx + k)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (c > 0) lds_barrier();  // the previous chunk's x reads are done
    // x of the chunk: each wave holds whole rows (64 lanes x 4 = KS values)
#pragma unroll
    for (int i = 0; i < XE; i++) {
      const int m = wave + 4 * i;
      const float v[4] = {xr[i].x, xr[i].y, xr[i].z, xr[i].w};
      const float mx = wave_max_dpp(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
      int ex = 0;
      if (mx > 16384.f) frexpf(mx * (1.f / 16384.f), &ex);  // mx / 2^ex < 16384
      const float down = ldexpf(1.f, -ex);
      _Float16 h[4], l[4];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float y = v[e] * down;
        h[e] = (_Float16)y;
        l[e] = (_Float16)(y - (float)h[e]);
      }
      __builtin_memcpy(&xh[m][4 * lane], h, 8);
      __builtin_memcpy(&xl[m][4 * lane], l, 8);
      // sum over the 8 lanes of a group: quads, then quad with quad (the half
      // mirror pairs lane i with 7 - i, the same two quad sums as lane ^ 4)
      float t = (v[0] + v[1]) + (v[2] + v[3]);
      t += dpp_mov<kDppXor1>(t);
      t += dpp_mov<kDppXor2>(t);
      t += dpp_mov<kDppHalfMirror>(t);
      if ((lane & 7) == 0) xs[m][lane >> 3] = t;
      if (lane == 0) fm[m] = ldexpf(1.f, 24 + ex);
    }
    lds_barrier();
#pragma unroll
    for (int st = 0; st < MS; st++) {
      if (gbeg + 4 * st >= gend) break;  // uniform per block
      uint32_t t4[RT][4];
#pragma unroll
      for (int rt = 0; rt < RT; rt++) {
        t4[rt][0] = wv[rt][st].x ^ 0x88888888u;
        t4[rt][1] = wv[rt][st].y ^ 0x88888888u;
        t4[rt][2] = wv[rt][st].z ^ 0x88888888u;
        t4[rt][3] = wv[rt][st].w ^ 0x88888888u;
        xpose4x4(t4[rt]);
      }
      // all MFMAs of the step first (independent accumulators), then the
      // per-group scaling, so no MFMA result is waited for right after issue
      w4f4 d[4][RT][MT];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int gl = min(4 * st + j, GQ - 1);  // groups past the chunk: computed, not used
        w4h8 a[MT];
#pragma unroll
        for (int t = 0; t < MT; t++) {
          const int m = 8 * t + ar;
          a[t] = w4h8{0, 0, 0, 0, 0, 0, 0, 0};
          if (m < M) a[t] = *(const w4h8 *)((n16 & 1 ? &xl[m][0] : &xh[m][0]) + 32 * gl + 8 * q);
        }
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
          const w4h8 b = nib8_f16(t4[rt][j]);
#pragma unroll
          for (int t = 0; t < MT; t++)
            d[j][rt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t], b, w4f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        }
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int gl = 4 * st + j;
        if (gbeg + gl >= gend) break;
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
          for (int e = 0; e < 2; e++) {
            const int m = 8 * t + 2 * q + e;  // D rows 4q + 2e (hi) and 4q + 2e + 1 (lo)
            const float f = fm[m], xsm = xs[m][gl];
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
              const float sv = sc[rt][st][j];
              acc[rt][t][e] = fmaf(sv * f, d[j][rt][t][2 * e] + d[j][rt][t][2 * e + 1],
                                   fmaf(-8.f * sv, xsm, acc[rt][t][e]));
            }
          }
      }
    }
  }
#pragma unroll
  for (int rt = 0; rt < RT; rt++) {
    const int nn = row0 + 16 * rt + n16;
    if (nn >= N) continue;
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
      for (int e = 0; e < 2; e++) {
        const int m = 8 * t + 2 * q + e;
        if (m >= M) continue;
        if (gridDim.y == 1) O[(int64_t)m * ldo + nn] = acc[rt][t][e];
        else P[((int64_t)blockIdx.y * M + m) * N + nn] = acc[rt][t][e];
      }
  }
}

// out[m][n] = sum over parts p (in order) of P[p][m][n]; the loads of B
// parts are issued together (B about nparts: one round of loads instead of
// one per part took 8640->3200 M=16 from 21.8 to 19.0 us).
template <int B>
__global__ void __launch_bounds__(256)
    w4s_sum_parts(const float *__restrict__ P, int nparts, float *__restrict__ O, int64_t ldo, int M,
                  int N) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)M * N) return;
  float t = 0.f;
  for (int p = 0; p < nparts; p += B) {
    float v[B];
#pragma unroll
    for (int u = 0; u < B; u++) v[u] = p + u < nparts ? P[(int64_t)(p + u) * M * N + i] : 0.f;
#pragma unroll
    for (int u = 0; u < B; u++)
      if (p + u < nparts) t += v[u];
  }
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

// out[i] = dequant_w4(Q, S, Z, idx0 + i, gs) for i < count: the unsigned
// nibble of flat element idx0 + i (low nibble = even element) times its
// group's scale, plus its group's zero, rounded after the multiply and after
// the add as the lowering's separate mulf and addf (ConvertSimpToMemRef.cpp:
// 2423-2424) do. Q, S and Z start at byte b0 and group g0 of the arrays.
__global__ void __launch_bounds__(256)
    dequant_w4_k(const uint8_t *__restrict__ Q, const float *__restrict__ S,
                 const float *__restrict__ Z, float *__restrict__ O, int64_t idx0, int64_t count,
                 int64_t gs, int64_t b0, int64_t g0) {
  // hipcc contracts a*b+c into one fma by default, which rounds once
#pragma clang fp contract(off)
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * 256) {
    const int64_t e = idx0 + i, g = e / gs - g0;
    const uint8_t b = Q[(e >> 1) - b0];
    const int q = (e & 1) ? (b >> 4) : (b & 15);
    const float scaled = (float)q * S[g];
    O[i] = scaled + Z[g];
  }
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
  } else if (M >= 2 && M <= 4 && w4d8_supported(K, gs, X, nullptr) &&
             (size_t)100 * (M <= 2 ? 2 : 4) * (K / 32) + 4096 <= 160 * 1024) {
    // up to four x vectors: the dot8 kernel with the limbs of every vector in
    // registers, the weights read once (w4d8.hip); their limb tables (100
    // bytes per vector and chunk) must fit the 160 KB of LDS
    W4D8Args a{};
    a.s[0] = W4D8Seg{W, S, O, ldw, lds, N};
    a.n = 1;
    a.K = K;
    a.gs = gs;
    a.x0 = X;
    a.nw = nullptr;
    a.eps = 0.f;
    a.out_mode = 0;
    a.mx = M;
    a.ldx = ldx;
    a.ldo = ldo;
    return launch_w4d8(a, st);
  } else if (M >= 2 && gs == 32) {
    // several x vectors, groups of 32: f16 MFMA.  A block takes 4 waves x RT
    // tiles of 16 weight rows and `chunks` chunks of 8 groups of K; the K parts
    // (gridDim.y) make about two blocks per CU, and with more than one part the
    // partial tiles go through a workspace and an ordered sum.
    constexpr int RT = 2;
    const int nb = (int)cdiv(N, 64 * RT), ng = K / 32, nck = (int)cdiv(ng, 8);
    const int want = (int)std::max<int64_t>(1, cdiv(2 * num_cus(), nb));
    const int chunks = (int)cdiv(nck, std::min(want, nck));
    const int parts = (int)cdiv(nck, chunks);
    float *P = nullptr;
    if (parts > 1) {
      int rc = workspace(st, sizeof(float) * (size_t)parts * M * N, (void **)&P, 2);
      if (rc) return rc;
    }
    KernelTimer kt(st, "w4s_h16");
    if (M <= 8)
      hipLaunchKernelGGL((w4s_h16<1, RT>), dim3((unsigned)nb, (unsigned)parts), dim3(256), 0, st, W,
                         ldw, S, lds, X, ldx, O, ldo, P, M, N, K, chunks);
    else
      hipLaunchKernelGGL((w4s_h16<2, RT>), dim3((unsigned)nb, (unsigned)parts), dim3(256), 0, st, W,
                         ldw, S, lds, X, ldx, O, ldo, P, M, N, K, chunks);
    if (parts > 1) {
      const dim3 g((unsigned)cdiv((int64_t)M * N, 256));
      if (parts <= 4) hipLaunchKernelGGL(w4s_sum_parts<4>, g, dim3(256), 0, st, P, parts, O, ldo, M, N);
      else if (parts <= 8) hipLaunchKernelGGL(w4s_sum_parts<8>, g, dim3(256), 0, st, P, parts, O, ldo, M, N);
      else hipLaunchKernelGGL(w4s_sum_parts<16>, g, dim3(256), 0, st, P, parts, O, ldo, M, N);
    }
  } else if (M == 1 && w4d8_supported(K, gs, X, nullptr)) {
    // one x vector: exact integer chunk products on v_dot8_i32_i4 (w4d8.hip)
    W4D8Args a{};
    a.s[0] = W4D8Seg{W, S, O, ldw, lds, N};
    a.n = 1;
    a.K = K;
    a.gs = gs;
    a.x0 = X;
    a.nw = nullptr;
    a.eps = 0.f;
    a.out_mode = 0;
    return launch_w4d8(a, st);
  } else if (M == 1 && K / 32 <= 32 * 16) {
    // one x vector: the barrier-free kernel, UB chunks per lane with G*UB >= K/32;
    // 8 waves per block for rows of more than 64 chunks unless there are 8 or
    // more blocks of 8 rows per CU (3200x8640: 7.45 -> 7.1 us, 8640x3200:
    // 10.6 -> 8.8 us; 3200x32000 measured no better)
    const int nchunk = K / 32;
    const dim3 grid((unsigned)cdiv(N, 8));
    KernelTimer kt(st, "w4s_gemv");
#define W4S1(U, V) \
  hipLaunchKernelGGL((w4s_gemv1<U, V>), grid, dim3(64 * V), 0, st, W, ldw, S, lds, X, O, N, K, gs)
    if (nchunk > 64 && (int64_t)grid.x < 8 * num_cus()) {
      if (nchunk <= 128) W4S1(2, 8);
      else if (nchunk <= 384) W4S1(6, 8);
      else W4S1(8, 8);
    } else {
      if (nchunk <= 64) W4S1(2, 4);
      else if (nchunk <= 128) W4S1(4, 4);
      else if (nchunk <= 256) W4S1(8, 4);
      else if (nchunk <= 384) W4S1(12, 4);
      else W4S1(16, 4);
    }
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
  } else if (w4d8_supported(cols, gs, X, nullptr)) {
    // exact integer chunk products on v_dot8_i32_i4 (w4d8.hip): groups start
    // at row starts (off and cols are multiples of gs), so row n's scales
    // and zeros are at (off + n cols) / gs
    W4D8Args a{};
    a.s[0] = W4D8Seg{Q + off / 2, S + off / gs, O, cols / 2, cols / gs, rows, Z + off / gs};
    a.n = 1;
    a.K = cols;
    a.gs = gs;
    a.x0 = X;
    a.nw = nullptr;
    a.eps = 0.f;
    a.out_mode = 0;
    return launch_w4d8(a, st);
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

int32_t simp_rt_dequant_w4(
    const int8_t *qw_alloc, const int8_t *qw, int64_t qw_off, int64_t qw_size, int64_t qw_stride,
    const float *s_alloc, const float *s, int64_t s_off, int64_t s_size, int64_t s_stride,
    const float *z_alloc, const float *z, int64_t z_off, int64_t z_size, int64_t z_stride,
    int64_t idx, int64_t group_size, float *out_alloc, float *out, int64_t out_off,
    int64_t out_size, int64_t out_stride, int64_t count) {
  (void)qw_alloc; (void)s_alloc; (void)z_alloc; (void)out_alloc;
  int rc;
  if ((rc = check_desc1("qweights", qw, qw_off, qw_size, qw_stride))) return rc;
  if ((rc = check_desc1("scales", s, s_off, s_size, s_stride))) return rc;
  if ((rc = check_desc1("zeros", z, z_off, z_size, z_stride))) return rc;
  if ((rc = check_desc1("output", out, out_off, out_size, out_stride))) return rc;
  if (idx < 0 || count < 0 || group_size <= 0)
    return set_error(SIMP_RT_EINVAL, "dequant_w4: bad idx/count/group_size");
  if (count == 0) return SIMP_RT_OK;
  const int64_t last = idx + count - 1;  // the last element dequantized
  const int64_t b0 = idx / 2, b1 = last / 2, g0 = idx / group_size, g1 = last / group_size;
  if (b1 >= qw_size || g1 >= s_size || g1 >= z_size || count > out_size)
    return set_error(SIMP_RT_EINVAL,
                     "dequant_w4: arrays too small for idx=%lld count=%lld gs=%lld",
                     (long long)idx, (long long)count, (long long)group_size);
  // only the bytes and groups the range touches are bound (a host array is
  // staged for that slice alone)
  Operand oq, os, oz, oo;
  if ((rc = oq.bind(qw + qw_off + b0, (size_t)(b1 - b0 + 1), Operand::kIn, "qweights"))) return rc;
  if ((rc = os.bind(s + s_off + g0, sizeof(float) * (size_t)(g1 - g0 + 1), Operand::kIn, "scales")))
    return rc;
  if ((rc = oz.bind(z + z_off + g0, sizeof(float) * (size_t)(g1 - g0 + 1), Operand::kIn, "zeros")))
    return rc;
  if ((rc = oo.bind(out + out_off, sizeof(float) * (size_t)count, Operand::kOut, "output"))) return rc;
  const unsigned grid = (unsigned)std::min<int64_t>(cdiv(count, 256), (int64_t)num_cus() * 16);
  hipLaunchKernelGGL(dequant_w4_k, dim3(grid), dim3(256), 0, cur_stream(),
                     (const uint8_t *)oq.dev(), (const float *)os.dev(), (const float *)oz.dev(),
                     (float *)oo.dev(), idx, count, group_size, b0, g0);
  SIMP_HIP(hipGetLastError());
  Operand *ops[] = {&oq, &os, &oz, &oo};
  return finish(ops, 4);
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
