// f32.hip -- fp32 matmul entry points.
//   matmul (array builtin)  C += A*B on 1-D arrays viewed as row-major matrices
//                           at element offsets (MatMulOpLowering,
//                           ConvertSimpToMemRef.cpp:1794-1920: linalg.matmul
//                           accumulates into the caller's buffer, F4)
//   tensor_matmul (f32)     C = A*B into a caller buffer (ConvertSimpToMemRef.cpp:3280-3284)
//   tensor_matmul_nt (f32)  C = A*B_T^T (naive float branch, :3445-3481)
//   tensor_matvecmul (f32)  the same product as tensor_matmul (:3632-3792, f32 loops :3763-3787)
// n == 1 (every LLaMA decode projection, stories110M.sl:77-83) is an HBM-bound
// GEMV: one wave per output row at a time, lanes along K with 16-byte loads, x
// held in registers for the whole kernel, the next row's loads in flight while
// the current row is reduced.  n > 1 runs an LDS-tiled fp32 GEMM.
#include <algorithm>
#include <type_traits>

#include "rt_device.h"
#include "rt_internal.h"

namespace simp {
namespace {

// y[i] = beta*y[i] + sum_k A[i*lda + k] x[k]; J = float4 slots of x per lane (K <= 256*J).
template <int J>
__global__ void __launch_bounds__(256)
    gemv_f32(const float *__restrict__ A, int64_t lda, const float *__restrict__ x,
             float *__restrict__ y, int rows, int K, float beta) {
  const int lane = threadIdx.x & 63;
  const int nw = gridDim.x * 4;
  int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  float4 xv[J];
#pragma unroll
  for (int j = 0; j < J; j++) {
    const int k = 4 * lane + 256 * j;
    xv[j] = k < K ? *(const float4 *)(x + k) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float4 a[J];
  auto load = [&](int r, float4 (&v)[J]) {
    const float *p = A + (int64_t)r * lda;
#pragma unroll
    for (int j = 0; j < J; j++) {
      const int k = 4 * lane + 256 * j;
      v[j] = k < K ? *(const float4 *)(p + k) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  if (row < rows) load(row, a);
  for (; row < rows; row += nw) {
    float4 b[J];
    if (row + nw < rows) load(row + nw, b);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < J; j++) {
      s = fmaf(a[j].x, xv[j].x, s);
      s = fmaf(a[j].y, xv[j].y, s);
      s = fmaf(a[j].z, xv[j].z, s);
      s = fmaf(a[j].w, xv[j].w, s);
    }
    s = wave_sum(s);
    if (lane == 0) y[row] = beta != 0.f ? y[row] + s : s;
#pragma unroll
    for (int j = 0; j < J; j++) a[j] = b[j];
  }
}

// Scalar-load GEMV for misaligned / long rows (x read from global, L1-resident).
__global__ void __launch_bounds__(256)
    gemv_f32_any(const float *__restrict__ A, int64_t lda, const float *__restrict__ x,
                 float *__restrict__ y, int rows, int K, float beta) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float *p = A + (int64_t)row * lda;
  float s = 0.f;
  for (int k = lane; k < K; k += 64) s = fmaf(p[k], x[k], s);
  s = wave_sum(s);
  if (lane == 0) y[row] = beta != 0.f ? y[row] + s : s;
}

__device__ __forceinline__ float fma_t(float a, float b, float c) { return fmaf(a, b, c); }
__device__ __forceinline__ double fma_t(double a, double b, double c) { return fma(a, b, c); }

// C = beta*C + A*B, 64x64 tile per 256 threads, each thread a 4x4 block; T is
// float or double.  BT: B is given transposed, B_T[N,K] (row n holds column n
// of B).  Workgroup x indexes the tiles (n fastest), z the batch: operand
// bases advance by sa/sb/sc elements per batch.
template <typename T, bool BT>
__global__ void __launch_bounds__(256)
    gemm_t(const T *__restrict__ A, int64_t lda, int64_t sa, const T *__restrict__ B, int64_t ldb,
           int64_t sb, T *__restrict__ C, int64_t ldc, int64_t sc, int M, int N, int K,
           int tiles_n, T beta) {
  __shared__ T sa_t[16][64 + 1];
  __shared__ T sb_t[16][64 + 1];
  A += blockIdx.z * sa;
  B += blockIdx.z * sb;
  C += blockIdx.z * sc;
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int tm = (int)(blockIdx.x / (unsigned)tiles_n), tn = (int)(blockIdx.x % (unsigned)tiles_n);
  const int m0 = tm * 64, n0 = tn * 64;
  T acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
    for (int i = threadIdx.x; i < 16 * 64; i += 256) {
      const int kk = i & 15, mm = i >> 4;  // A tile, k fastest
      const int gm = m0 + mm, gk = k0 + kk;
      sa_t[kk][mm] = (gm < M && gk < K) ? A[(int64_t)gm * lda + gk] : T(0);
      if constexpr (BT) {
        const int gn = n0 + mm;  // B_T tile, k fastest (rows of B_T are contiguous in k)
        sb_t[kk][mm] = (gn < N && gk < K) ? B[(int64_t)gn * ldb + gk] : T(0);
      } else {
        const int nn = i & 63, kb = i >> 6;  // B tile, n fastest
        const int gn = n0 + nn, gk2 = k0 + kb;
        sb_t[kb][nn] = (gn < N && gk2 < K) ? B[(int64_t)gk2 * ldb + gn] : T(0);
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; kk++) {
      T av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; i++) av[i] = sa_t[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; j++) bv[j] = sb_t[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = fma_t(av[i], bv[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int gm = m0 + ty * 4 + i, gn = n0 + tx * 4 + j;
      if (gm < M && gn < N) {
        T *c = C + (int64_t)gm * ldc + gn;
        *c = beta != T(0) ? *c + acc[i][j] : acc[i][j];
      }
    }
}

// ---------------------------------------------------------------- MFMA path
// fp32 GEMM on v_mfma_f32_16x16x4_f32.  Block tile BM x BN (WGM x WGN waves,
// each (BM/WGM) x (BN/WGN) in 16x16 MFMA tiles), K in steps of BK through a
// double-buffered LDS tile filled from registers (the next step's global loads
// are in flight while the current step's MFMAs run).  Within each 16 of K,
// lane group g = lane/16 takes k = 4g..4g+3 over the four MFMAs, so each lane
// reads its A (and B_T) operands as one float4 from k-contiguous LDS rows; B
// given as [K,N] stays n-contiguous in LDS and is read as four floats.
// grid: x = output tiles (n fastest), y = K splits, z = batch.  With one split
// the result goes to C (beta 0: overwrite, 1: accumulate); with several, each
// split writes its own partial slice P[z][split][M][N] for gemm_f32_sum_parts.
// Requirements (checked by the dispatch): K, lda (and ldb for B_T) multiples of
// 4, N and ldb multiples of 4 for B[K,N], 16-byte aligned bases and batch strides.
typedef float v4f __attribute__((ext_vector_type(4)));

template <int BM, int BN, int WGM, int WGN, bool BT, int BK = 16>
__global__ void __launch_bounds__(WGM *WGN * 64)
    gemm_f32_mfma(const float *__restrict__ A, int64_t lda, int64_t sa, const float *__restrict__ B,
                  int64_t ldb, int64_t sb, float *__restrict__ C, int64_t ldc, int64_t sc,
                  float *__restrict__ P, int M, int N, int K, int tiles_n, int k_span, float beta) {
  constexpr int NT = WGM * WGN * 64;
  static_assert(BK % 16 == 0, "K step");
  constexpr int WM = BM / WGM, WN = BN / WGN, FM = WM / 16, FN = WN / 16;
  static_assert(WM % 16 == 0 && WN % 16 == 0, "wave tile");
  constexpr int LDA = BK + 4;                  // k-contiguous rows (A, and B_T)
  constexpr int LDB = BT ? BK + 4 : BN + 4;    // B[K,N]: n-contiguous rows
  constexpr int KQ = BK / 4;                   // float4 per k-contiguous row
  constexpr int A_TOT = BM * BK / 4, A_PER = (A_TOT + NT - 1) / NT;
  constexpr int B_TOT = BN * BK / 4, B_PER = (B_TOT + NT - 1) / NT;
  __shared__ __align__(16) float As[2][BM * LDA];
  __shared__ __align__(16) float Bs[2][BT ? BN * LDB : BK * LDB];

  A += blockIdx.z * sa;
  B += blockIdx.z * sb;
  C += blockIdx.z * sc;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;
  const int tm = (int)(blockIdx.x / (unsigned)tiles_n), tn = (int)(blockIdx.x % (unsigned)tiles_n);
  const int m0 = tm * BM, n0 = tn * BN;
  const int kbeg = blockIdx.y * k_span, kend = min(K, kbeg + k_span);
  const int nk = kbeg < kend ? (kend - kbeg + BK - 1) / BK : 0;

  float4 ra[A_PER], rb[B_PER];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_PER; i++) {
      const int c = tid + i * NT;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (A_TOT % NT == 0 || c < A_TOT) {
        const int m = c / KQ, gm = m0 + m, gk = k0 + 4 * (c % KQ);
        if (gm < M && gk < kend) v = *(const float4 *)(A + (int64_t)gm * lda + gk);
      }
      ra[i] = v;
    }
#pragma unroll
    for (int i = 0; i < B_PER; i++) {
      const int c = tid + i * NT;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (B_TOT % NT == 0 || c < B_TOT) {
        if constexpr (BT) {
          const int n = c / KQ, gn = n0 + n, gk = k0 + 4 * (c % KQ);
          if (gn < N && gk < kend) v = *(const float4 *)(B + (int64_t)gn * ldb + gk);
        } else {
          const int kr = c / (BN / 4), gk = k0 + kr, gn = n0 + 4 * (c % (BN / 4));
          if (gk < kend && gn < N) v = *(const float4 *)(B + (int64_t)gk * ldb + gn);
        }
      }
      rb[i] = v;
    }
  };
  auto store = [&](int st) {
#pragma unroll
    for (int i = 0; i < A_PER; i++) {
      const int c = tid + i * NT;
      if (A_TOT % NT == 0 || c < A_TOT) *(float4 *)&As[st][(c / KQ) * LDA + 4 * (c % KQ)] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_PER; i++) {
      const int c = tid + i * NT;
      if (B_TOT % NT == 0 || c < B_TOT) {
        if constexpr (BT) *(float4 *)&Bs[st][(c / KQ) * LDB + 4 * (c % KQ)] = rb[i];
        else *(float4 *)&Bs[st][(c / (BN / 4)) * LDB + 4 * (c % (BN / 4))] = rb[i];
      }
    }
  };

  v4f acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  if (nk > 0) {
    load(kbeg);
    store(0);
    __syncthreads();
  }
  for (int kt = 0; kt < nk; kt++) {
    const int st = kt & 1;
    if (kt + 1 < nk) load(kbeg + (kt + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      float4 a[FM];
#pragma unroll
      for (int i = 0; i < FM; i++)
        a[i] = *(const float4 *)&As[st][(wm0 + 16 * i + r16) * LDA + kk + 4 * g];
      float b[FN][4];
#pragma unroll
      for (int j = 0; j < FN; j++) {
        if constexpr (BT) {
          const float4 v = *(const float4 *)&Bs[st][(wn0 + 16 * j + r16) * LDB + kk + 4 * g];
          b[j][0] = v.x; b[j][1] = v.y; b[j][2] = v.z; b[j][3] = v.w;
        } else {
#pragma unroll
          for (int q = 0; q < 4; q++) b[j][q] = Bs[st][(kk + 4 * g + q) * LDB + wn0 + 16 * j + r16];
        }
      }
#pragma unroll
      for (int q = 0; q < 4; q++)
#pragma unroll
        for (int i = 0; i < FM; i++) {
          const float av = q == 0 ? a[i].x : q == 1 ? a[i].y : q == 2 ? a[i].z : a[i].w;
#pragma unroll
          for (int j = 0; j < FN; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b[j][q], acc[i][j], 0, 0, 0);
        }
    }
    if (kt + 1 < nk) {
      store(st ^ 1);  // the other buffer was last read before the previous barrier
      __syncthreads();
    }
  }
  // D layout: lane holds rows 4g + r (r < 4) of column r16 of each 16x16 tile
  float *Pz = P ? P + ((int64_t)blockIdx.z * gridDim.y + blockIdx.y) * M * N : nullptr;
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++) {
      const int col = n0 + wn0 + 16 * j + r16;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int row = m0 + wm0 + 16 * i + 4 * g + r;
        if (row < M && col < N) {
          const float v = acc[i][j][r];
          if (Pz) {
            Pz[(int64_t)row * N + col] = v;
          } else {
            float *c = C + (int64_t)row * ldc + col;
            *c = beta != 0.f ? *c + v : v;
          }
        }
      }
    }
}

// fp32 GEMM fed by an LDS-DMA ring, K % 32 == 0: BM x BN C tiles of `batch`
// products (operand bases sa / sb / sc elements apart), WGM x WGN waves,
// v_mfma_f32_16x16x4f32, the whole of K in one workgroup (no split-K partials
// to sum afterwards).
//   * K-stages of 32 floats: an A (or B_T) row gives one whole 128-byte line
//     per stage.  Operand tiles go global -> LDS directly
//     (global_load_lds_dwordx4, each instruction 1 KB in lane order) into a
//     ring of SLOTS stages, SLOTS-1 stages ahead of the MFMAs, one barrier per
//     stage; the loads are counted with the kernel's own s_waitcnt vmcnt.
//   * A / B_T: an instruction is 8 rows x 128 B, lane l row l/8; slot l%8 of
//     row r holds 16-byte chunk (l%8) ^ ((r >> 1) & 7), so the 16 lanes of an
//     operand read (rows R..R+15, one chunk) fall on 16 distinct 16-byte bank
//     groups.
//   * B given as [K,N]: a stage is 32 k-rows of BN floats; slot s of k-row k
//     holds chunk s ^ (4 ((k >> 2) & 3)), so the four k-rows read together
//     (one per 16-lane group) fall on four distinct 64-byte bank ranges.
//   * Within each 16 of K, lane group g = lane/16 takes k = 4g..4g+3 over the
//     four MFMAs: one 16-byte LDS read per A (B_T) fragment, four 4-byte reads
//     per B fragment.  Fragments are double-buffered in registers.
//   * The MFMA computes C^T tiles (B fragment first), so a lane ends with 4
//     consecutive columns of one row of C: 16-byte stores.
//   * Persistent: gridDim.x workgroups walk the products' tiles, each product's
//     in tile_of_block order.
//     Rows past M and columns past N load from clamped in-bounds addresses and
//     are never stored.
// Requirements (checked by the dispatch): K % 32 == 0, N % 4 == 0, lda, ldb,
// ldc and the batch strides multiples of 4, 16-byte aligned A, B and C.
template <int BM, int BN, int WGM, int WGN, int SLOTS, bool BT>
__global__ void __launch_bounds__(64 * WGM * WGN)
    gemm_f32_ring(const float *__restrict__ A, int64_t lda, int64_t sa, const float *__restrict__ B,
                  int64_t ldb, int64_t sb, float *__restrict__ C, int64_t ldc, int64_t sc, int M,
                  int N, int K, int tiles_m, int tiles_n, int batch, float beta) {
  constexpr int NW = WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN, FM = WM / 16, FN = WN / 16;
  constexpr int BK = 32;                                   // floats per stage
  constexpr int SA = BM * BK * 4, SB = BN * BK * 4, STAGE = SA + SB;  // bytes
  constexpr int DA = SA / 1024 / NW, DB = SB / 1024 / NW;  // DMA instructions per wave
  constexpr int DPW = DA + DB;
  static_assert(WM % 16 == 0 && WN % 16 == 0, "wave tile");
  static_assert(DA >= 1 && DB >= 1 && DA * NW * 1024 == SA && DB * NW * 1024 == SB, "DMA split");
  static_assert(DPW * (SLOTS - 1) <= 63, "vmcnt range");
  // [K,N] B: the swizzle XORs chunk indices with up to 12, so a k-row needs 16 chunks
  static_assert(BT || BN % 64 == 0, "B[K,N] tile width");
  constexpr int LPR = BN / 4, RPI = 64 / LPR;  // [K,N] B: lanes per k-row, k-rows per DMA
  __shared__ float4 lds[SLOTS * STAGE / 16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;
  const int r16 = lane & 15, g = lane >> 4;
  const int ns = K / BK;
  const int ntiles = tiles_m * tiles_n;
  const uint32_t lds_base = lds_offset(lds);
  const float *lds_f = (const float *)lds;

  for (int vb = blockIdx.x; vb < ntiles * batch; vb += gridDim.x) {
    // product z = vb / ntiles, its tile in tile_of_block order
    const int z = vb / ntiles;
    int tm, tn;
    tile_of_block(vb - z * ntiles, ntiles, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const float *Az = A + z * sa, *Bz = B + z * sb;
    float *Cz = C + z * sc;
    const float *srcA[DA], *srcB[DB];
#pragma unroll
    for (int i = 0; i < DA; i++) {
      const int r = 8 * (wave * DA + i) + (lane >> 3);
      srcA[i] = Az + (int64_t)min(m0 + r, M - 1) * lda + 4 * ((lane & 7) ^ ((r >> 1) & 7));
    }
#pragma unroll
    for (int i = 0; i < DB; i++) {
      if constexpr (BT) {
        const int r = 8 * (wave * DB + i) + (lane >> 3);
        srcB[i] = Bz + (int64_t)min(n0 + r, N - 1) * ldb + 4 * ((lane & 7) ^ ((r >> 1) & 7));
      } else {
        const int kr = RPI * (wave * DB + i) + lane / LPR;  // k-row within the stage
        const int cb = (lane % LPR) ^ (((kr >> 2) & 3) << 2);
        srcB[i] = Bz + (int64_t)kr * ldb + min(n0 + 4 * cb, N - 4);
      }
    }
    auto issue = [&](int st) {
      const uint32_t dst = lds_base + (uint32_t)(st % SLOTS) * STAGE;
      const int64_t ka = (int64_t)st * BK;
#pragma unroll
      for (int i = 0; i < DA; i++) dma16(srcA[i] + ka, dst + 1024 * (wave * DA + i));
      const int64_t kb = BT ? ka : ka * ldb;
#pragma unroll
      for (int i = 0; i < DB; i++) dma16(srcB[i] + kb, dst + SA + 1024 * (wave * DB + i));
    };
    // fragment reads of stage st, K half h (k = 16 h .. 16 h + 15 of the stage)
    auto afrag = [&](int st, int r0, int h) {
      const int r = r0 + r16;
      const uint32_t off = (uint32_t)(st % SLOTS) * STAGE + r * 128 + (((4 * h + g) ^ ((r >> 1) & 7)) << 4);
      return lds[off >> 4];
    };
    auto bfrag = [&](int st, int c0, int h) {
      if constexpr (BT) {
        const int r = c0 + r16;
        const uint32_t off = (uint32_t)(st % SLOTS) * STAGE + SA + r * 128 +
                             (((4 * h + g) ^ ((r >> 1) & 7)) << 4);
        return lds[off >> 4];
      } else {
        // k-row 16 h + 4 g + t, column c0 + r16: chunk (c0 + r16) / 4 sits in
        // slot chunk ^ 4g (rows 16h+4g..16h+4g+3 share the swizzle)
        const int n = c0 + r16;
        const uint32_t base = (uint32_t)(st % SLOTS) * STAGE + SA + (16 * h + 4 * g) * (4 * BN) +
                              ((((n >> 2) ^ (4 * g))) << 4) + 4 * (n & 3);
        float4 v;
        v.x = lds_f[(base + 0 * 4 * BN) >> 2];
        v.y = lds_f[(base + 1 * 4 * BN) >> 2];
        v.z = lds_f[(base + 2 * 4 * BN) >> 2];
        v.w = lds_f[(base + 3 * 4 * BN) >> 2];
        return v;
      }
    };
    v4f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
    float4 fra[2][FM], frb[2][FN];
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // the previous tile's stores
    const int first = min(SLOTS, ns);
    for (int st = 0; st < first; st++) issue(st);
    auto wait_after = [&](int n_after) { wait_vm_le<DPW, SLOTS - 1>(n_after); };
    wait_after(first - 1);  // stage 0 done on this wave ...
    block_barrier();        // ... and on every wave
#pragma unroll
    for (int j = 0; j < FN; j++) frb[0][j] = bfrag(0, wn0 + 16 * j, 0);
#pragma unroll
    for (int i = 0; i < FM; i++) fra[0][i] = afrag(0, wm0 + 16 * i, 0);
    auto mfmas = [&](int cb) {
#pragma unroll
      for (int t = 0; t < 4; t++)
#pragma unroll
        for (int i = 0; i < FM; i++) {
          const float av = t == 0 ? fra[cb][i].x : t == 1 ? fra[cb][i].y : t == 2 ? fra[cb][i].z : fra[cb][i].w;
#pragma unroll
          for (int j = 0; j < FN; j++) {
            const float bv = t == 0 ? frb[cb][j].x : t == 1 ? frb[cb][j].y : t == 2 ? frb[cb][j].z : frb[cb][j].w;
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(bv, av, acc[i][j], 0, 0, 0);
          }
        }
    };
    for (int s = 0; s < ns; s++) {
      // half (s,0): read (s,1)'s fragments, run (s,0)
#pragma unroll
      for (int j = 0; j < FN; j++) frb[1][j] = bfrag(s, wn0 + 16 * j, 1);
#pragma unroll
      for (int i = 0; i < FM; i++) fra[1][i] = afrag(s, wm0 + 16 * i, 1);
      mfmas(0);
      const bool more = s + 1 < ns;
      // stages issued so far: 0 .. min(s + SLOTS - 1, ns - 1); stage s+1 must be done
      if (more) wait_after(min(SLOTS - 2, ns - 2 - s));
      __builtin_amdgcn_s_waitcnt(waitcnt_lgkm0);  // this wave's reads of stage s landed
      block_barrier();
      if (s + SLOTS < ns) issue(s + SLOTS);
      // half (s,1): read (s+1,0)'s fragments, run (s,1)
      if (more) {
#pragma unroll
        for (int j = 0; j < FN; j++) frb[0][j] = bfrag(s + 1, wn0 + 16 * j, 0);
#pragma unroll
        for (int i = 0; i < FM; i++) fra[0][i] = afrag(s + 1, wm0 + 16 * i, 0);
      }
      mfmas(1);
    }
    // acc[i][j][r] = C[m0 + wm0 + 16 i + r16][n0 + wn0 + 16 j + 4 g + r]
#pragma unroll
    for (int j = 0; j < FN; j++) {
      const int col = n0 + wn0 + 16 * j + 4 * g;
#pragma unroll
      for (int i = 0; i < FM; i++) {
        const int row = m0 + wm0 + 16 * i + r16;
        if (row >= M || col >= N) continue;  // N % 4 == 0: col < N covers col..col+3
        float4 *dst = (float4 *)(Cz + (int64_t)row * ldc + col);
        float4 v = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
        if (beta != 0.f) {
          const float4 o = *dst;
          v.x += o.x; v.y += o.y; v.z += o.z; v.w += o.w;
        }
        *dst = v;
      }
    }
  }
}

// C[z] = beta*C[z] + sum_s P[z][s] (s increasing: deterministic); the loads
// of B parts are issued together.
template <int B>
__global__ void __launch_bounds__(256)
    gemm_f32_sum_parts(const float *__restrict__ P, float *__restrict__ C, int64_t ldc, int64_t sc,
                       int M, int N, int parts, float beta) {
  const int64_t mn = (int64_t)M * N;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= mn) return;
  const float *p = P + (int64_t)blockIdx.z * parts * mn + i;
  float v = 0.f;
  for (int s = 0; s < parts; s += B) {
    float t[B];
#pragma unroll
    for (int u = 0; u < B; u++) t[u] = s + u < parts ? p[(int64_t)(s + u) * mn] : 0.f;
#pragma unroll
    for (int u = 0; u < B; u++)
      if (s + u < parts) v += t[u];
  }
  const int64_t r = i / N, c = i - r * N;
  float *o = C + blockIdx.z * sc + r * ldc + c;
  *o = beta != 0.f ? *o + v : v;
}

template <int BM, int BN, int WGM, int WGN, bool BT, int BK = 16>
int launch_mfma_f32(const float *A, int64_t lda, int64_t sa, const float *B, int64_t ldb,
                    int64_t sb, float *C, int64_t ldc, int64_t sc, int M, int N, int K, int batch,
                    float beta, hipStream_t st) {
  const int64_t tiles_n = cdiv(N, BN), tiles = cdiv(M, BM) * tiles_n;
  if (tiles > INT32_MAX)
    return set_error(SIMP_RT_EUNSUPPORTED, "gemm: %lld output tiles exceed one launch",
                     (long long)tiles);
  // split K until there are about four blocks per CU: each split at least 64
  // deep, the partials no larger than the operands (they are written and read
  // once more) and within 1 GiB
  const int64_t cus = num_cus(), nkt = cdiv(K, 16);
  int64_t splits = 1;
  if (tiles * batch < 4 * cus && K >= 512) {
    const int64_t mn = (int64_t)M * N, ops = (int64_t)M * K + (int64_t)K * N;
    splits = std::min<int64_t>(std::min<int64_t>(cdiv(4 * cus, tiles * batch), 32), nkt / 4);
    splits = std::min<int64_t>(splits, ops / std::max<int64_t>(mn, 1));
    while (splits > 1 && (int64_t)batch * splits * mn * 4 > (int64_t(1) << 30)) splits--;
    splits = std::max<int64_t>(splits, 1);
  }
  const int k_span = (int)(cdiv(nkt, splits) * 16);
  splits = cdiv(K, k_span);
  float *P = nullptr;
  if (splits > 1) {
    int rc = workspace(st, sizeof(float) * (size_t)batch * splits * M * N, (void **)&P, 3);
    if (rc) return rc;
  }
  KernelTimer kt(st, "gemm_f32_mfma");
  hipLaunchKernelGGL((gemm_f32_mfma<BM, BN, WGM, WGN, BT, BK>),
                     dim3((unsigned)tiles, (unsigned)splits, (unsigned)batch), dim3(WGM * WGN * 64),
                     0, st, A, lda, sa, B, ldb, sb, C, ldc, sc, P, M, N, K, (int)tiles_n, k_span,
                     beta);
  SIMP_HIP(hipGetLastError());
  if (splits > 1) {
    const dim3 g((unsigned)cdiv((int64_t)M * N, 256), 1, (unsigned)batch);
    if (splits <= 4)
      hipLaunchKernelGGL(gemm_f32_sum_parts<4>, g, dim3(256), 0, st, (const float *)P, C, ldc, sc,
                         M, N, (int)splits, beta);
    else if (splits <= 8)
      hipLaunchKernelGGL(gemm_f32_sum_parts<8>, g, dim3(256), 0, st, (const float *)P, C, ldc, sc,
                         M, N, (int)splits, beta);
    else
      hipLaunchKernelGGL(gemm_f32_sum_parts<16>, g, dim3(256), 0, st, (const float *)P, C, ldc, sc,
                         M, N, (int)splits, beta);
    SIMP_HIP(hipGetLastError());
  }
  return SIMP_RT_OK;
}

// gemm_f32_ring over the tiles of `batch` products: persistent, up to per_cu
// workgroups per CU.
template <int BM, int BN, int WGM, int WGN, int SLOTS, bool BT>
int launch_ring_f32(const float *A, int64_t lda, int64_t sa, const float *B, int64_t ldb,
                    int64_t sb, float *C, int64_t ldc, int64_t sc, int M, int N, int K, int batch,
                    float beta, int per_cu, hipStream_t st) {
  const int64_t tm = cdiv(M, BM), tn = cdiv(N, BN), tiles = tm * tn * batch;
  if (tiles > INT32_MAX)
    return set_error(SIMP_RT_EUNSUPPORTED, "gemm: %lld output tiles exceed one launch",
                     (long long)tiles);
  const int grid = (int)std::min<int64_t>(tiles, (int64_t)per_cu * num_cus());
  KernelTimer kt(st, "gemm_f32_ring");
  hipLaunchKernelGGL((gemm_f32_ring<BM, BN, WGM, WGN, SLOTS, BT>), dim3(grid),
                     dim3(64 * WGM * WGN), 0, st, A, lda, sa, B, ldb, sb, C, ldc, sc, M, N, K,
                     (int)tm, (int)tn, batch, beta);
  SIMP_HIP(hipGetLastError());
  return SIMP_RT_OK;
}

// fp32 GEMM dispatch on the MFMA path (returns 1 when the operands do not meet
// its requirements, for the caller's SIMT fallback).
template <bool BT>
int dispatch_mfma_f32(const float *A, int64_t lda, int64_t sa, const float *B, int64_t ldb,
                      int64_t sb, float *C, int64_t ldc, int64_t sc, int M, int N, int K, int batch,
                      float beta, hipStream_t st) {
  auto al = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
  const bool ok = K % 4 == 0 && lda % 4 == 0 && sa % 4 == 0 && sb % 4 == 0 && al(A) && al(B) &&
                  (BT ? ldb % 4 == 0 : (N % 4 == 0 && ldb % 4 == 0)) && K > 0;
  if (!ok) return 1;
  const int64_t cus = num_cus();
  auto tiles = [&](int bm, int bn) { return cdiv(M, bm) * cdiv(N, bn) * batch; };
  if (M <= 16)
    return launch_mfma_f32<16, 256, 1, 4, BT>(A, lda, sa, B, ldb, sb, C, ldc, sc, M, N, K, batch, beta, st);
  if (M <= 32)
    return launch_mfma_f32<32, 128, 1, 4, BT>(A, lda, sa, B, ldb, sb, C, ldc, sc, M, N, K, batch, beta, st);
  // Tiles (of all the batch's products) covering the chip, K % 32 == 0, 16-byte
  // C rows: the LDS-DMA ring kernel, the whole of K per workgroup.  Two ring slots (plain
  // double buffering) measured fastest: 4, 6, 8 and 10 slots ran 7-27% slower
  // at the prefill shapes, the deeper prefetch spreading the CUs of an XCD
  // over more operand lines than its L2 keeps.  128x128 tiles on 16 waves
  // from one tile per CU (2048^3: 139.8 us against 157.6 for gemm_f32_mfma;
  // 4096^3: 1074 against 1104), else 64x64 tiles on 8 waves (128x2048x8192 and
  // 512x2048x2048: 42.9 us against 49.9 with split-K and its ordered sum).
  // With K <= 256 (eight K-stages or fewer) four 64x64 workgroups per CU
  // overlap each other's short K loops: 32 x (512x128x512) 25.1 us against
  // 28.9 on 128x128 tiles (28.1 for gemm_f32_mfma), 8 x (1024x256x1024) 42.5
  // against 44.2; from K = 512 on the 128x128 tiles stay ahead.  From two
  // 256x128 tiles per CU, 8 waves of 128x32 (half the operand bytes per flop
  // of the 128x128 tiles): 4096^3 1028 us against 1077, 4096x1024x4096 270
  // against 281, 8192x2048x8192 2078 against 2168 (128x256 tiles: 1038, 270,
  // 2096; 64x64 waves: 1039 at 4096^3; three ring slots: 1056).
  const bool ring_ok = K % 32 == 0 && N % 4 == 0 && ldc % 4 == 0 && sc % 4 == 0 && al(C);
  if (ring_ok && K <= 256 && tiles(64, 64) >= cus)
    return launch_ring_f32<64, 64, 2, 4, 2, BT>(A, lda, sa, B, ldb, sb, C, ldc, sc, M, N, K,
                                                batch, beta, 4, st);
  if (ring_ok && tiles(256, 128) >= 2 * cus)
    return launch_ring_f32<256, 128, 2, 4, 2, BT>(A, lda, sa, B, ldb, sb, C, ldc, sc, M, N, K,
                                                  batch, beta, 1, st);
  if (ring_ok && tiles(128, 128) >= cus)
    return launch_ring_f32<128, 128, 4, 4, 2, BT>(A, lda, sa, B, ldb, sb, C, ldc, sc, M, N, K,
                                                  batch, beta, 1, st);
  if (ring_ok && tiles(64, 64) >= cus)
    return launch_ring_f32<64, 64, 2, 4, 2, BT>(A, lda, sa, B, ldb, sb, C, ldc, sc, M, N, K,
                                                batch, beta, 2, st);
  if (tiles(128, 128) >= cus)
    return launch_mfma_f32<128, 128, 2, 2, BT, 32>(A, lda, sa, B, ldb, sb, C, ldc, sc, M, N, K, batch, beta, st);
  return launch_mfma_f32<64, 64, 2, 2, BT>(A, lda, sa, B, ldb, sb, C, ldc, sc, M, N, K, batch, beta, st);
}

// Batched launch of gemm_t: `batch` products, operand bases `sa`/`sb`/`sc`
// elements apart.  The batch goes on grid z in chunks of at most 65535.
template <typename T, bool BT>
int launch_gemm_t(const T *A, int64_t lda, int64_t sa, const T *B, int64_t ldb, int64_t sb, T *C,
                  int64_t ldc, int64_t sc, int M, int N, int K, int64_t batch, T beta,
                  hipStream_t st) {
  if (M == 0 || N == 0 || batch == 0) return SIMP_RT_OK;
  if constexpr (std::is_same<T, float>::value) {
    if (batch <= 65535) {
      const int rc = dispatch_mfma_f32<BT>(A, lda, sa, B, ldb, sb, C, ldc, sc, M, N, K, (int)batch,
                                           beta, st);
      if (rc != 1) return rc;
    }
  }
  const int64_t tiles_n = cdiv(N, 64), tiles = cdiv(M, 64) * tiles_n;
  if (tiles > INT32_MAX)
    return set_error(SIMP_RT_EUNSUPPORTED, "gemm: %lld output tiles exceed one launch",
                     (long long)tiles);
  for (int64_t b0 = 0; b0 < batch; b0 += 65535) {
    const unsigned nb = (unsigned)std::min<int64_t>(65535, batch - b0);
    hipLaunchKernelGGL((gemm_t<T, BT>), dim3((unsigned)tiles, 1, nb), dim3(256), 0, st,
                       A + b0 * sa, lda, sa, B + b0 * sb, ldb, sb, C + b0 * sc, ldc, sc, M, N, K,
                       (int)tiles_n, beta);
    SIMP_HIP(hipGetLastError());
  }
  return SIMP_RT_OK;
}

// y[0..rows) = beta*y + W x: W rows of lda floats, x and y contiguous.
int launch_gemv_f32(const float *W, int64_t lda, const float *x, float *y, int rows, int K,
                    float beta, hipStream_t st) {
  const bool vec = K % 4 == 0 && lda % 4 == 0 && ((uintptr_t)W & 15) == 0 &&
                   ((uintptr_t)x & 15) == 0;
  const int blocks_cap = num_cus() * 4;
  const unsigned grid = (unsigned)std::min<int64_t>(cdiv(rows, 4), blocks_cap);
  if (vec && K > 0 && K <= 256 * 16) {
    const int J = (int)cdiv(K, 256);
#define GEMV_CASE(JJ) \
  case JJ: hipLaunchKernelGGL(gemv_f32<JJ>, dim3(grid), dim3(256), 0, st, W, lda, x, y, rows, K, beta); break;
    switch (J) {
      GEMV_CASE(1) GEMV_CASE(2) GEMV_CASE(3) GEMV_CASE(4) GEMV_CASE(5) GEMV_CASE(6)
      GEMV_CASE(7) GEMV_CASE(8) GEMV_CASE(9) GEMV_CASE(10) GEMV_CASE(11) GEMV_CASE(12)
      GEMV_CASE(13) GEMV_CASE(14) GEMV_CASE(15) GEMV_CASE(16)
      default: break;
    }
#undef GEMV_CASE
  } else {
    hipLaunchKernelGGL(gemv_f32_any, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, st, W, lda, x, y,
                       rows, K, beta);
  }
  SIMP_HIP(hipGetLastError());
  return SIMP_RT_OK;
}

}  // namespace

int launch_matmul_f32(const float *A, int64_t lda, const float *B, int64_t ldb, float *C,
                      int64_t ldc, int M, int N, int K, float beta, hipStream_t st) {
  if (M == 0 || N == 0) return SIMP_RT_OK;
  // column vector operand (B[k*ldb], ldb == 1) and a contiguous C column: GEMV
  if (N == 1 && ldb == 1 && ldc == 1) return launch_gemv_f32(A, lda, B, C, M, K, beta, st);
  return launch_gemm_t<float, false>(A, lda, 0, B, ldb, 0, C, ldc, 0, M, N, K, 1, beta, st);
}

namespace {
// C = A * B_T^T (fresh C): a single row of A against B_T[N,K] is a GEMV over the
// rows of B_T.
int launch_matmul_nt_f32(const float *A, int64_t lda, const float *BT, int64_t ldb, float *C,
                         int64_t ldc, int M, int N, int K, hipStream_t st) {
  if (M == 0 || N == 0) return SIMP_RT_OK;
  if (M == 1) return launch_gemv_f32(BT, ldb, A, C, N, K, 0.f, st);
  return launch_gemm_t<float, true>(A, lda, 0, BT, ldb, 0, C, ldc, 0, M, N, K, 1, 0.f, st);
}
}  // namespace

}  // namespace simp

namespace simp {
namespace {
// Shared body of the rank-2 fp32 entry points: C[M,N] = A[M,K] x B (B[K,N], or
// B_T[N,K] when BT), C overwritten.
template <bool BT>
int tensor_f32_entry(const char *name, const float *a_alloc, const float *a, int64_t a_off,
                     int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
                     const float *b_alloc, const float *b, int64_t b_off, int64_t b_s0,
                     int64_t b_s1, int64_t b_st0, int64_t b_st1, float *c_alloc, float *c,
                     int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1) {
  (void)a_alloc; (void)b_alloc; (void)c_alloc;
  int rc;
  if ((rc = check_desc2("A", a, a_off, a_s0, a_s1, a_st0, a_st1))) return rc;
  if ((rc = check_desc2("B", b, b_off, b_s0, b_s1, b_st0, b_st1))) return rc;
  if ((rc = check_desc2("C", c, c_off, c_s0, c_s1, c_st0, c_st1))) return rc;
  const int64_t M = a_s0, K = a_s1, N = BT ? b_s0 : b_s1;
  const int64_t Kb = BT ? b_s1 : b_s0;
  if (Kb != K || c_s0 != M || c_s1 != N)
    return set_error(SIMP_RT_EINVAL, "%s: shape mismatch A[%lld,%lld] B%s[%lld,%lld] C[%lld,%lld]",
                     name, (long long)a_s0, (long long)a_s1, BT ? "_T" : "", (long long)b_s0,
                     (long long)b_s1, (long long)c_s0, (long long)c_s1);
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return set_error(SIMP_RT_EUNSUPPORTED, "%s: dimension above 2^31-1", name);
  if (M == 0 || N == 0) return SIMP_RT_OK;
  Operand oa, ob, oc;
  const size_t ab = K ? 4 * (size_t)((M - 1) * a_st0 + K) : 0;
  const size_t bb = (b_s0 && b_s1) ? 4 * (size_t)((b_s0 - 1) * b_st0 + b_s1) : 0;
  const size_t cb = 4 * (size_t)((M - 1) * c_st0 + N);
  if ((rc = oa.bind(a + a_off, ab, Operand::kIn, "A"))) return rc;
  if ((rc = ob.bind(b + b_off, bb, Operand::kIn, "B"))) return rc;
  if ((rc = oc.bind(c + c_off, cb, Operand::kOut, "C"))) return rc;
  if constexpr (BT)
    rc = launch_matmul_nt_f32((const float *)oa.dev(), a_st0, (const float *)ob.dev(), b_st0,
                              (float *)oc.dev(), c_st0, (int)M, (int)N, (int)K, cur_stream());
  else
    rc = launch_matmul_f32((const float *)oa.dev(), a_st0, (const float *)ob.dev(), b_st0,
                           (float *)oc.dev(), c_st0, (int)M, (int)N, (int)K, 0.f, cur_stream());
  if (rc) return rc;
  Operand *ops[] = {&oa, &ob, &oc};
  return finish(ops, 3);
}

// Shared body of the rank-3 entry points: C[b] = A[b] x B[b] for every batch b,
// A[Bt,M,K], B[Bt,K,N], C[Bt,M,N], C overwritten (linalg.batch_matmul into a
// zero-filled result, ConvertSimpToMemRef.cpp:2926-2933,3286-3291).
template <typename T>
int batch_entry(const char *name, const T *a, int64_t a_off, const int64_t *as, const int64_t *ast,
                const T *b, int64_t b_off, const int64_t *bs, const int64_t *bst, T *c,
                int64_t c_off, const int64_t *cs, const int64_t *cst) {
  int rc;
  int64_t an, bn, cn;
  if ((rc = check_descn("A", a, a_off, 3, as, ast, &an))) return rc;
  if ((rc = check_descn("B", b, b_off, 3, bs, bst, &bn))) return rc;
  if ((rc = check_descn("C", c, c_off, 3, cs, cst, &cn))) return rc;
  const int64_t Bt = as[0], M = as[1], K = as[2], N = bs[2];
  if (bs[0] != Bt || bs[1] != K || cs[0] != Bt || cs[1] != M || cs[2] != N)
    return set_error(SIMP_RT_EINVAL,
                     "%s: shape mismatch A[%lld,%lld,%lld] B[%lld,%lld,%lld] C[%lld,%lld,%lld]",
                     name, (long long)as[0], (long long)as[1], (long long)as[2], (long long)bs[0],
                     (long long)bs[1], (long long)bs[2], (long long)cs[0], (long long)cs[1],
                     (long long)cs[2]);
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return set_error(SIMP_RT_EUNSUPPORTED, "%s: dimension above 2^31-1", name);
  if (Bt == 0 || M == 0 || N == 0) return SIMP_RT_OK;
  Operand oa, ob, oc;
  if ((rc = oa.bind(a + a_off, sizeof(T) * (size_t)an, Operand::kIn, "A"))) return rc;
  if ((rc = ob.bind(b + b_off, sizeof(T) * (size_t)bn, Operand::kIn, "B"))) return rc;
  if ((rc = oc.bind(c + c_off, sizeof(T) * (size_t)cn, Operand::kOut, "C"))) return rc;
  const T *da = (const T *)oa.dev(), *db = (const T *)ob.dev();
  T *dc = (T *)oc.dev();
  bool done = false;
  if constexpr (std::is_same<T, float>::value) {
    if (Bt == 1) {  // one product: the rank-2 dispatch (GEMV for a column B)
      rc = launch_matmul_f32(da, ast[1], db, bst[1], dc, cst[1], (int)M, (int)N, (int)K, 0.f,
                             cur_stream());
      done = true;
    }
  }
  if (!done)
    rc = launch_gemm_t<T, false>(da, ast[1], ast[0], db, bst[1], bst[0], dc, cst[1], cst[0],
                                 (int)M, (int)N, (int)K, Bt, T(0), cur_stream());
  if (rc) return rc;
  Operand *ops[] = {&oa, &ob, &oc};
  return finish(ops, 3);
}

// Shared body of the rank-4 entry points: out[n,h,w,:] = W[C_out,C_in] x
// in[n,h,w,:] (ConvertSimpToMemRef.cpp:3293-3361: collapse (N,H,W), multiply by
// the transposed weights, expand back).  The collapse needs the three outer
// dimensions of `in` and `out` to be one run of rows (stride0 = H*stride1,
// stride1 = W*stride2), as memref.collapse_shape does.
template <typename T>
int nhwc_entry(const char *name, const T *x, int64_t x_off, const int64_t *xs, const int64_t *xst,
               const T *w, int64_t w_off, int64_t w_s0, int64_t w_s1, int64_t w_st0,
               int64_t w_st1, T *y, int64_t y_off, const int64_t *ys, const int64_t *yst) {
  int rc;
  int64_t xn, yn;
  if ((rc = check_descn("input", x, x_off, 4, xs, xst, &xn))) return rc;
  if ((rc = check_desc2("weights", w, w_off, w_s0, w_s1, w_st0, w_st1))) return rc;
  if ((rc = check_descn("output", y, y_off, 4, ys, yst, &yn))) return rc;
  const int64_t Cin = xs[3], Cout = w_s0;
  if (w_s1 != Cin || ys[0] != xs[0] || ys[1] != xs[1] || ys[2] != xs[2] || ys[3] != Cout)
    return set_error(SIMP_RT_EINVAL,
                     "%s: shape mismatch input[%lld,%lld,%lld,%lld] weights[%lld,%lld] "
                     "output[%lld,%lld,%lld,%lld]",
                     name, (long long)xs[0], (long long)xs[1], (long long)xs[2], (long long)xs[3],
                     (long long)w_s0, (long long)w_s1, (long long)ys[0], (long long)ys[1],
                     (long long)ys[2], (long long)ys[3]);
  const int64_t rows = xs[0] * xs[1] * xs[2];
  if (rows == 0 || Cout == 0) return SIMP_RT_OK;
  auto collapsible = [](const int64_t *sz, const int64_t *st) {
    return (sz[0] == 1 || st[0] == sz[1] * st[1]) && (sz[1] == 1 || st[1] == sz[2] * st[2]);
  };
  if (!collapsible(xs, xst) || !collapsible(ys, yst))
    return set_error(SIMP_RT_EINVAL, "%s: (N,H,W) of input/output do not collapse to one row run",
                     name);
  if (rows > INT32_MAX || Cout > INT32_MAX || Cin > INT32_MAX)
    return set_error(SIMP_RT_EUNSUPPORTED, "%s: dimension above 2^31-1", name);
  Operand ox, ow, oy;
  const size_t wn = Cin ? (size_t)((w_s0 - 1) * w_st0 + w_s1) : 0;
  if ((rc = ox.bind(x + x_off, sizeof(T) * (size_t)xn, Operand::kIn, "input"))) return rc;
  if ((rc = ow.bind(w + w_off, sizeof(T) * wn, Operand::kIn, "weights"))) return rc;
  if ((rc = oy.bind(y + y_off, sizeof(T) * (size_t)yn, Operand::kOut, "output"))) return rc;
  // collapsed row pitch: the W-dimension stride (N, H and W step in whole rows)
  const T *dx = (const T *)ox.dev(), *dw = (const T *)ow.dev();
  T *dy = (T *)oy.dev();
  if constexpr (std::is_same<T, float>::value)
    rc = launch_matmul_nt_f32(dx, xst[2], dw, w_st0, dy, yst[2], (int)rows, (int)Cout, (int)Cin,
                              cur_stream());
  else
    rc = launch_gemm_t<T, true>(dx, xst[2], 0, dw, w_st0, 0, dy, yst[2], 0, (int)rows, (int)Cout,
                                (int)Cin, 1, T(0), cur_stream());
  if (rc) return rc;
  Operand *ops[] = {&ox, &ow, &oy};
  return finish(ops, 3);
}

// tensor_matmul on f64 tensors (the general linalg.matmul branch, :3280-3284).
int f64_entry(const double *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0,
              int64_t a_st1, const double *b, int64_t b_off, int64_t b_s0, int64_t b_s1,
              int64_t b_st0, int64_t b_st1, double *c, int64_t c_off, int64_t c_s0, int64_t c_s1,
              int64_t c_st0, int64_t c_st1) {
  const int64_t as[3] = {1, a_s0, a_s1}, ast[3] = {a_s0 * a_st0, a_st0, a_st1};
  const int64_t bs[3] = {1, b_s0, b_s1}, bst[3] = {b_s0 * b_st0, b_st0, b_st1};
  const int64_t cs[3] = {1, c_s0, c_s1}, cst[3] = {c_s0 * c_st0, c_st0, c_st1};
  return batch_entry<double>("tensor_matmul_f64", a, a_off, as, ast, b, b_off, bs, bst, c, c_off,
                             cs, cst);
}
}  // namespace
}  // namespace simp

using namespace simp;

extern "C" {

int32_t simp_rt_matmul_f32(const float *a_alloc, const float *lhs, int64_t a_doff, int64_t a_size,
                           int64_t a_stride, const float *b_alloc, const float *rhs,
                           int64_t b_doff, int64_t b_size, int64_t b_stride, float *c_alloc,
                           float *out, int64_t c_doff, int64_t c_size, int64_t c_stride, int64_t m,
                           int64_t k, int64_t n, int64_t lhs_offset, int64_t rhs_offset,
                           int64_t out_offset) {
  (void)a_alloc; (void)b_alloc; (void)c_alloc;
  int rc;
  if ((rc = check_desc1("lhs", lhs, a_doff, a_size, a_stride))) return rc;
  if ((rc = check_desc1("rhs", rhs, b_doff, b_size, b_stride))) return rc;
  if ((rc = check_desc1("output", out, c_doff, c_size, c_stride))) return rc;
  if (m < 0 || k < 0 || n < 0 || lhs_offset < 0 || rhs_offset < 0 || out_offset < 0 ||
      lhs_offset + m * k > a_size || rhs_offset + k * n > b_size || out_offset + m * n > c_size)
    return set_error(SIMP_RT_EINVAL, "matmul: m=%lld k=%lld n=%lld with offsets exceeds arrays",
                     (long long)m, (long long)k, (long long)n);
  if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX)
    return set_error(SIMP_RT_EUNSUPPORTED, "matmul: dimension above 2^31-1");
  if (m == 0 || n == 0) return SIMP_RT_OK;
  Operand oa, ob, oc;
  if ((rc = oa.bind(lhs + a_doff + lhs_offset, 4 * (size_t)(m * k), Operand::kIn, "lhs"))) return rc;
  if ((rc = ob.bind(rhs + b_doff + rhs_offset, 4 * (size_t)(k * n), Operand::kIn, "rhs"))) return rc;
  if ((rc = oc.bind(out + c_doff + out_offset, 4 * (size_t)(m * n), Operand::kInOut, "output"))) return rc;
  if ((rc = launch_matmul_f32((const float *)oa.dev(), k, (const float *)ob.dev(), n,
                              (float *)oc.dev(), n, (int)m, (int)n, (int)k, 1.f, cur_stream())))
    return rc;
  Operand *ops[] = {&oa, &ob, &oc};
  return finish(ops, 3);
}

int32_t simp_rt_tensor_matmul_f32(
    const float *a_alloc, const float *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const float *b_alloc, const float *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_st0, int64_t b_st1,
    float *c_alloc, float *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1) {
  return tensor_f32_entry<false>("tensor_matmul_f32", a_alloc, a, a_off, a_s0, a_s1, a_st0, a_st1,
                                 b_alloc, b, b_off, b_s0, b_s1, b_st0, b_st1, c_alloc, c, c_off,
                                 c_s0, c_s1, c_st0, c_st1);
}

int32_t simp_rt_tensor_matmul_nt_f32(
    const float *a_alloc, const float *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const float *bt_alloc, const float *bt, int64_t bt_off, int64_t bt_s0, int64_t bt_s1, int64_t bt_st0, int64_t bt_st1,
    float *c_alloc, float *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1) {
  return tensor_f32_entry<true>("tensor_matmul_nt_f32", a_alloc, a, a_off, a_s0, a_s1, a_st0,
                                a_st1, bt_alloc, bt, bt_off, bt_s0, bt_s1, bt_st0, bt_st1, c_alloc,
                                c, c_off, c_s0, c_s1, c_st0, c_st1);
}

int32_t simp_rt_tensor_matvecmul_f32(
    const float *a_alloc, const float *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const float *b_alloc, const float *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_st0, int64_t b_st1,
    float *c_alloc, float *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1) {
  return tensor_f32_entry<false>("tensor_matvecmul_f32", a_alloc, a, a_off, a_s0, a_s1, a_st0,
                                 a_st1, b_alloc, b, b_off, b_s0, b_s1, b_st0, b_st1, c_alloc, c,
                                 c_off, c_s0, c_s1, c_st0, c_st1);
}

int32_t simp_rt_tensor_batch_matmul_f32(
    const float *a_alloc, const float *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_s2,
    int64_t a_st0, int64_t a_st1, int64_t a_st2,
    const float *b_alloc, const float *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_s2,
    int64_t b_st0, int64_t b_st1, int64_t b_st2,
    float *c_alloc, float *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_s2,
    int64_t c_st0, int64_t c_st1, int64_t c_st2) {
  (void)a_alloc; (void)b_alloc; (void)c_alloc;
  const int64_t as[3] = {a_s0, a_s1, a_s2}, ast[3] = {a_st0, a_st1, a_st2};
  const int64_t bs[3] = {b_s0, b_s1, b_s2}, bst[3] = {b_st0, b_st1, b_st2};
  const int64_t cs[3] = {c_s0, c_s1, c_s2}, cst[3] = {c_st0, c_st1, c_st2};
  return batch_entry<float>("tensor_batch_matmul_f32", a, a_off, as, ast, b, b_off, bs, bst, c,
                            c_off, cs, cst);
}

int32_t simp_rt_tensor_batch_matmul_f64(
    const double *a_alloc, const double *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_s2,
    int64_t a_st0, int64_t a_st1, int64_t a_st2,
    const double *b_alloc, const double *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_s2,
    int64_t b_st0, int64_t b_st1, int64_t b_st2,
    double *c_alloc, double *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_s2,
    int64_t c_st0, int64_t c_st1, int64_t c_st2) {
  (void)a_alloc; (void)b_alloc; (void)c_alloc;
  const int64_t as[3] = {a_s0, a_s1, a_s2}, ast[3] = {a_st0, a_st1, a_st2};
  const int64_t bs[3] = {b_s0, b_s1, b_s2}, bst[3] = {b_st0, b_st1, b_st2};
  const int64_t cs[3] = {c_s0, c_s1, c_s2}, cst[3] = {c_st0, c_st1, c_st2};
  return batch_entry<double>("tensor_batch_matmul_f64", a, a_off, as, ast, b, b_off, bs, bst, c,
                             c_off, cs, cst);
}

int32_t simp_rt_tensor_matmul_f64(
    const double *a_alloc, const double *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const double *b_alloc, const double *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_st0, int64_t b_st1,
    double *c_alloc, double *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1) {
  (void)a_alloc; (void)b_alloc; (void)c_alloc;
  return f64_entry(a, a_off, a_s0, a_s1, a_st0, a_st1, b, b_off, b_s0, b_s1, b_st0, b_st1, c,
                   c_off, c_s0, c_s1, c_st0, c_st1);
}

int32_t simp_rt_tensor_matmul_nhwc_f32(
    const float *x_alloc, const float *x, int64_t x_off, int64_t x_s0, int64_t x_s1, int64_t x_s2,
    int64_t x_s3, int64_t x_st0, int64_t x_st1, int64_t x_st2, int64_t x_st3,
    const float *w_alloc, const float *w, int64_t w_off, int64_t w_s0, int64_t w_s1, int64_t w_st0,
    int64_t w_st1,
    float *y_alloc, float *y, int64_t y_off, int64_t y_s0, int64_t y_s1, int64_t y_s2,
    int64_t y_s3, int64_t y_st0, int64_t y_st1, int64_t y_st2, int64_t y_st3) {
  (void)x_alloc; (void)w_alloc; (void)y_alloc;
  const int64_t xs[4] = {x_s0, x_s1, x_s2, x_s3}, xst[4] = {x_st0, x_st1, x_st2, x_st3};
  const int64_t ys[4] = {y_s0, y_s1, y_s2, y_s3}, yst[4] = {y_st0, y_st1, y_st2, y_st3};
  return nhwc_entry<float>("tensor_matmul_nhwc_f32", x, x_off, xs, xst, w, w_off, w_s0, w_s1,
                           w_st0, w_st1, y, y_off, ys, yst);
}

int32_t simp_rt_tensor_matmul_nhwc_f64(
    const double *x_alloc, const double *x, int64_t x_off, int64_t x_s0, int64_t x_s1, int64_t x_s2,
    int64_t x_s3, int64_t x_st0, int64_t x_st1, int64_t x_st2, int64_t x_st3,
    const double *w_alloc, const double *w, int64_t w_off, int64_t w_s0, int64_t w_s1, int64_t w_st0,
    int64_t w_st1,
    double *y_alloc, double *y, int64_t y_off, int64_t y_s0, int64_t y_s1, int64_t y_s2,
    int64_t y_s3, int64_t y_st0, int64_t y_st1, int64_t y_st2, int64_t y_st3) {
  (void)x_alloc; (void)w_alloc; (void)y_alloc;
  const int64_t xs[4] = {x_s0, x_s1, x_s2, x_s3}, xst[4] = {x_st0, x_st1, x_st2, x_st3};
  const int64_t ys[4] = {y_s0, y_s1, y_s2, y_s3}, yst[4] = {y_st0, y_st1, y_st2, y_st3};
  return nhwc_entry<double>("tensor_matmul_nhwc_f64", x, x_off, xs, xst, w, w_off, w_s0, w_s1,
                            w_st0, w_st1, y, y_off, ys, yst);
}

}  // extern "C"
