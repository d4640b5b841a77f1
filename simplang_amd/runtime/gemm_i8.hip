// gemm_i8.hip -- exact int8 GEMM on CDNA4 int8 MFMA.
//
// Semantics replaced (citations into the SimpLang tree):
//   s8 x s8 -> i32  tensor_matmul i8 branch, ConvertSimpToMemRef.cpp:3136-3279
//                   (both operands sign-extended, :3233-3239), rewritten onto
//                   vpdpbusd by VNNIPass.cpp:597-999 (A^0x80 and a 128*colsum(B)
//                   bias correction, :817-830,899-906).  MFMA multiplies s8 x s8
//                   natively, so this path needs no correction at all.
//   u8 x s8 -> i32  raw vpdpbusd (simptensor/tests/test_vnni_correctness.cpp:28-42).
//                   MFMA has no u8 x s8 form: A is flipped to A^0x80 = A-128 as s8
//                   and C = MFMA(A^0x80, B) + 128*colsum(B)[j].
// Integer sums are order independent, so every tiling / split-K choice is
// bit-exact with the reference's sequential K loop.
//
// Kernels, by problem size (dispatch<> picks one):
//   * gemm_i8_dma -- problems of at least one 256x256 tile per CU, K % 64 == 0:
//     persistent, global -> LDS DMA ring, v_mfma_i32_16x16x64_i8, 16-byte
//     nontemporal C stores.  B given as [K,N] with 16-byte aligned rows is
//     read in place and transposed by the LDS reads (ds_read_b64_tr_b8);
//     B_T[N,K] inputs are read as rows.  The u8 column sums come from the
//     kernel's own B fragments on the MFMA pipe.  A [K,N] B the in-place read
//     cannot serve is first transposed into a workspace B_T (transpose_i8,
//     which forms the column sums on the way), as the reference materialises
//     B_T (ConvertSimpToMemRef.cpp:3168-3216).
//   * gemm_i8_nt16 -- the same tile sizes for K % 64 != 0 (K % 16 == 0), LDS
//     double-buffered through registers, on B_T.
//   * gemm_i8_mfma -- smaller problems and batches (grid z): BMxBN tiles on
//     v_mfma_i32_32x32x32_i8, K walked in double-buffered LDS tiles; B given as
//     [K,N] is transposed on the way into LDS (4x4 byte blocks with v_perm_b32);
//     the u8 column sums come from the B fragments in registers (v_dot4
//     against 0x01010101).  Skinny problems split K over grid y and combine
//     partial tiles with integer atomics into a zero-filled C (exact).
//   * gemm_i8_generic -- operands the MFMA kernels cannot load with aligned
//     vector loads (K % 16 != 0, N % 4 != 0 for B[K,N], misaligned bases): one
//     output element per thread.
// Workgroup ids are remapped so that each of the 8 XCDs owns a contiguous range
// of tiles (blocks are dispatched round-robin over XCDs), and tiles are ordered
// in groups of 8 tile-rows so co-resident tiles share A and B in L2.
#include <algorithm>
#include <type_traits>
#include <mutex>
#include <vector>

#include "rt_device.h"
#include "rt_internal.h"

namespace simp {
namespace {

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// Row swizzle for chunk-major tiles loaded row-wise (A, and B_T): within a
// wave's store, lanes cover 8 chunks of 2 rows; h(kc) = kc ^ (kc << 1) keeps
// both 8-lane and 16-lane groups on distinct 16-byte bank slots.
__device__ __forceinline__ int swz_rows(int r, int kc) { return r ^ ((kc ^ (kc << 1)) & 15); }
// Swizzle for B transposed in registers: a store instruction covers columns
// n = 4*lane + j; n ^ ((n >> 2) & 15) spreads them over distinct slots.
__device__ __forceinline__ int swz_tr(int n) { return n ^ ((n >> 2) & 15); }

// 4x4 byte transpose: d_r holds bytes (r, 0..3); o_j gets bytes (0..3, j).
__device__ __forceinline__ void transpose4x4(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3,
                                             uint32_t &o0, uint32_t &o1, uint32_t &o2,
                                             uint32_t &o3) {
  uint32_t x0 = __builtin_amdgcn_perm(d1, d0, 0x05010400u);  // a0 b0 a1 b1
  uint32_t x1 = __builtin_amdgcn_perm(d1, d0, 0x07030602u);  // a2 b2 a3 b3
  uint32_t y0 = __builtin_amdgcn_perm(d3, d2, 0x05010400u);  // c0 e0 c1 e1
  uint32_t y1 = __builtin_amdgcn_perm(d3, d2, 0x07030602u);  // c2 e2 c3 e3
  o0 = __builtin_amdgcn_perm(y0, x0, 0x05040100u);           // a0 b0 c0 e0
  o1 = __builtin_amdgcn_perm(y0, x0, 0x07060302u);           // a1 b1 c1 e1
  o2 = __builtin_amdgcn_perm(y1, x1, 0x05040100u);
  o3 = __builtin_amdgcn_perm(y1, x1, 0x07060302u);
}

template <int BM, int BN, int BK, int WGM, int WGN, bool BNK, bool AU8, bool ATOMIC>
__global__ void __launch_bounds__(WGM *WGN * 64)
    gemm_i8_mfma(const int8_t *__restrict__ A, int64_t lda, const int8_t *__restrict__ B,
                 int64_t ldb, int32_t *__restrict__ C, int64_t ldc, int M, int N, int K,
                 int tiles_m, int tiles_n, int k_span, int64_t sa, int64_t sb, int64_t sc) {
  constexpr int NT = WGM * WGN * 64;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int FM = WM / 32, FN = WN / 32;
  constexpr int KC = BK / 16;
  static_assert(FM >= 1 && FN >= 1 && WM % 32 == 0 && WN % 32 == 0, "wave tile");
  static_assert(BK % 32 == 0, "K tile");
  constexpr int A_TOT = BM * KC;                           // 16 B chunks of A per tile
  constexpr int A_PER = (A_TOT + NT - 1) / NT;
  constexpr int B_TOT = BNK ? BN * KC : (BK / 16) * (BN / 4);  // chunks or 16x4 units
  constexpr int B_PER = (B_TOT + NT - 1) / NT;

  __shared__ uint4 sA[2][KC * BM];
  __shared__ uint4 sB[2][KC * BN];

  A += blockIdx.z * sa;  // batch z of a batched product (0 strides otherwise)
  B += blockIdx.z * sb;
  C += blockIdx.z * sc;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;
  int tm, tn;
  tile_of_block(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int kbeg = blockIdx.y * k_span;
  const int kend = min(K, kbeg + k_span);
  if (kbeg >= kend) return;  // uniform per workgroup
  const int nk = (kend - kbeg + BK - 1) / BK;

  uint4 ra[A_PER];
  uint4 rbq[BNK ? B_PER : 1];
  uint32_t rbd[BNK ? 1 : B_PER][16];

  auto load_tile = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_PER; i++) {
      const int c = tid + i * NT;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (A_TOT % NT == 0 || c < A_TOT) {
        const int kc = c % KC, m = c / KC;
        const int gm = m0 + m, gk = k0 + kc * 16;
        if (gm < M && gk < kend) v = *(const uint4 *)(A + (int64_t)gm * lda + gk);
      }
      ra[i] = v;
    }
    if constexpr (BNK) {
#pragma unroll
      for (int i = 0; i < B_PER; i++) {
        const int c = tid + i * NT;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (B_TOT % NT == 0 || c < B_TOT) {
          const int kc = c % KC, n = c / KC;
          const int gn = n0 + n, gk = k0 + kc * 16;
          if (gn < N && gk < kend) v = *(const uint4 *)(B + (int64_t)gn * ldb + gk);
        }
        rbq[i] = v;
      }
    } else {
#pragma unroll
      for (int i = 0; i < B_PER; i++) {
        const int u = tid + i * NT;
        const bool on = (B_TOT % NT == 0 || u < B_TOT);
        const int nq = u % (BN / 4), kq = u / (BN / 4);
        const int gn = n0 + nq * 4;
        const int8_t *p = B + (int64_t)(k0 + kq * 16) * ldb + gn;
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int gk = k0 + kq * 16 + r;
          rbd[i][r] = (on && gn < N && gk < kend) ? *(const uint32_t *)(p + (int64_t)r * ldb) : 0u;
        }
      }
    }
  };

  auto store_tile = [&](int s) {
#pragma unroll
    for (int i = 0; i < A_PER; i++) {
      const int c = tid + i * NT;
      if (A_TOT % NT == 0 || c < A_TOT) {
        const int kc = c % KC, m = c / KC;
        uint4 v = ra[i];
        if constexpr (AU8) {
          v.x ^= 0x80808080u; v.y ^= 0x80808080u; v.z ^= 0x80808080u; v.w ^= 0x80808080u;
        }
        sA[s][kc * BM + swz_rows(m, kc)] = v;
      }
    }
    if constexpr (BNK) {
#pragma unroll
      for (int i = 0; i < B_PER; i++) {
        const int c = tid + i * NT;
        if (B_TOT % NT == 0 || c < B_TOT) {
          const int kc = c % KC, n = c / KC;
          sB[s][kc * BN + swz_rows(n, kc)] = rbq[i];
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < B_PER; i++) {
        const int u = tid + i * NT;
        if (B_TOT % NT == 0 || u < B_TOT) {
          const int nq = u % (BN / 4), kq = u / (BN / 4);
          uint32_t o[4][4];  // o[j][q]: column j, K bytes 4q..4q+3
#pragma unroll
          for (int q = 0; q < 4; q++)
            transpose4x4(rbd[i][4 * q], rbd[i][4 * q + 1], rbd[i][4 * q + 2], rbd[i][4 * q + 3],
                         o[0][q], o[1][q], o[2][q], o[3][q]);
#pragma unroll
          for (int j = 0; j < 4; j++)
            sB[s][kq * BN + swz_tr(nq * 4 + j)] = make_uint4(o[j][0], o[j][1], o[j][2], o[j][3]);
        }
      }
    }
  };

  v16i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0;
  int cs[FN];
#pragma unroll
  for (int j = 0; j < FN; j++) cs[j] = 0;

  load_tile(kbeg);
  store_tile(0);
  __syncthreads();

  const int lrow = lane & 31, lk = lane >> 5;
  for (int kt = 0; kt < nk; kt++) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_tile(kbeg + (kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK / 32; ks++) {
      const int kc = ks * 2 + lk;
      v4i af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; i++) {
        const int m = wm0 + i * 32 + lrow;
        uint4 v = sA[cur][kc * BM + swz_rows(m, kc)];
        af[i] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
      }
#pragma unroll
      for (int j = 0; j < FN; j++) {
        const int n = wn0 + j * 32 + lrow;
        uint4 v = sB[cur][kc * BN + (BNK ? swz_rows(n, kc) : swz_tr(n))];
        bf[j] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
        if constexpr (AU8) {
          cs[j] = __builtin_amdgcn_sdot4(bf[j].x, 0x01010101, cs[j], false);
          cs[j] = __builtin_amdgcn_sdot4(bf[j].y, 0x01010101, cs[j], false);
          cs[j] = __builtin_amdgcn_sdot4(bf[j].z, 0x01010101, cs[j], false);
          cs[j] = __builtin_amdgcn_sdot4(bf[j].w, 0x01010101, cs[j], false);
        }
      }
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store_tile(cur ^ 1);
    __syncthreads();
  }

  if constexpr (AU8) {
    // Lanes l and l^32 hold the two K halves of the same column.
#pragma unroll
    for (int j = 0; j < FN; j++) {
      const int tot = cs[j] + __shfl_xor(cs[j], 32);
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][j][r] += 128 * tot;
    }
  }

  // Output of a 32x32 i32 MFMA: lane l holds column l%32, rows 8*(r/4) + 4*(l/32) + r%4.
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++) {
      const int col = n0 + wn0 + j * 32 + lrow;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = m0 + wm0 + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
        if (row < M && col < N) {
          int32_t *dst = C + (int64_t)row * ldc + col;
          if constexpr (ATOMIC) atomicAdd(dst, acc[i][j][r]);
          else *dst = acc[i][j][r];
        }
      }
    }
}

// Large-problem kernel: B given as B_T[N,K] (callers with B[K,N] transpose it
// first into a workspace), v_mfma_i32_16x16x64_i8, 8 waves (2 per SIMD) on a
// 256x256 tile, BK = 128, LDS double-buffered.  All global loads are issued
// unconditionally from clamped (in-bounds) addresses and zeroed when out of
// range, so each K iteration is one basic block the scheduler can interleave.
// Two waves per SIMD hide the LDS and barrier latency of one behind the MFMAs
// of the other; the 16x16x64 shape sustains a higher int8 rate on random data
// than 32x32x32 on MI355X.
template <int BM, int BN, int BK, int WGM, int WGN, bool AU8>
__global__ void __launch_bounds__(WGM *WGN * 64)
    gemm_i8_nt16(const int8_t *__restrict__ A, int64_t lda, const int8_t *__restrict__ B,
                 int64_t ldb, int32_t *__restrict__ C, int64_t ldc, int M, int N, int K,
                 int tiles_m, int tiles_n, const int32_t *__restrict__ colsum) {
  constexpr int NT = WGM * WGN * 64;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int FM = WM / 16, FN = WN / 16;
  constexpr int KC = BK / 16;
  constexpr int A_PER = BM * KC / NT, B_PER = BN * KC / NT;
  static_assert(BM * KC % NT == 0 && BN * KC % NT == 0, "tile/threads");
  static_assert(BK % 64 == 0 && WM % 16 == 0 && WN % 16 == 0, "tile");
  __shared__ uint4 sA[2][KC * BM];
  __shared__ uint4 sB[2][KC * BN];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;
  int tm, tn;
  tile_of_block(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int nk = (K + BK - 1) / BK;
  uint4 ra[A_PER], rb[B_PER];
  // Clamped (always valid) addresses; out-of-range data is zeroed by a mask applied
  // when the tile is written to LDS (recomputed there rather than kept in registers).
  // A branch around the load, or masking right after it, makes the compiler wait for
  // each load in turn.
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_PER; i++) {
      const int c = tid + i * NT, kc = c % KC, m = c / KC;
      ra[i] = *(const uint4 *)(A + (int64_t)min(m0 + m, M - 1) * lda + min(k0 + kc * 16, K - 16));
    }
#pragma unroll
    for (int i = 0; i < B_PER; i++) {
      const int c = tid + i * NT, kc = c % KC, n = c / KC;
      rb[i] = *(const uint4 *)(B + (int64_t)min(n0 + n, N - 1) * ldb + min(k0 + kc * 16, K - 16));
    }
  };
  auto store_tile = [&](int s, int k0) {
#pragma unroll
    for (int i = 0; i < A_PER; i++) {
      const int c = tid + i * NT, kc = c % KC, m = c / KC;
      const uint32_t keep = (m0 + m < M && k0 + kc * 16 < K) ? 0xffffffffu : 0u;
      uint4 v = ra[i];
      v.x &= keep; v.y &= keep; v.z &= keep; v.w &= keep;
      if constexpr (AU8) {
        v.x ^= 0x80808080u; v.y ^= 0x80808080u; v.z ^= 0x80808080u; v.w ^= 0x80808080u;
      }
      sA[s][kc * BM + swz_rows(m, kc)] = v;
    }
#pragma unroll
    for (int i = 0; i < B_PER; i++) {
      const int c = tid + i * NT, kc = c % KC, n = c / KC;
      const uint32_t keep = (n0 + n < N && k0 + kc * 16 < K) ? 0xffffffffu : 0u;
      uint4 v = rb[i];
      v.x &= keep; v.y &= keep; v.z &= keep; v.w &= keep;
      sB[s][kc * BN + swz_rows(n, kc)] = v;
    }
  };
  v4i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++) acc[i][j] = v4i{0, 0, 0, 0};

  load_tile(0);
  store_tile(0, 0);
  __syncthreads();
  const int lr = lane & 15, lk = lane >> 4;
  for (int kt = 0; kt < nk; kt++) {
    const int cur = kt & 1;
    const int knext = min(kt + 1, nk - 1) * BK;  // the last prefetch repeats a tile; never read
    load_tile(knext);
    // keep the next tile's loads at the top of the iteration: left alone, the
    // scheduler sinks them next to the LDS stores and their latency is exposed
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < BK / 64; ks++) {
      const int kc = ks * 4 + lk;  // 16x16x64 operand: lane holds row l%16, K bytes 16*(l/16)..+16
      v4i af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; i++) {
        const uint4 v = sA[cur][kc * BM + swz_rows(wm0 + i * 16 + lr, kc)];
        af[i] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
      }
#pragma unroll
      for (int j = 0; j < FN; j++) {
        const uint4 v = sB[cur][kc * BN + swz_rows(wn0 + j * 16 + lr, kc)];
        bf[j] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
      }
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    // and the masking of those loads at the bottom, so no MFMA above waits for them
    __builtin_amdgcn_sched_barrier(0);
    store_tile(cur ^ 1, knext);
    __syncthreads();
  }
  // Output of a 16x16 i32 MFMA: lane l holds column l%16, rows 4*(l/16) + r.
#pragma unroll
  for (int j = 0; j < FN; j++) {
    const int col = n0 + wn0 + j * 16 + lr;
    // u8 x s8: C = (A^0x80) B + 128 colsum(B)
    const int bias = (AU8 && col < N) ? 128 * colsum[col] : 0;
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int row = m0 + wm0 + i * 16 + 4 * lk + r;
        if (row < M && col < N) C[(int64_t)row * ldc + col] = acc[i][j][r] + bias;
      }
  }
}

// ds_read_b64_tr_b8 at byte offset `off` of the shared array `lds`.
__device__ __forceinline__ v2i lds_read_tr8(const void *lds, uint32_t off) {
  auto *p = (__attribute__((address_space(3))) v2i *)((__attribute__((address_space(3))) char *)(
                (const __attribute__((address_space(3))) char *)lds) + off);
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32(p);
}

// Large-problem kernel for K % 64 == 0, B given as B_T[N,K]: 256x256 C tiles,
// 8 waves (2 per SIMD) of 128x64, v_mfma_i32_16x16x64_i8, BK = 64.
//   * Operand tiles go global -> LDS directly (global_load_lds_dwordx4), with no
//     register staging, into a ring of STAGES 32 KB stages, STAGES-1 K-steps
//     ahead of the MFMAs that consume them; one barrier per K-step.
//   * Per stage, A and B are each 16 blocks of 1 KB = 16 rows x 64 B.  A DMA
//     instruction fills one block in lane order; lane l loads row l/4, 16-byte
//     chunk (l%4)^((row>>1)&3), so four consecutive lanes read one row's 64
//     contiguous bytes (the coalescer merges consecutive lanes only) and the
//     XOR keeps the MFMA operand reads (lane l: row l%16, chunk l/16) at full
//     LDS bandwidth.
//   * Operand fragments are double-buffered in registers: each K-step certifies
//     the next stage (wait + barrier), starts reading its fragments, and runs
//     the MFMAs of the current stage meanwhile.
//   * Persistent: gridDim.x (a multiple of 8) workgroups walk the tiles, so a
//     tile's stores drain while the next tile's loads start.  Virtual block ids
//     keep the XCD-contiguous, row-grouped tile order of tile_of_block.
//   * Rows beyond M (N) load from a clamped in-bounds row; their results are
//     never stored.
//   * The MFMA computes C^T tiles (B fragment as the first operand), so a lane
//     ends with 4 consecutive columns of one row of C: 16-byte nontemporal
//     stores.
//   * B given as [K,N] (BNK false) is read as it lies, with no transpose pass:
//     a stage's B part is 64 k-rows x 256 columns, one DMA instruction = 4
//     k-rows (16 lanes read one row's 256 bytes), and the MFMA's K-contiguous
//     B fragments come from ds_read_b64_tr_b8, which gives lane p of a 16-lane
//     group byte p of the 8 rows of 16 bytes that lanes 2j, 2j+1 address.
//     Column block cb of k-row k sits at block cb ^ (k & 7) ^ 8 ((k >> 4) & 1),
//     so the 32 lanes of a half-wave read 32 distinct 8-byte bank pairs.
//     Columns past N read a clamped in-bounds block; they are never stored.
// Where gemm_i8_dma's u8 x s8 column sums come from (CSM):
constexpr int kColsumPass = 0;  // colsum[], from a pass over B before the kernel
constexpr int kColsumRows = 1;  // the kernel's MFMAs; tiles grouped by tile rows, so a
                                // workgroup forms the sums for every tile
constexpr int kColsumOnce = 2;  // the kernel's MFMAs; tiles grouped by tile columns, so a
                                // workgroup forms them once per column tile it visits
template <int STAGES, bool AU8, bool BNK, int CSM = kColsumPass>
__global__ void __launch_bounds__(512)
    gemm_i8_dma(const int8_t *__restrict__ A, int64_t lda, const int8_t *__restrict__ B,
                int64_t ldb, int32_t *__restrict__ C, int64_t ldc, int M, int N, int K,
                int tiles_m, int tiles_n, const int32_t *__restrict__ colsum, int vec_store) {
  constexpr int BM = 256, BN = 256, BK = 64, WGN = 4;
  constexpr int WM = 128, WN = 64, FM = WM / 16, FN = WN / 16;
  constexpr int STAGE = (BM + BN) * BK;  // bytes
  __shared__ uint4 lds[STAGES * STAGE / 16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;
  const int nk = K / BK;
  const int ntiles = tiles_m * tiles_n;
  const int lrow = lane & 15, lkc = lane >> 4;
  const int drow = lane >> 2, dkc = (lane & 3) ^ ((drow >> 1) & 3);  // DMA lane -> row, chunk
  const int rslot = lrow * 4 + (lkc ^ ((lrow >> 1) & 3));          // operand lane -> slot
  const uint32_t lds_wave = lds_offset(lds) + 2048 * wave;  // wave w fills blocks 2w, 2w+1
  // CS: u8 column sums on the MFMA pipe.  Wave row wy takes its B fragments in
  // the order j ^ jx (jx = 2 wy), so that its fragments 0 and 1, whose column
  // sums it forms, are columns 2 wy and 2 wy + 1 of the wave's four.  The
  // sums stay in cs_lds for the workgroup's next tile of the same columns.
  constexpr bool CS = AU8 && CSM != kColsumPass;
  __shared__ v4i cs_lds[CS ? BN / 4 : 1];
  const int jx = CS ? 2 * (wave / WGN) : 0;
  const v4i ones = v4i{0x01010101, 0x01010101, 0x01010101, 0x01010101};
  int cs_tn = -1;  // column tile whose sums cs_lds holds
  // [K,N] B: lane l reads k-row 16 (l/16) + (l%16)/2 (+8), swizzle of that row
  const uint32_t boff = (16 * lkc + (lrow >> 1)) * 256 + 8 * (lrow & 1);
  const int bsw = (lrow >> 1) ^ ((lkc & 1) << 3);

  for (int vb = blockIdx.x; vb < ntiles; vb += gridDim.x) {
    int tm, tn;
    // kColsumOnce walks the tiles in groups of 8 tile columns instead of rows,
    // so that a workgroup's successive tiles share their columns
    if constexpr (CSM == kColsumOnce) tile_of_block(vb, ntiles, tiles_n, tiles_m, tn, tm);
    else tile_of_block(vb, ntiles, tiles_m, tiles_n, tm, tn);
    const bool form_cs = CS && tn != cs_tn;  // uniform over the workgroup
    const int m0 = tm * BM, n0 = tn * BN;
    const int8_t *srcA0 = A + (int64_t)min(m0 + 32 * wave + drow, M - 1) * lda + 16 * dkc;
    const int8_t *srcA1 = A + (int64_t)min(m0 + 32 * wave + 16 + drow, M - 1) * lda + 16 * dkc;
    const int8_t *srcB0, *srcB1;
    if constexpr (BNK) {
      srcB0 = B + (int64_t)min(n0 + 32 * wave + drow, N - 1) * ldb + 16 * dkc;
      srcB1 = B + (int64_t)min(n0 + 32 * wave + 16 + drow, N - 1) * ldb + 16 * dkc;
    } else {
      // k-rows 8w + 4d + lane/16 (d = 0, 1) of the stage; lane l fills column
      // block slot l%16 with block (l%16) ^ (k & 7) ^ 8 ((k >> 4) & 1)
      const int kr = lane >> 4, sw8 = ((wave >> 1) & 1) << 3;
      const int cb0 = (lane & 15) ^ kr ^ sw8, cb1 = (lane & 15) ^ (4 + kr) ^ sw8;
      srcB0 = B + (int64_t)(8 * wave + kr) * ldb + min(n0 + 16 * cb0, N - 16);
      srcB1 = B + (int64_t)(8 * wave + 4 + kr) * ldb + min(n0 + 16 * cb1, N - 16);
    }
    auto issue = [&](int kt) {
      const uint32_t st = lds_wave + (kt % STAGES) * STAGE;
      const int64_t k0 = (int64_t)kt * BK;
      dma16(srcA0 + k0, st);
      dma16(srcA1 + k0, st + 1024);
      const int64_t kb = BNK ? k0 : k0 * ldb;
      dma16(srcB0 + kb, st + BM * BK);
      dma16(srcB1 + kb, st + BM * BK + 1024);
    };
    v4i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++) acc[i][j] = v4i{0, 0, 0, 0};
    // Fragments: A single-buffered and refilled in place right after its last
    // MFMA of the step; B double-buffered (read at the start of the step).
    v4i fa[FM], fb[2][FN];
    v4i csacc[2] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};
    auto frag = [&](int kt, int blk) {
      const uint4 v = lds[(kt % STAGES) * (STAGE / 16) + blk * 64 + rslot];
      return v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
    };
    constexpr int BOFF = BM * BK / 1024;  // first B block of a stage
    // B fragment j of stage kt: B_T rows (BNK) or two transposing reads of the
    // [k][n] tile, k = 16 (l/16) + 8 t + (l%16)/2, bytes 8 (l & 1) of its block
    auto bfrag = [&](int kt, int j) {
      if constexpr (BNK) {
        return frag(kt, BOFF + wn0 / 16 + (j ^ jx));
      } else {
        const int cb = ((wn0 >> 4) + (j ^ jx)) ^ bsw;
        const uint32_t base = (kt % STAGES) * STAGE + BM * BK + (cb << 4) + boff;
        const v2i lo = lds_read_tr8(lds, base);
        const v2i hi = lds_read_tr8(lds, base + 8 * 256);
        return v4i{lo.x, lo.y, hi.x, hi.y};
      }
    };
    // The previous tile's stores (also counted by vmcnt) drain before this tile's
    // load accounting starts; every wave finished reading LDS at that tile's last
    // barrier, so its stages may be overwritten.
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
#pragma unroll
    for (int p = 0; p < STAGES; p++)
      if (p < nk) issue(p);
    // stage 0 done on this wave (later issued stages may be outstanding) ...
    if (nk >= STAGES) __builtin_amdgcn_s_waitcnt(waitcnt_vm(4 * (STAGES - 1)));
    else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    block_barrier();  // ... and on every wave
#pragma unroll
    for (int j = 0; j < FN; j++) fb[0][j] = bfrag(0, j);
#pragma unroll
    for (int i = 0; i < FM; i++) fa[i] = frag(0, wm0 / 16 + i);
    // K-step kt: certify stage kt+1, refill the buffer of stage kt (its fragments
    // are in registers on every wave) with stage kt+STAGES, and run stage kt's
    // MFMAs while stage kt+1's fragments are read.  The refill is issued after
    // MFMA row 3, not right after the barrier: issued at the barrier, its LDS
    // writes land while every wave reads stage kt+1's B fragments, and the whole
    // kernel at 8192^3 measured 3-4% slower (issuing after any row from 1 to 7
    // is within 1% of row 3).
    // steady (a compile-time flag): stages kt+1 .. kt+STAGES exist, so the
    // step has no branches on nk.  Those branches split the step's schedule,
    // and u8's A flips of a row then wait behind the previous row's MFMAs:
    // u8 8192^3 474-478 us against 480 with them, 8192x4096x8192 262-263
    // against 266.5.  s8 x s8 (no flips) ran 1-2% slower without them, so it
    // keeps them.
    auto step = [&](int kt, int cb, auto steady) {
      constexpr bool S = decltype(steady)::value;
      const bool more = S || kt + 1 < nk;  // stage kt+1 exists
      if (more) {
        // issued: stages up to min(kt+STAGES-1, nk-1); stage kt+1 must be done
        if (S || kt + STAGES - 1 < nk) __builtin_amdgcn_s_waitcnt(waitcnt_vm(4 * (STAGES - 2)));
        else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
      }
      __builtin_amdgcn_s_waitcnt(waitcnt_lgkm0);  // this wave's reads of stage kt landed
      block_barrier();
      if (more) {
#pragma unroll
        for (int j = 0; j < FN; j++) fb[cb ^ 1][j] = bfrag(kt + 1, j);
      }
      // kColsumOnce: the same two MFMAs, on the tiles that form the sums, ahead
      // of the step's main MFMAs (a branch between those split their schedule)
      if constexpr (CS && CSM == kColsumOnce) {
        if (form_cs) {
          csacc[0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fb[cb][0], ones, csacc[0], 0, 0, 0);
          csacc[1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fb[cb][1], ones, csacc[1], 0, 0, 0);
        }
      }
#pragma unroll
      for (int i = 0; i < FM; i++) {
        v4i a = fa[i];
        if constexpr (AU8) a ^= (int)0x80808080;  // u8 a -> s8 (a - 128)
#pragma unroll
        for (int j = 0; j < FN; j++)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fb[cb][j], a, acc[i][j], 0, 0, 0);
        if (more) fa[i] = frag(kt + 1, wm0 / 16 + i);
        if (i == 3 && (S || kt + STAGES < nk)) issue(kt + STAGES);
        // CS: B fragments 0 and 1 also meet an all-ones operand, which leaves
        // every lane the sums of its four output columns of those fragments
        // (two more MFMAs per 32 on every wave)
        if constexpr (CS && CSM == kColsumRows) {
          if (i == 1 || i == 5) {
            const int t = i == 1 ? 0 : 1;
            csacc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fb[cb][t], ones, csacc[t], 0, 0, 0);
          }
        }
      }
    };
    int kt = 0;
    using Steady = std::integral_constant<bool, AU8>;
    for (; kt + 1 + STAGES < nk; kt += 2) {
      step(kt, 0, Steady{});
      step(kt + 1, 1, Steady{});
    }
    for (; kt + 1 < nk; kt += 2) {
      step(kt, 0, std::false_type{});
      step(kt + 1, 1, std::false_type{});
    }
    if (kt < nk) step(kt, 0, std::false_type{});
    if (form_cs) {
      // csacc[t][r] = sum of column wn0 + 16 (t ^ jx) + 4 (l/16) + r; the
      // other wave row of the same columns holds the other two fragments.
      // Every wave read the previous sums in cs_lds before this tile's first
      // barrier.
      if (lrow == 0) {
        cs_lds[(wn0 + 16 * jx) / 4 + lkc] = csacc[0];
        cs_lds[(wn0 + 16 * (1 ^ jx)) / 4 + lkc] = csacc[1];
      }
      __syncthreads();
      cs_tn = tn;
    }
    // acc[i][j][r] = C[m0 + wm0 + 16 i + l%16][n0 + wn0 + 16 (j ^ jx) + 4 (l/16) + r]
#pragma unroll
    for (int j = 0; j < FN; j++) {
      const int col = n0 + wn0 + 16 * (j ^ jx) + 4 * lkc;
      // u8 x s8: C = (A^0x80) B + 128 colsum(B)
      // (N % 16 == 0 and col % 4 == 0, so col < N covers col..col+3)
      v4i bias = v4i{0, 0, 0, 0};
      if constexpr (CS) {
        bias = cs_lds[(wn0 + 16 * (j ^ jx)) / 4 + lkc] * 128;
      } else if constexpr (AU8) {
        if (col < N) bias = *(const v4i *)(colsum + col) * 128;
      }
#pragma unroll
      for (int i = 0; i < FM; i++) {
        const int row = m0 + wm0 + 16 * i + lrow;
        if (row >= M || col >= N) continue;
        const v4i v = acc[i][j] + bias;
        int32_t *dst = C + (int64_t)row * ldc + col;
        if (vec_store) {
          // streaming store: C is not re-read here, and the all-CU store burst
          // at a tile's end drains faster without allocating in L2 (measured
          // 4-5% on the whole kernel at 8192^3)
          __builtin_nontemporal_store(v, (v4i *)dst);
        } else {
#pragma unroll
          for (int r = 0; r < 4; r++)
            if (col + r < N) dst[r] = v[r];
        }
      }
    }
  }
}

// Mid-size kernel (K % 128 == 0): BMxBN tiles (128x128 or 64x64, one per CU at
// 2048^2 / 1024^2 outputs), 4 waves of (BM/2)x(BN/2), v_mfma_i32_16x16x64_i8,
// K-stages of 128 through a ring of SLOTS stages filled by LDS DMA.
//   * A and B_T rows contribute 128 bytes (a whole line) per stage: a DMA
//     instruction is 8 rows x 128 B, lane l row l/8, 16-byte chunk
//     (l%8) ^ ((row >> 1) & 7), which keeps the 16 lanes of an operand read
//     (rows R0..R0+15, one chunk) on 16 distinct 4-bank groups.
//   * B as [K,N] is read in place: a stage's B part is 128 k-rows of BN bytes,
//     turned into K-contiguous fragments by ds_read_b64_tr_b8 (as in
//     gemm_i8_dma), with column block cb of k-row k at cb ^ fB(k), fB chosen
//     per row width so that each half-wave's 32 reads cover the 64 banks.
//   * A stage is two K-steps of 64; fragments are double-buffered in registers
//     and the stage's one barrier sits between its two K-steps (as in the
//     whole-line variant of gemm_i8_dma): this wave's DMAs of stage s+1 are
//     waited for, every wave has read stage s, and stage s+SLOTS is issued into
//     its slot.
//   * u8 x s8: the waves also sum their B fragments (v_dot4 against
//     0x01010101) into column sums, wave row h % WGM taking half-stage h; the
//     rows' partial sums meet in LDS.
template <int BN>
__device__ __forceinline__ int ring_fb(int lrow, int lkc) {
  if constexpr (BN == 256) return (lrow >> 1) ^ ((lkc & 1) << 3);
  else if constexpr (BN == 128) return ((lrow >> 2) & 3) | ((lkc & 1) << 2);
  else return ((lrow >> 3) & 1) | ((lkc & 1) << 1);
}
template <int BN>
__device__ __forceinline__ int ring_fb_row(int k) {  // the same swizzle by k-row
  if constexpr (BN == 256) return (k & 7) ^ (((k >> 4) & 1) << 3);
  else if constexpr (BN == 128) return ((k >> 1) & 3) | (((k >> 4) & 1) << 2);
  else return ((k >> 2) & 1) | (((k >> 4) & 1) << 1);
}

// v_mfma_i32_16x16x64_i8 with the accumulator held in the same VGPRs across
// the K loop (inline asm: the compiler's own allocation renames the
// accumulators between unrolled K-steps, copying them through AGPRs and
// chaining MFMAs through the copies).  The compiler does not insert the wait
// states such an MFMA needs after VALU writes of its sources or before VALU
// reads of its result; the caller places them.
__device__ __forceinline__ void mfma_v(v4i &acc, const v4i &a, const v4i &b) {
  asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
}

template <int BM, int BN, int WGM, int WGN, int SLOTS, bool AU8, bool BNK>
__global__ void __launch_bounds__(64 * WGM * WGN)
    gemm_i8_ring(const int8_t *__restrict__ A, int64_t lda, const int8_t *__restrict__ B,
                 int64_t ldb, int32_t *__restrict__ C, int64_t ldc, int M, int N, int K,
                 int tiles_m, int tiles_n, int vec_store) {
  constexpr int NW = WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN, FM = WM / 16, FN = WN / 16;
  constexpr int BK = 128;
  constexpr int SA = BM * BK, SB = BN * BK, STAGE = SA + SB;  // bytes
  constexpr int DA = SA / 1024 / NW, DB = SB / 1024 / NW;    // DMA instructions per wave
  constexpr int DPW = DA + DB;
  static_assert(DA >= 1 && DB >= 1 && DPW * (SLOTS - 1) <= 63, "ring shape");
  __shared__ uint4 lds[SLOTS * STAGE / 16];
  __shared__ int cs_lds[AU8 ? BN : 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wy = wave / WGN, wx = wave % WGN;
  const int wm0 = wy * WM, wn0 = wx * WN;
  const int ns = K / BK;
  const int ntiles = tiles_m * tiles_n;
  const int lrow = lane & 15, lkc = lane >> 4;
  const uint32_t lds_base = lds_offset(lds);
  const int fa = (lrow >> 1) & 7;   // A / B_T chunk swizzle of this lane's operand rows
  const int fb = ring_fb<BN>(lrow, lkc);
  constexpr int RPI = 1024 / BN, LPR = BN / 16;  // [K,N] B: k-rows per DMA, lanes per k-row

  for (int vb = blockIdx.x; vb < ntiles; vb += gridDim.x) {
    int tm, tn;
    tile_of_block(vb, ntiles, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int8_t *srcA[DA], *srcB[DB];
#pragma unroll
    for (int i = 0; i < DA; i++) {
      const int r = 8 * (wave * DA + i) + (lane >> 3);  // row within the tile
      srcA[i] = A + (int64_t)min(m0 + r, M - 1) * lda + 16 * ((lane & 7) ^ ((r >> 1) & 7));
    }
#pragma unroll
    for (int i = 0; i < DB; i++) {
      if constexpr (BNK) {
        const int r = 8 * (wave * DB + i) + (lane >> 3);
        srcB[i] = B + (int64_t)min(n0 + r, N - 1) * ldb + 16 * ((lane & 7) ^ ((r >> 1) & 7));
      } else {
        const int kr = RPI * (wave * DB + i) + lane / LPR;  // k-row within the stage
        const int cb = (lane % LPR) ^ ring_fb_row<BN>(kr);
        srcB[i] = B + (int64_t)kr * ldb + min(n0 + 16 * cb, N - 16);
      }
    }
    auto issue = [&](int st) {
      const uint32_t dst = lds_base + (uint32_t)(st % SLOTS) * STAGE;
      const int64_t ka = (int64_t)st * BK;
#pragma unroll
      for (int i = 0; i < DA; i++) dma16(srcA[i] + ka, dst + 1024 * (wave * DA + i));
      const int64_t kb = BNK ? ka : ka * ldb;
#pragma unroll
      for (int i = 0; i < DB; i++) dma16(srcB[i] + kb, dst + SA + 1024 * (wave * DB + i));
    };
    auto afrag = [&](int st, int r0, int h) {
      const uint32_t off = (uint32_t)(st % SLOTS) * STAGE + (r0 + lrow) * 128 +
                           (((4 * h + lkc) ^ fa) << 4);
      const uint4 v = lds[off >> 4];
      return v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
    };
    auto bfrag = [&](int st, int c0, int h) {
      if constexpr (BNK) {
        const uint32_t off = (uint32_t)(st % SLOTS) * STAGE + SA + (c0 + lrow) * 128 +
                             (((4 * h + lkc) ^ fa) << 4);
        const uint4 v = lds[off >> 4];
        return v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
      } else {
        const uint32_t off = (uint32_t)(st % SLOTS) * STAGE + SA +
                             (64 * h + 16 * lkc + (lrow >> 1)) * BN +
                             ((((c0 >> 4) ^ fb)) << 4) + 8 * (lrow & 1);
        const v2i lo = lds_read_tr8(lds, off);
        const v2i hi = lds_read_tr8(lds, off + 8 * BN);
        return v4i{lo.x, lo.y, hi.x, hi.y};
      }
    };
    v4i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++) acc[i][j] = v4i{0, 0, 0, 0};
    v4i csacc[AU8 ? FN : 1];  // u8 x s8 column sums (first wave row)
#pragma unroll
    for (int j = 0; j < (AU8 ? FN : 1); j++) csacc[j] = v4i{0, 0, 0, 0};
    const v4i ones = v4i{0x01010101, 0x01010101, 0x01010101, 0x01010101};
    v4i fra[2][FM], frb[2][FN];
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 7");  // VALU writes of the accumulators -> MFMA reads
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // previous tile's stores
    const int first = min(SLOTS, ns);
    for (int st = 0; st < first; st++) issue(st);
    // stage 0 done on this wave (the later stages may be outstanding) ...
    auto wait_after = [&](int n_after) { wait_vm_le<DPW, SLOTS - 1>(n_after); };
    wait_after(first - 1);
    block_barrier();  // ... and on every wave
#pragma unroll
    for (int j = 0; j < FN; j++) frb[0][j] = bfrag(0, wn0 + 16 * j, 0);
#pragma unroll
    for (int i = 0; i < FM; i++) fra[0][i] = afrag(0, wm0 + 16 * i, 0);
    auto mfmas = [&](int cb) {
      v4i a[FM];
#pragma unroll
      for (int i = 0; i < FM; i++) a[i] = AU8 ? (fra[cb][i] ^ (int)0x80808080) : fra[cb][i];
      if constexpr (AU8) {
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_nop 7");  // VALU writes (a ^ 0x80) -> MFMA reads
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) mfma_v(acc[i][j], frb[cb][j], a[i]);
      // u8 x s8: the first wave row also multiplies each B fragment by ones,
      // which leaves every lane the column sums of its four output columns
      // (MFMA work, asynchronous to the wave: the same sums by v_dot4 on the
      // VALU held the other waves at every barrier, 1024^3 6.2 us against 5.4
      // for s8 x s8).  The builtin, not asm: the compiler keeps `ones` in
      // SGPRs and copies it into VGPRs right before each use, a VALU write
      // that only its own hazard tracking separates from the MFMA read.
      if constexpr (AU8) {
        if (wy == 0) {
#pragma unroll
          for (int j = 0; j < FN; j++)
            csacc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(frb[cb][j], ones, csacc[j], 0, 0, 0);
        }
      }
    };
    for (int s = 0; s < ns; s++) {
      // K-step (s,0): read (s,1)'s fragments, run (s,0)
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
      // K-step (s,1): read (s+1,0)'s fragments, run (s,1)
      if (more) {
#pragma unroll
        for (int j = 0; j < FN; j++) frb[0][j] = bfrag(s + 1, wn0 + 16 * j, 0);
#pragma unroll
        for (int i = 0; i < FM; i++) fra[0][i] = afrag(s + 1, wm0 + 16 * i, 0);
      }
      mfmas(1);
    }
    // MFMA results -> VALU reads of the same registers
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 15\n\ts_nop 15" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    // u8 x s8: column sums of this tile's columns, from the first wave row:
    // csacc[j][r] = sum of column wn0 + 16 j + 4 (l/16) + r in every lane
    if constexpr (AU8) {
      if (wy == 0 && lrow == 0) {
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
          for (int r = 0; r < 4; r++) cs_lds[wn0 + 16 * j + 4 * lkc + r] = csacc[j][r];
      }
      __syncthreads();
    }
    // acc[i][j][r] = C[m0 + wm0 + 16 i + l%16][n0 + wn0 + 16 j + 4 (l/16) + r]
#pragma unroll
    for (int j = 0; j < FN; j++) {
      const int cl = wn0 + 16 * j + 4 * lkc, col = n0 + cl;
      v4i bias = v4i{0, 0, 0, 0};
      if constexpr (AU8) {
#pragma unroll
        for (int r = 0; r < 4; r++) bias[r] = cs_lds[cl + r] * 128;
      }
#pragma unroll
      for (int i = 0; i < FM; i++) {
        const int row = m0 + wm0 + 16 * i + lrow;
        if (row >= M || col >= N) continue;
        const v4i v = acc[i][j] + bias;
        int32_t *dst = C + (int64_t)row * ldc + col;
        if (vec_store) {
          *(v4i *)dst = v;
        } else {
#pragma unroll
          for (int r = 0; r < 4; r++)
            if (col + r < N) dst[r] = v[r];
        }
      }
    }
    if constexpr (AU8) __syncthreads();  // cs_lds is rewritten by the next tile
  }
}

// B[K,N] -> B_T[N,K] (K % 16 == 0, N % 16 == 0): a workgroup takes 128
// columns and KT rows of B, through 128x128 LDS tiles.  Reads: 8 lanes per row,
// 16 bytes each, so a wave reads whole 128-byte lines.  Writes: a thread
// transposes four 4x4 byte blocks in registers and stores 16 bytes of each of
// 4 B_T rows; 8 lanes cover 128 contiguous bytes of a row.  The reference
// materialises the same B_T (ConvertSimpToMemRef.cpp:3168-3216).  With
// colsum != nullptr (u8 x s8) each column's sum over the KT rows is added into
// colsum[n], which the caller zero-fills first.
template <int KT>
__global__ void __launch_bounds__(256)
    transpose_i8(const int8_t *__restrict__ B, int64_t ldb, int8_t *__restrict__ BT, int K, int N,
                 int32_t *__restrict__ colsum) {
  constexpr int P = 33;            // LDS row pitch in words (32 words of data)
  __shared__ uint32_t s[128 * P];  // [k][n/4]
  const int t = threadIdx.x;
  const int n0 = blockIdx.x * 128;
  const int k_begin = blockIdx.y * KT, k_end = min(K, k_begin + KT);
  const int rk = t >> 3, rc = t & 7;    // phase 1: rows rk, rk+32, .., 16-byte chunk rc
  const int qn = t >> 3, ko = t & 7;    // phase 2: columns 4qn..+3, rows 16ko..+15
  int sum[4] = {0, 0, 0, 0};
  for (int k0 = k_begin; k0 < k_end; k0 += 128) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int k = rk + 32 * i, gk = k0 + k, gn = n0 + 16 * rc;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (gk < K && gn < N) v = *(const uint4 *)(B + (int64_t)gk * ldb + gn);
      uint32_t *row = s + k * P + 4 * rc;
      row[0] = v.x;
      row[1] = v.y;
      row[2] = v.z;
      row[3] = v.w;
    }
    __syncthreads();
    uint32_t o[4][4];  // o[j][q]: column 4qn+j, rows 16ko+4q..+3
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int k = 16 * ko + 4 * q;
      transpose4x4(s[k * P + qn], s[(k + 1) * P + qn], s[(k + 2) * P + qn], s[(k + 3) * P + qn],
                   o[0][q], o[1][q], o[2][q], o[3][q]);
    }
    const int gk = k0 + 16 * ko;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int gn = n0 + 4 * qn + j;
      if (gn < N && gk < K)
        *(uint4 *)(BT + (int64_t)gn * K + gk) = make_uint4(o[j][0], o[j][1], o[j][2], o[j][3]);
#pragma unroll
      for (int q = 0; q < 4; q++)
        sum[j] = __builtin_amdgcn_sdot4((int)o[j][q], 0x01010101, sum[j], false);
    }
    __syncthreads();
  }
  if (colsum) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      int v = sum[j];
      v += __shfl_xor(v, 1);
      v += __shfl_xor(v, 2);
      v += __shfl_xor(v, 4);
      const int gn = n0 + 4 * qn + j;
      if (ko == 0 && gn < N) atomicAdd(colsum + gn, v);
    }
  }
}

// colsum[n] = sum_k B_T[n,k] as signed bytes, one wave per row (K % 16 == 0,
// 16-byte aligned rows).
__global__ void __launch_bounds__(256)
    colsum_nk_i8(const int8_t *__restrict__ BT, int64_t ldb, int32_t *__restrict__ colsum, int N,
                 int K) {
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (n >= N) return;
  const int8_t *row = BT + (int64_t)n * ldb;
  int acc = 0;
  for (int k = lane * 16; k < K; k += 64 * 16) {
    const uint4 v = *(const uint4 *)(row + k);
    acc = __builtin_amdgcn_sdot4((int)v.x, 0x01010101, acc, false);
    acc = __builtin_amdgcn_sdot4((int)v.y, 0x01010101, acc, false);
    acc = __builtin_amdgcn_sdot4((int)v.z, 0x01010101, acc, false);
    acc = __builtin_amdgcn_sdot4((int)v.w, 0x01010101, acc, false);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
  if (lane == 0) colsum[n] = acc;
}

// Skinny product, M <= MR <= 2 rows of A, B as [K,N] (K % 16 == 0, N % 8 == 0,
// 8-byte aligned rows): a v_dot4_i32_i8 GEMV instead of MFMA tiles.
//   * Workgroup (g, s) takes columns 512 g .. 512 g + 511 and the K band
//     s*k_span .. +k_span; lane l the 8 columns 512 g + 8 l, wave w every 4th
//     quad of k-rows of the band, U quads (4U 8-byte row loads) in flight.  A
//     quad's row pieces are transposed in registers (two 4x4 byte blocks,
//     v_perm) so each column's 4 k-values form one dword: one v_dot4 per column
//     and row of A.  A's 4 bytes of a quad are uniform (scalar loads).
//   * u8 x s8 flips A to A^0x80 = A-128 and adds 128 * colsum(B) over the
//     band, summed here from the same dwords (v_dot4 against 0x01010101).
//   * The 4 waves meet in LDS; with one K band the workgroup stores C, with
//     more it adds its band's sums into a zero-filled C with integer atomics
//     (exact in any order).
// With more rows of A the dot4 work per byte of B grows and the MFMA tiles
// (16 times the MACs per instruction) are faster from M = 3 on (measured).
template <int MR, bool AU8, bool ATOMIC>
__global__ void __launch_bounds__(256)
    gemv_i8_kn(const int8_t *__restrict__ A, int64_t lda, const int8_t *__restrict__ B,
               int64_t ldb, int32_t *__restrict__ C, int64_t ldc, int M, int N, int K,
               int k_span) {
  constexpr int NR = MR + (AU8 ? 1 : 0);  // sums per column: MR products (+ column sum)
  constexpr int U = 8;                    // quads in flight per wave
  constexpr int CW = 512;                 // columns per workgroup
  __shared__ int red[4][NR][CW];
  // wave index made visibly uniform, so A's bytes come through scalar loads
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = blockIdx.x, s = blockIdx.y;
  const int c0 = g * CW + 8 * lane;
  const int kb = s * k_span, ke = min(K, kb + k_span);
  int acc[NR][8];
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int j = 0; j < 8; j++) acc[r][j] = 0;
  const int8_t *bp = B + min(c0, N - 8);  // lanes past N read in-bounds bytes, never stored
  auto quad = [&](int k, const uint2 (&d)[4]) {
    uint32_t o[8];
    transpose4x4(d[0].x, d[1].x, d[2].x, d[3].x, o[0], o[1], o[2], o[3]);
    transpose4x4(d[0].y, d[1].y, d[2].y, d[3].y, o[4], o[5], o[6], o[7]);
#pragma unroll
    for (int m = 0; m < MR; m++) {
      int a4 = 0;
      if (m < M) a4 = *(const int *)(A + (int64_t)m * lda + k);
      if constexpr (AU8) a4 ^= (int)0x80808080;
#pragma unroll
      for (int j = 0; j < 8; j++) acc[m][j] = __builtin_amdgcn_sdot4((int)o[j], a4, acc[m][j], false);
    }
    if constexpr (AU8) {
#pragma unroll
      for (int j = 0; j < 8; j++)
        acc[MR][j] = __builtin_amdgcn_sdot4((int)o[j], 0x01010101, acc[MR][j], false);
    }
  };
  // U quads per round trip; a band's last batch loads clamped rows for the
  // quads past its end and skips them (bands and K are multiples of 16, so a
  // quad is wholly inside or outside)
  for (int k = kb + 4 * wave; k < ke; k += 16 * U) {
    uint2 d[U][4];
#pragma unroll
    for (int u = 0; u < U; u++)
#pragma unroll
      for (int r = 0; r < 4; r++)
        d[u][r] = *(const uint2 *)(bp + (int64_t)min(k + 16 * u + r, K - 1) * ldb);
#pragma unroll
    for (int u = 0; u < U; u++)
      if (k + 16 * u < ke) quad(k + 16 * u, d[u]);
  }
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int j = 0; j < 8; j++) red[wave][r][8 * lane + j] = acc[r][j];
  __syncthreads();
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int col = threadIdx.x + 256 * h, n = g * CW + col;
    if (n >= N) break;
    int t[NR];
#pragma unroll
    for (int r = 0; r < NR; r++)
      t[r] = red[0][r][col] + red[1][r][col] + red[2][r][col] + red[3][r][col];
#pragma unroll
    for (int m = 0; m < MR; m++) {
      if (m >= M) break;
      const int v = AU8 ? t[m] + 128 * t[MR] : t[m];
      if constexpr (ATOMIC) atomicAdd(C + (int64_t)m * ldc + n, v);
      else C[(int64_t)m * ldc + n] = v;
    }
  }
}

// Correctness fallback for shapes the MFMA path cannot load with aligned
// vector loads (K % 16 != 0, N % 4 != 0 for B[K,N], misaligned bases).  Rows
// stride over grid y; z is the batch.
template <bool BNK, bool AU8>
__global__ void __launch_bounds__(256)
    gemm_i8_generic(const int8_t *__restrict__ A, int64_t lda, const int8_t *__restrict__ B,
                    int64_t ldb, int32_t *__restrict__ C, int64_t ldc, int M, int N, int K,
                    int64_t sa, int64_t sb, int64_t sc) {
  A += blockIdx.z * sa;
  B += blockIdx.z * sb;
  C += blockIdx.z * sc;
  const int col = blockIdx.x * 64 + (threadIdx.x & 63);
  if (col >= N) return;
  for (int row = blockIdx.y * 4 + (threadIdx.x >> 6); row < M; row += gridDim.y * 4) {
    uint32_t s = 0;
    for (int k = 0; k < K; k++) {
      const int32_t a = AU8 ? (int32_t)(uint8_t)A[(int64_t)row * lda + k]
                            : (int32_t)A[(int64_t)row * lda + k];
      const int32_t b =
          BNK ? (int32_t)B[(int64_t)col * ldb + k] : (int32_t)B[(int64_t)k * ldb + col];
      s += (uint32_t)(a * b);
    }
    C[(int64_t)row * ldc + col] = (int32_t)s;
  }
}

// C[z][r, c] = 0 for r < M, c < N (z: batch, sc elements apart).
__global__ void __launch_bounds__(256)
    fill_i32_2d(int32_t *__restrict__ C, int64_t ldc, int M, int N, int64_t sc) {
  C += blockIdx.z * sc;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)M * N) return;
  const int64_t r = i / N, c = i - r * N;
  C[r * ldc + c] = 0;
}

struct GemmArgs {
  const int8_t *A;
  int64_t lda;
  const int8_t *B;
  int64_t ldb;
  int32_t *C;
  int64_t ldc;
  int M, N, K;
  int batch = 1;                   // products on grid z (at most 65535)
  int64_t sa = 0, sb = 0, sc = 0;  // element distance between consecutive products
  // Caller-provided device scratch for the column sums and B_T of the large
  // path (the allocation-free entry point); null: the stream's workspace.
  void *scratch = nullptr;
  size_t scratch_bytes = 0;
};

template <int BM, int BN, int BK, int WGM, int WGN, bool BNK, bool AU8>
int launch_mfma(const GemmArgs &g, int splits, hipStream_t st) {
  const int tiles_m = (int)cdiv(g.M, BM), tiles_n = (int)cdiv(g.N, BN);
  const int nkt = (int)cdiv(g.K, BK);
  splits = std::max(1, std::min(splits, nkt));
  const int k_span = (int)cdiv(nkt, splits) * BK;
  splits = (int)cdiv(g.K, k_span);
  dim3 grid(tiles_m * tiles_n, splits, g.batch), block(WGM * WGN * 64);
  KernelTimer kt(st, "gemm_i8_mfma");
  if (splits > 1) {
    const int64_t tot = (int64_t)g.M * g.N;
    hipLaunchKernelGGL(fill_i32_2d, dim3((unsigned)cdiv(tot, 256), 1, g.batch), dim3(256), 0, st,
                       g.C, g.ldc, g.M, g.N, g.sc);
    hipLaunchKernelGGL((gemm_i8_mfma<BM, BN, BK, WGM, WGN, BNK, AU8, true>), grid, block, 0, st,
                       g.A, g.lda, g.B, g.ldb, g.C, g.ldc, g.M, g.N, g.K, tiles_m, tiles_n,
                       k_span, g.sa, g.sb, g.sc);
  } else {
    hipLaunchKernelGGL((gemm_i8_mfma<BM, BN, BK, WGM, WGN, BNK, AU8, false>), grid, block, 0,
                       st, g.A, g.lda, g.B, g.ldb, g.C, g.ldc, g.M, g.N, g.K, tiles_m, tiles_n,
                       k_span, g.sa, g.sb, g.sc);
  }
  SIMP_HIP(hipGetLastError());
  return SIMP_RT_OK;
}

template <bool BNK, bool AU8>
int dispatch(const GemmArgs &g, hipStream_t st) {
  if (g.M == 0 || g.N == 0 || g.batch == 0) return SIMP_RT_OK;
  const int64_t cus = num_cus();
  auto tiles = [&](int bm, int bn) { return cdiv(g.M, bm) * cdiv(g.N, bn); };
  if (g.batch > 1 && tiles(256, 256) >= cus) {
    // each product fills the chip alone: one dispatch per product, in stream order
    for (int b = 0; b < g.batch; b++) {
      GemmArgs h = g;
      h.A += b * g.sa;
      h.B += b * g.sb;
      h.C += b * g.sc;
      h.batch = 1;
      h.sa = h.sb = h.sc = 0;
      int rc = dispatch<BNK, AU8>(h, st);
      if (rc) return rc;
    }
    return SIMP_RT_OK;
  }
  if (g.K == 0) {
    const int64_t tot = (int64_t)g.M * g.N;
    hipLaunchKernelGGL(fill_i32_2d, dim3((unsigned)cdiv(tot, 256), 1, g.batch), dim3(256), 0, st,
                       g.C, g.ldc, g.M, g.N, g.sc);
    SIMP_HIP(hipGetLastError());
    return SIMP_RT_OK;
  }
  const bool a_ok = g.K % 16 == 0 && g.lda % 16 == 0 && ((uintptr_t)g.A & 15) == 0 &&
                    g.sa % 16 == 0;
  const bool b_ok = BNK ? (g.ldb % 16 == 0 && ((uintptr_t)g.B & 15) == 0 && g.sb % 16 == 0)
                        : (g.N % 4 == 0 && g.ldb % 4 == 0 && ((uintptr_t)g.B & 3) == 0 &&
                           g.sb % 4 == 0);
  if (!a_ok || !b_ok) {
    dim3 grid((unsigned)cdiv(g.N, 64), (unsigned)std::min<int64_t>(cdiv(g.M, 4), 65535),
              g.batch);
    hipLaunchKernelGGL((gemm_i8_generic<BNK, AU8>), grid, dim3(256), 0, st, g.A, g.lda, g.B,
                       g.ldb, g.C, g.ldc, g.M, g.N, g.K, g.sa, g.sb, g.sc);
    SIMP_HIP(hipGetLastError());
    return SIMP_RT_OK;
  }
  if (g.batch == 1 && tiles(256, 256) >= cus && g.N % 16 == 0) {
    const int tm = (int)cdiv(g.M, 256), tn = (int)cdiv(g.N, 256);
    const int vec = g.ldc % 4 == 0 && ((uintptr_t)g.C & 15) == 0;
    // persistent grid: one workgroup per CU, a multiple of 8 (XCD round-robin)
    const int grid = (int)std::max<int64_t>(8, std::min<int64_t>(cus, (int64_t)tm * tn) / 8 * 8);
    // B[K,N] with 16-byte aligned rows is read in place by gemm_i8_dma
    const bool direct = !BNK && g.K % 64 == 0 && g.ldb % 16 == 0 && ((uintptr_t)g.B & 15) == 0;
    // u8 x s8 column sums inside gemm_i8_dma, on the MFMA pipe (two more MFMAs
    // per 32 while a workgroup forms them), wherever it reads B directly:
    //   * up to 16 tile rows, tiles grouped by rows and the sums formed for
    //     every tile (kColsumRows): whole call 4096^3 71.0-73.7 us against
    //     74.5-81.3 with a pass over B and its zero fill ahead of the GEMM,
    //     4096x8192x4096 131 against 141;
    //   * beyond, tiles grouped by columns, so a workgroup's tiles share their
    //     columns and it forms the sums once per column tile (kColsumOnce):
    //     8192^3 476 against 485 us with the pass (every tile: 488),
    //     8192x4096x8192 263 against 272-276.  (Grouped by columns, s8 x s8
    //     ran 443 against 449 us at 8192^3; at 4096^3 the row groups stay
    //     ahead, 71.0 against 72.1 us.)
    const bool csk = AU8 && (direct || (BNK && g.K % 64 == 0));
    // Workspace: [colsum: N int32, 256-byte aligned, unless in the kernel][B_T:
    // N x K bytes when B is [K,N] and not read in place]
    GemmArgs h = g;
    const size_t cs_bytes = AU8 && !csk ? ((size_t)g.N * 4 + 255) / 256 * 256 : 0;
    void *ws = nullptr;
    const size_t need = cs_bytes + (BNK || direct ? 0 : (size_t)g.K * g.N);
    if (g.scratch) {
      if (need > g.scratch_bytes)
        return set_error(SIMP_RT_EINVAL,
                         "scratch of %zu bytes needed for M=%d N=%d K=%d, above the "
                         "allocation-free maximum of %zu bytes", need, g.M, g.N, g.K,
                         g.scratch_bytes);
      ws = g.scratch;
    } else if (need) {
      int rc = workspace(st, need, &ws);
      if (rc) return rc;
    }
    int32_t *colsum = AU8 && !csk ? (int32_t *)ws : nullptr;
    if (csk || direct) {
      KernelTimer kt(st, "gemm_i8_dma");
      auto launch = [&](auto bnk, auto csm) {
        hipLaunchKernelGGL((gemm_i8_dma<4, AU8, decltype(bnk)::value, decltype(csm)::value>),
                           dim3(grid), dim3(512), 0, st, g.A, g.lda, g.B, g.ldb, g.C, g.ldc, g.M,
                           g.N, g.K, tm, tn, (const int32_t *)nullptr, vec);
      };
      using Rows = std::integral_constant<int, kColsumRows>;
      using Once = std::integral_constant<int, kColsumOnce>;
      using Pass = std::integral_constant<int, kColsumPass>;
      if constexpr (!AU8) {
        // s8 x s8 (no sums): tiles grouped by columns beyond 16 tile rows
        if (tm <= 16) launch(std::false_type{}, Pass{});
        else launch(std::false_type{}, Once{});
      } else if (direct) {
        if (tm <= 16) launch(std::false_type{}, Rows{});
        else launch(std::false_type{}, Once{});
      } else {
        if (tm <= 16) launch(std::true_type{}, Rows{});
        else launch(std::true_type{}, Once{});
      }
      SIMP_HIP(hipGetLastError());
      return SIMP_RT_OK;
    }
    if (!BNK) {  // B[K,N] -> B_T[N,K], column sums on the way
      constexpr int KT = 256;
      int8_t *bt = (int8_t *)ws + cs_bytes;
      if (AU8)
        hipLaunchKernelGGL(fill_i32_2d, dim3((unsigned)cdiv(g.N, 256)), dim3(256), 0, st, colsum,
                           (int64_t)g.N, 1, g.N, (int64_t)0);
      KernelTimer kt(st, "transpose_i8");
      hipLaunchKernelGGL(transpose_i8<KT>, dim3((unsigned)cdiv(g.N, 128), (unsigned)cdiv(g.K, KT)),
                         dim3(256), 0, st, g.B, g.ldb, bt, g.K, g.N, colsum);
      h.B = bt;
      h.ldb = g.K;
    } else if (AU8) {
      hipLaunchKernelGGL(colsum_nk_i8, dim3((unsigned)cdiv(g.N, 4)), dim3(256), 0, st, g.B, g.ldb,
                         colsum, g.N, g.K);
    }
    if (g.K % 64 == 0) {
      KernelTimer kt(st, "gemm_i8_dma");
      hipLaunchKernelGGL((gemm_i8_dma<4, AU8, true>), dim3(grid), dim3(512), 0, st, h.A, h.lda,
                         h.B, h.ldb, h.C, h.ldc, h.M, h.N, h.K, tm, tn, (const int32_t *)colsum,
                         vec);
    } else {
      KernelTimer kt(st, "gemm_i8_nt16");
      hipLaunchKernelGGL((gemm_i8_nt16<256, 256, 128, 2, 4, AU8>), dim3(tm * tn), dim3(512), 0,
                         st, h.A, h.lda, h.B, h.ldb, h.C, h.ldc, h.M, h.N, h.K, tm, tn,
                         (const int32_t *)colsum);
    }
    SIMP_HIP(hipGetLastError());
    return SIMP_RT_OK;
  }
  {
    // mid sizes (K % 128 == 0): the ring kernel, 128x128 tiles from about half
    // a tile per CU on, else 64x64 tiles; 8 waves (2 per SIMD) either way.
    // Ring depth (u8 x s8 whole calls, graph replay, 2 against 4 slots):
    //   * 128x128 tiles: 2 slots at every shape measured: 2048^3 x K = 3200,
    //     4096, 8192: 22.2 / 24.0, 26.5 / 28.8, 46.8 / 50.4 us; 3072^3 (several
    //     tiles per workgroup) 56.9 / 60.2; 512x3200x8640 41.1 / 42.4.
    //   * 64x64 tiles: 2 slots while every workgroup has one tile and K <= 2048
    //     (768^3 4.55 / 4.79 / 5.05 us with 2 / 4 / 8, 1024^3 5.36 / 5.66 /
    //     6.23), or K <= 4096 with the chip about full (1024x3200x1024 11.5 /
    //     12.3, 1024x4096x1024 13.7 / 15.1); else 4 (1024x8192x1024 33.2 /
    //     26.5, 64x3200x8640 on 135 tiles 14.2 / 12.3).
    // A deeper prefetch spreads an XCD's CUs over more operand lines than its
    // L2 keeps; a shallower one exposes the load latency when a CU has the
    // memory system to itself for longer (long K, part of the chip idle).
    const bool ok = g.batch == 1 && g.K % 128 == 0 && g.N % 16 == 0 && g.ldb % 16 == 0 &&
                    ((uintptr_t)g.B & 15) == 0;
    const int vec = g.ldc % 4 == 0 && ((uintptr_t)g.C & 15) == 0;
    auto ring = [&](auto bm, auto slots) {
      constexpr int BM = decltype(bm)::value, SL = decltype(slots)::value;
      const int tm = (int)cdiv(g.M, BM), tn = (int)cdiv(g.N, BM);
      const int grid = (int)std::min<int64_t>((int64_t)tm * tn, cus);
      KernelTimer kt(st, "gemm_i8_ring");
      hipLaunchKernelGGL((gemm_i8_ring<BM, BM, 4, 2, SL, AU8, BNK>), dim3(grid), dim3(512), 0, st,
                         g.A, g.lda, g.B, g.ldb, g.C, g.ldc, g.M, g.N, g.K, tm, tn, vec);
      SIMP_HIP(hipGetLastError());
      return SIMP_RT_OK;
    };
    using I2 = std::integral_constant<int, 2>;
    using I4 = std::integral_constant<int, 4>;
    using I64 = std::integral_constant<int, 64>;
    using I128 = std::integral_constant<int, 128>;
    // 128x128 tiles also where 64x64 ones would need a second round on some
    // CUs and K is long (96 and 128 x 3200 x 8640: 20.2 and 21.4 us on 68
    // tiles against 22.4 and 22.7 on 270); 4 slots where the operands stream
    // from HBM rather than L2 (128x3200x32000: 24.5 against 25.0 us).
    const int64_t t128 = tiles(128, 128), t64 = tiles(64, 64);
    if (ok && g.M > 64 && (2 * t128 >= cus || (t64 > cus && 4 * t128 >= cus && g.K >= 3072))) {
      if ((int64_t)g.K * (g.M + g.N) >= (int64_t(64) << 20)) return ring(I128(), I4());
      return ring(I128(), I2());
    }
    if (ok && 2 * t64 >= cus && g.M > 32) {
      if (t64 <= cus && (g.K <= 2048 || (g.K <= 4096 && 4 * t64 >= 3 * cus)))
        return ring(I64(), I2());
      return ring(I64(), I4());
    }
  }
  if constexpr (!BNK) {
    // M = 1 with B of 4 MB or more, M = 2 with 8 MB or more (smaller B is
    // launch-bound either way): the dot4 GEMV, K split into bands for about
    // 2048 waves (bands of at least 64 rows; more waves measured slower, the
    // atomics growing with them), summed into a zero-filled C when there is
    // more than one
    const int64_t kn = (int64_t)g.K * g.N;
    const bool gemv = (g.M == 1 && kn >= (int64_t(4) << 20)) || (g.M == 2 && kn >= (int64_t(8) << 20));
    if (g.batch == 1 && gemv && g.N % 8 == 0 && g.ldb % 8 == 0 && ((uintptr_t)g.B & 7) == 0) {
      const int G = (int)cdiv(g.N, 512);
      int S = (int)std::max<int64_t>(1, std::min<int64_t>(g.K / 64, cdiv(2048, 4 * (int64_t)G)));
      const int k_span = (int)cdiv(cdiv(g.K, S), 16) * 16;
      S = (int)cdiv(g.K, k_span);
      if (S > 1) {
        const int64_t tot = (int64_t)g.M * g.N;
        hipLaunchKernelGGL(fill_i32_2d, dim3((unsigned)cdiv(tot, 256)), dim3(256), 0, st, g.C,
                           g.ldc, g.M, g.N, (int64_t)0);
      }
      dim3 grid(G, S);
      KernelTimer kt(st, "gemv_i8_kn");
      auto go = [&](auto mr) {
        constexpr int MR = decltype(mr)::value;
        if (S > 1)
          hipLaunchKernelGGL((gemv_i8_kn<MR, AU8, true>), grid, dim3(256), 0, st, g.A, g.lda, g.B,
                             g.ldb, g.C, g.ldc, g.M, g.N, g.K, k_span);
        else
          hipLaunchKernelGGL((gemv_i8_kn<MR, AU8, false>), grid, dim3(256), 0, st, g.A, g.lda,
                             g.B, g.ldb, g.C, g.ldc, g.M, g.N, g.K, k_span);
      };
      if (g.M == 1) go(std::integral_constant<int, 1>{});
      else go(std::integral_constant<int, 2>{});
      SIMP_HIP(hipGetLastError());
      return SIMP_RT_OK;
    }
  }
  // Split K for about four workgroups per CU (at most 16 splits): 8x8640x3200
  // 9.4 us with 8 splits against 12.5 with the 4 that two per CU gave and 10.7
  // with 16; the 768 / 2048 shapes reach their K or the cap either way.  One
  // split (no zero fill, no atomics) is 1.6-3.5x slower at these sizes.
  if (tiles(128, 128) * g.batch >= cus) return launch_mfma<128, 128, 128, 2, 2, BNK, AU8>(g, 1, st);
  if (g.M > 32) {
    const int64_t t = tiles(64, 64) * g.batch;
    const int s = (int)std::min<int64_t>(cdiv(4 * cus, t), 16);
    return launch_mfma<64, 64, 128, 2, 2, BNK, AU8>(g, t >= cus ? 1 : s, st);
  }
  const int64_t t = tiles(32, 64) * g.batch;
  const int s = (int)std::min<int64_t>(cdiv(4 * cus, t), 16);
  return launch_mfma<32, 64, 128, 1, 2, BNK, AU8>(g, t >= cus ? 1 : s, st);
}

// ------------------------------------------------------------------ int4 --
// Packed signed nibbles (ConvertSimpToMemRef.cpp:2953-3133): element e of a row
// is nibble e%2 (low = even) of byte e/2, sign-extended.  The product is formed
// exactly on the int8 MFMA path from unpacked operands; the i32 sums are then
// truncated to i16 (:3119-3122).
__device__ __forceinline__ uint32_t sext4(uint32_t nib) { return (nib ^ 8u) - 8u; }

// A[rows, K] packed along K (rows of ldp bytes) -> out[rows, Kp] s8, zero for
// K <= k < Kp (Kp % 16 == 0).  One thread per 16 outputs (8 packed bytes).
__global__ void __launch_bounds__(256)
    unpack_i4_rows(const uint8_t *__restrict__ P, int64_t ldp, int8_t *__restrict__ out,
                   int64_t ldo, int rows, int K, int Kp) {
  const int64_t chunks = Kp / 16;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)rows * chunks) return;
  const int64_t r = idx / chunks;
  const int c = (int)(idx - r * chunks);
  const uint8_t *src = P + r * ldp;
  uint32_t w[4];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    uint32_t word = 0;
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const int byte = c * 8 + q * 2 + b, e = 2 * byte;
      const uint32_t v = e < K ? src[byte] : 0u;
      const uint32_t lo = sext4(v & 15u) & 255u;
      const uint32_t hi = e + 1 < K ? sext4(v >> 4) & 255u : 0u;  // odd K: pad nibble
      word |= (lo | (hi << 8)) << (16 * b);
    }
    w[q] = word;
  }
  *(uint4 *)(out + r * ldo + 16 * c) = make_uint4(w[0], w[1], w[2], w[3]);
}

// B[K, N] packed along N (rows of ldp bytes) -> B_T[N, Kp] s8 (row pitch ldt),
// zero for K <= k < Kp, through a 64x64 LDS tile.
__global__ void __launch_bounds__(256)
    unpack_i4_transpose(const uint8_t *__restrict__ P, int64_t ldp, int8_t *__restrict__ BT,
                        int64_t ldt, int K, int N, int Kp) {
  __shared__ uint8_t s[64][64 + 4];
  const int t = threadIdx.x;
  const int k0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  {
    const int k = t >> 2, c = t & 3, gk = k0 + k;
#pragma unroll
    for (int b = 0; b < 8; b++) {
      const int n = n0 + 16 * c + 2 * b;  // even element of the pair
      const uint32_t v = (gk < K && n < N) ? P[(int64_t)gk * ldp + n / 2] : 0u;
      s[k][16 * c + 2 * b] = (uint8_t)sext4(v & 15u);
      s[k][16 * c + 2 * b + 1] = n + 1 < N ? (uint8_t)sext4(v >> 4) : (uint8_t)0;
    }
  }
  __syncthreads();
  {
    const int n = t >> 2, c = t & 3;
    const int gn = n0 + n, gk = k0 + 16 * c;
    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 16; j++) w[j >> 2] |= (uint32_t)s[16 * c + j][n] << (8 * (j & 3));
    if (gn < N && gk < Kp) *(uint4 *)(BT + (int64_t)gn * ldt + gk) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// C16[r, c] = (int16) C32[r, c]
__global__ void __launch_bounds__(256)
    store_i16(const int32_t *__restrict__ C32, int64_t ld32, int16_t *__restrict__ C, int64_t ldc,
              int M, int N) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)M * N) return;
  const int64_t r = i / N, c = i - r * N;
  C[r * ldc + c] = (int16_t)C32[r * ld32 + c];
}

// Shared body of the four entry points.
template <bool BNK, bool AU8>
int gemm_entry(const char *name, const void *a, int64_t a_off, int64_t a_s0, int64_t a_s1,
               int64_t a_st0, int64_t a_st1, const int8_t *b, int64_t b_off, int64_t b_s0,
               int64_t b_s1, int64_t b_st0, int64_t b_st1, int32_t *c, int64_t c_off,
               int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1) {
  int rc;
  if ((rc = check_desc2("A", a, a_off, a_s0, a_s1, a_st0, a_st1))) return rc;
  if ((rc = check_desc2("B", b, b_off, b_s0, b_s1, b_st0, b_st1))) return rc;
  if ((rc = check_desc2("C", c, c_off, c_s0, c_s1, c_st0, c_st1))) return rc;
  const int64_t M = a_s0, K = a_s1;
  const int64_t N = BNK ? b_s0 : b_s1;
  const int64_t Kb = BNK ? b_s1 : b_s0;
  if (Kb != K || c_s0 != M || c_s1 != N)
    return set_error(SIMP_RT_EINVAL,
                     "%s: shape mismatch A[%lld,%lld] B%s[%lld,%lld] C[%lld,%lld]", name,
                     (long long)a_s0, (long long)a_s1, BNK ? "_T" : "", (long long)b_s0,
                     (long long)b_s1, (long long)c_s0, (long long)c_s1);
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return set_error(SIMP_RT_EUNSUPPORTED, "%s: dimension above 2^31-1", name);
  Operand oa, ob, oc;
  const size_t a_bytes = (M && K) ? (size_t)((M - 1) * a_st0 + K) : 0;
  const size_t b_bytes = (b_s0 && b_s1) ? (size_t)((b_s0 - 1) * b_st0 + b_s1) : 0;
  const size_t c_bytes = (M && N) ? (size_t)((M - 1) * c_st0 + N) * 4 : 0;
  if ((rc = oa.bind((const int8_t *)a + a_off, a_bytes, Operand::kIn, "A"))) return rc;
  if ((rc = ob.bind(b + b_off, b_bytes, Operand::kIn, "B"))) return rc;
  if ((rc = oc.bind(c + c_off, c_bytes, Operand::kOut, "C"))) return rc;
  GemmArgs g{(const int8_t *)oa.dev(), a_st0, (const int8_t *)ob.dev(), b_st0,
             (int32_t *)oc.dev(),      c_st0, (int)M, (int)N, (int)K};
  if ((rc = dispatch<BNK, AU8>(g, cur_stream()))) return rc;
  Operand *ops[] = {&oa, &ob, &oc};
  return finish(ops, 3);
}

// Rank-3 s8 x s8 -> i32: C[b] = A[b] x B[b] for every batch b (linalg.batch_matmul
// on i8 operands into the zero-filled i32 result, ConvertSimpToMemRef.cpp:
// 2926-2933,3286-3291; linalg sign-extends both operands).
int batch_i8_entry(const int8_t *a, int64_t a_off, const int64_t *as, const int64_t *ast,
                   const int8_t *b, int64_t b_off, const int64_t *bs, const int64_t *bst,
                   int32_t *c, int64_t c_off, const int64_t *cs, const int64_t *cst) {
  const char *name = "tensor_batch_matmul_i8";
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
  if ((rc = oa.bind(a + a_off, (size_t)an, Operand::kIn, "A"))) return rc;
  if ((rc = ob.bind(b + b_off, (size_t)bn, Operand::kIn, "B"))) return rc;
  if ((rc = oc.bind(c + c_off, 4 * (size_t)cn, Operand::kOut, "C"))) return rc;
  const int8_t *da = (const int8_t *)oa.dev(), *db = (const int8_t *)ob.dev();
  int32_t *dc = (int32_t *)oc.dev();
  for (int64_t b0 = 0; b0 < Bt; b0 += 65535) {  // grid z holds at most 65535 products
    GemmArgs g{da + b0 * ast[0], ast[1], db + b0 * bst[0], bst[1], dc + b0 * cst[0], cst[1],
               (int)M, (int)N, (int)K};
    g.batch = (int)std::min<int64_t>(65535, Bt - b0);
    g.sa = ast[0];
    g.sb = bst[0];
    g.sc = cst[0];
    if ((rc = dispatch<false, false>(g, cur_stream()))) return rc;
  }
  Operand *ops[] = {&oa, &ob, &oc};
  return finish(ops, 3);
}

}  // namespace

// ------------------------------------------------ allocation-free variant --
// Scratch of simp_rt_matmul_u8s8_i32_noalloc: the column sums of B (N i32,
// rounded up to 256 bytes) followed, when B is not read in place, by B_T[N,K],
// as the stream workspace holds them.  One copy per GPU, for the life of the
// process.
constexpr size_t kNoAllocScratchBytes = (size_t(64) << 20) + (size_t(64) << 10);
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
std::mutex g_scratch_mu;
std::vector<void *> g_scratch_addr;  // device address of `scratch`, per device
}  // namespace

// The host-side name `scratch` is not a device address: the device address of
// each GPU's copy is looked up once, with that device current, and kept.
int noalloc_scratch(void **ptr) {
  const int dev = ensure_device();
  if (dev < 0) return dev;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if ((int)g_scratch_addr.size() <= dev) g_scratch_addr.resize(dev + 1, nullptr);
  if (!g_scratch_addr[dev]) {
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p) return set_error(SIMP_RT_EHIP, "hipGetSymbolAddress(scratch) returned null");
    g_scratch_addr[dev] = p;
  }
  *ptr = g_scratch_addr[dev];
  return SIMP_RT_OK;
}

}  // namespace simp

using namespace simp;

extern "C" {

int32_t simp_rt_matmul_u8s8_i32_noalloc(
    const uint8_t *a_alloc, const uint8_t *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const int8_t *b_alloc, const int8_t *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_st0, int64_t b_st1,
    int32_t *c_alloc, int32_t *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1) {
  (void)a_alloc; (void)b_alloc; (void)c_alloc;
  const char *name = "matmul_u8s8_i32_noalloc";
  int rc;
  if ((rc = check_desc2("A", a, a_off, a_s0, a_s1, a_st0, a_st1))) return rc;
  if ((rc = check_desc2("B", b, b_off, b_s0, b_s1, b_st0, b_st1))) return rc;
  if ((rc = check_desc2("C", c, c_off, c_s0, c_s1, c_st0, c_st1))) return rc;
  const int64_t M = a_s0, K = a_s1, N = b_s1;
  if (b_s0 != K || c_s0 != M || c_s1 != N)
    return set_error(SIMP_RT_EINVAL, "%s: shape mismatch A[%lld,%lld] B[%lld,%lld] C[%lld,%lld]",
                     name, (long long)a_s0, (long long)a_s1, (long long)b_s0, (long long)b_s1,
                     (long long)c_s0, (long long)c_s1);
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return set_error(SIMP_RT_EUNSUPPORTED, "%s: dimension above 2^31-1", name);
  if (M == 0 || N == 0) return SIMP_RT_OK;
  // operands must already be on the device: staging host memory would allocate
  const void *da = nullptr, *db = nullptr, *dc = nullptr;
  const size_t a_bytes = K ? (size_t)((M - 1) * a_st0 + K) : 0;
  const size_t b_bytes = K ? (size_t)((K - 1) * b_st0 + N) : 0;
  const size_t c_bytes = (size_t)((M - 1) * c_st0 + N) * 4;
  if (K && ((rc = device_view(a + a_off, a_bytes, &da, "A")) ||
            (rc = device_view(b + b_off, b_bytes, &db, "B"))))
    return rc;
  if ((rc = device_view(c + c_off, c_bytes, &dc, "C"))) return rc;
  void *ws = nullptr;
  if ((rc = noalloc_scratch(&ws))) return rc;
  GemmArgs g{(const int8_t *)da, a_st0, (const int8_t *)db, b_st0, (int32_t *)dc, c_st0,
             (int)M, (int)N, (int)K};
  g.scratch = ws;
  g.scratch_bytes = kNoAllocScratchBytes;
  if ((rc = dispatch<false, true>(g, cur_stream()))) return rc;
  SIMP_HIP(hipGetLastError());
  return SIMP_RT_OK;
}

int32_t simp_rt_tensor_matmul_i8(
    const int8_t *a_alloc, const int8_t *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const int8_t *b_alloc, const int8_t *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_st0, int64_t b_st1,
    int32_t *c_alloc, int32_t *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1) {
  (void)a_alloc; (void)b_alloc; (void)c_alloc;
  return gemm_entry<false, false>("tensor_matmul_i8", a, a_off, a_s0, a_s1, a_st0, a_st1, b, b_off,
                                  b_s0, b_s1, b_st0, b_st1, c, c_off, c_s0, c_s1, c_st0, c_st1);
}

int32_t simp_rt_tensor_matmul_nt_i8(
    const int8_t *a_alloc, const int8_t *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const int8_t *bt_alloc, const int8_t *bt, int64_t bt_off, int64_t bt_s0, int64_t bt_s1, int64_t bt_st0, int64_t bt_st1,
    int32_t *c_alloc, int32_t *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1) {
  (void)a_alloc; (void)bt_alloc; (void)c_alloc;
  return gemm_entry<true, false>("tensor_matmul_nt_i8", a, a_off, a_s0, a_s1, a_st0, a_st1, bt,
                                 bt_off, bt_s0, bt_s1, bt_st0, bt_st1, c, c_off, c_s0, c_s1, c_st0,
                                 c_st1);
}

int32_t simp_rt_matmul_u8s8_i32(
    const uint8_t *a_alloc, const uint8_t *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const int8_t *b_alloc, const int8_t *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_st0, int64_t b_st1,
    int32_t *c_alloc, int32_t *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1) {
  (void)a_alloc; (void)b_alloc; (void)c_alloc;
  return gemm_entry<false, true>("matmul_u8s8_i32", a, a_off, a_s0, a_s1, a_st0, a_st1, b, b_off,
                                 b_s0, b_s1, b_st0, b_st1, c, c_off, c_s0, c_s1, c_st0, c_st1);
}

int32_t simp_rt_matmul_nt_u8s8_i32(
    const uint8_t *a_alloc, const uint8_t *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const int8_t *bt_alloc, const int8_t *bt, int64_t bt_off, int64_t bt_s0, int64_t bt_s1, int64_t bt_st0, int64_t bt_st1,
    int32_t *c_alloc, int32_t *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1) {
  (void)a_alloc; (void)bt_alloc; (void)c_alloc;
  return gemm_entry<true, true>("matmul_nt_u8s8_i32", a, a_off, a_s0, a_s1, a_st0, a_st1, bt,
                                bt_off, bt_s0, bt_s1, bt_st0, bt_st1, c, c_off, c_s0, c_s1, c_st0,
                                c_st1);
}

int32_t simp_rt_tensor_matvecmul_i8(
    const int8_t *a_alloc, const int8_t *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const int8_t *b_alloc, const int8_t *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_st0, int64_t b_st1,
    int32_t *c_alloc, int32_t *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1) {
  (void)a_alloc; (void)b_alloc; (void)c_alloc;
  return gemm_entry<false, false>("tensor_matvecmul_i8", a, a_off, a_s0, a_s1, a_st0, a_st1, b,
                                  b_off, b_s0, b_s1, b_st0, b_st1, c, c_off, c_s0, c_s1, c_st0,
                                  c_st1);
}

int32_t simp_rt_tensor_batch_matmul_i8(
    const int8_t *a_alloc, const int8_t *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_s2,
    int64_t a_st0, int64_t a_st1, int64_t a_st2,
    const int8_t *b_alloc, const int8_t *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_s2,
    int64_t b_st0, int64_t b_st1, int64_t b_st2,
    int32_t *c_alloc, int32_t *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_s2,
    int64_t c_st0, int64_t c_st1, int64_t c_st2) {
  (void)a_alloc; (void)b_alloc; (void)c_alloc;
  const int64_t as[3] = {a_s0, a_s1, a_s2}, ast[3] = {a_st0, a_st1, a_st2};
  const int64_t bs[3] = {b_s0, b_s1, b_s2}, bst[3] = {b_st0, b_st1, b_st2};
  const int64_t cs[3] = {c_s0, c_s1, c_s2}, cst[3] = {c_st0, c_st1, c_st2};
  return batch_i8_entry(a, a_off, as, ast, b, b_off, bs, bst, c, c_off, cs, cst);
}

int32_t simp_rt_tensor_matmul_i4(
    const int8_t *a_alloc, const int8_t *a, int64_t a_off, int64_t a_s0, int64_t a_s1, int64_t a_st0, int64_t a_st1,
    const int8_t *b_alloc, const int8_t *b, int64_t b_off, int64_t b_s0, int64_t b_s1, int64_t b_st0, int64_t b_st1,
    int16_t *c_alloc, int16_t *c, int64_t c_off, int64_t c_s0, int64_t c_s1, int64_t c_st0, int64_t c_st1) {
  (void)a_alloc; (void)b_alloc; (void)c_alloc;
  const char *name = "tensor_matmul_i4";
  int rc;
  if ((rc = check_desc2("A", a, a_off, a_s0, a_s1, a_st0, a_st1))) return rc;
  if ((rc = check_desc2("B", b, b_off, b_s0, b_s1, b_st0, b_st1))) return rc;
  if ((rc = check_desc2("C", c, c_off, c_s0, c_s1, c_st0, c_st1))) return rc;
  // logical sizes: M = A rows, K = B rows, N = C columns; packed widths follow
  const int64_t M = a_s0, K = b_s0, N = c_s1;
  if (c_s0 != M || a_s1 != (K + 1) / 2 || b_s1 != (N + 1) / 2)
    return set_error(SIMP_RT_EINVAL,
                     "%s: shape mismatch A[%lld,%lld] B[%lld,%lld] C[%lld,%lld] "
                     "(packed: A[M,(K+1)/2], B[K,(N+1)/2], C[M,N])",
                     name, (long long)a_s0, (long long)a_s1, (long long)b_s0, (long long)b_s1,
                     (long long)c_s0, (long long)c_s1);
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX - 64)
    return set_error(SIMP_RT_EUNSUPPORTED, "%s: dimension above 2^31-1", name);
  if (M == 0 || N == 0) return SIMP_RT_OK;
  Operand oa, ob, oc;
  const size_t a_bytes = a_s1 ? (size_t)((M - 1) * a_st0 + a_s1) : 0;
  const size_t b_bytes = (K && b_s1) ? (size_t)((K - 1) * b_st0 + b_s1) : 0;
  const size_t c_bytes = (size_t)((M - 1) * c_st0 + N) * 2;
  if ((rc = oa.bind(a + a_off, a_bytes, Operand::kIn, "A"))) return rc;
  if ((rc = ob.bind(b + b_off, b_bytes, Operand::kIn, "B"))) return rc;
  if ((rc = oc.bind(c + c_off, c_bytes, Operand::kOut, "C"))) return rc;
  hipStream_t st = cur_stream();
  // staging (workspace slot 1): A8[M,Kp] | B_T8[N,Kp] | C32[M,N], 256-byte aligned
  const int64_t Kp = std::max<int64_t>(64, cdiv(K, 64) * 64);
  auto al = [](size_t x) { return (x + 255) / 256 * 256; };
  const size_t a8 = al((size_t)M * Kp), b8 = al((size_t)N * Kp), c32 = al((size_t)M * N * 4);
  void *ws = nullptr;
  if ((rc = workspace(st, a8 + b8 + c32, &ws, 1))) return rc;
  int8_t *A8 = (int8_t *)ws, *BT8 = A8 + a8;
  int32_t *C32 = (int32_t *)(BT8 + b8);
  hipLaunchKernelGGL(unpack_i4_rows, dim3((unsigned)cdiv(M * (Kp / 16), 256)), dim3(256), 0, st,
                     (const uint8_t *)oa.dev(), a_st0, A8, Kp, (int)M, (int)K, (int)Kp);
  hipLaunchKernelGGL(unpack_i4_transpose, dim3((unsigned)cdiv(N, 64), (unsigned)(Kp / 64)),
                     dim3(256), 0, st, (const uint8_t *)ob.dev(), b_st0, BT8, Kp, (int)K, (int)N,
                     (int)Kp);
  SIMP_HIP(hipGetLastError());
  GemmArgs g{A8, Kp, BT8, Kp, C32, N, (int)M, (int)N, (int)Kp};
  if ((rc = dispatch<true, false>(g, st))) return rc;
  hipLaunchKernelGGL(store_i16, dim3((unsigned)cdiv(M * N, 256)), dim3(256), 0, st,
                     (const int32_t *)C32, N, (int16_t *)oc.dev(), c_st0, (int)M, (int)N);
  SIMP_HIP(hipGetLastError());
  Operand *ops[] = {&oa, &ob, &oc};
  return finish(ops, 3);
}

}  // extern "C"
