// w4d8.hip -- W4 GEMV (symmetric nibbles, or unsigned with zeros) with one to four x vectors on v_dot8_i32_i4.
//
// The product out[n] = sum_k q[n,k] * s[n, k/gs] * x[k] of
// MatMulQuantOpLowering (ConvertSimpToMemRef.cpp:3906-4005) for the signed
// nibble format (q in [-8,7], two per byte, low nibble = even k), computed as
// exact integer dot products per 32-weight chunk:
//   * x is converted once per block into six signed 4-bit limbs per element:
//     with e the exponent of the chunk's largest |x| (|x| < 2^e),
//     I = round(x * 2^(22-e)) is a 23-bit integer, written in balanced base 16
//     as I = sum_j d_j 16^j with d_j in [-8,7].  Limb j of eight consecutive
//     elements forms one dword whose nibble i is d_j of element i -- the same
//     nibble order as the weight dword, so v_dot8_i32_i4(w, L_j) is
//     sum_i q_i d_{j,i} exactly.
//   * Per chunk (4 weight dwords) T = sum_j 16^j sum_d dot8(w_d, L_{j,d}) is
//     evaluated Horner-style in one int32 chain (|T| < 32 * 8 * 2^22 = 2^30,
//     so it is exact), then out += (s * 2^(e-22)) * float(T).  The only
//     departure from exact products of the fp32 inputs is x rounded to 23
//     significant bits relative to its chunk's maximum, and the order of the
//     fp32 sums over chunks and lanes.
// Layout: lane -> K.  A wave's lanes own fixed chunks of K (C per lane, KT
// waves cover a row), so the limbs live in registers for the whole kernel and
// a wave load covers a contiguous run of one row.  Rows of a block are split
// over its teams of KT waves; each team streams its rows through a window of
// D rows in flight (row i + D is requested right after row i is consumed),
// which keeps the memory queues short enough for x (requested first) to
// arrive early, and keeps arrival order close to consumption order.
// Segments: up to three matrices with their own weights, scales and outputs
// (Wq | Wk | Wv as one launch), or, in the paired mode, rows i of W1 and W3
// computed by the same wave and combined as silu(h1) * h3.
// Unsigned nibbles with a zero per group (weight = u * s + z, the format of
// MatMulQuantOpLowering): u - 8 is the signed nibble u ^ 8, so a chunk is
// s * sum (u - 8) x + (8 s + z) * sum x; the chunk's sum of x is kept per
// chunk from the same 23-bit integers, sum_i I_i exact in int32.
#include <algorithm>

#include "rt_device.h"
#include "rt_internal.h"

namespace simp {
namespace {

// u[i]: 24-bit offset-binary values I_i + 0x888888 (six nibbles each).  L[j]
// nibble i = nibble j of u[i] xor 8 (= the balanced digit d_j of I_i in
// two's complement).  Byte permutes gather 16-bit halves, then bytes, then a
// bitfield insert interleaves the nibbles of even and odd elements.
__device__ __forceinline__ void limbs8(const uint32_t (&u)[8], uint32_t (&L)[6]) {
  uint32_t a[4], b[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    a[i] = __builtin_amdgcn_perm(u[i + 4], u[i], 0x05040100u);  // bytes 0,1 of u_i, u_i+4
    b[i] = __builtin_amdgcn_perm(u[i + 4], u[i], 0x0C060C02u);  // byte 2 of u_i, u_i+4
  }
  uint32_t c[2], d[2], e[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    c[i] = __builtin_amdgcn_perm(a[i + 2], a[i], 0x06020400u);  // byte 0 of u_i, i+2, i+4, i+6
    d[i] = __builtin_amdgcn_perm(a[i + 2], a[i], 0x07030501u);  // byte 1
    e[i] = __builtin_amdgcn_perm(b[i + 2], b[i], 0x06020400u);  // byte 2
  }
  const uint32_t m = 0x0F0F0F0Fu;
  L[0] = (c[0] & m) | ((c[1] << 4) & ~m);
  L[1] = ((c[0] >> 4) & m) | (c[1] & ~m);
  L[2] = (d[0] & m) | ((d[1] << 4) & ~m);
  L[3] = ((d[0] >> 4) & m) | (d[1] & ~m);
  L[4] = (e[0] & m) | ((e[1] << 4) & ~m);
  L[5] = ((e[0] >> 4) & m) | (e[1] & ~m);
#pragma unroll
  for (int j = 0; j < 6; j++) L[j] ^= 0x88888888u;
}

// Sums each of the RM per-lane values over the 64 lanes of the wave.  After
// the call, lane l holds the total of row l >> (6 - log2 RM) in p[0]
// (transposed butterfly: each exchange step halves the values per lane).  The
// exchanges across 32 and 16 lanes are v_permlane{32,16}_swap (a' + b' pairs
// each value with the other half's), the ones inside a row DPP moves with a
// select; every step stays in the VALU.
template <int RM>
__device__ __forceinline__ void rows_reduce(float (&p)[RM], int lane) {
  int cnt = RM;
  // masks 32 and 16
  if (cnt > 1) {
#pragma unroll
    for (int i = 0; i < RM / 2; i++) {
      float a = p[i], b = p[i + RM / 2];
      permlane32_swap(a, b);
      p[i] = a + b;
    }
    cnt >>= 1;
  } else {
    float a = p[0], b = p[0];
    permlane32_swap(a, b);
    p[0] = a + b;
  }
  if (cnt > 1) {
#pragma unroll
    for (int i = 0; i < RM / 4; i++) {
      if (i < cnt / 2) {
        float a = p[i], b = p[i + cnt / 2];
        permlane16_swap(a, b);
        p[i] = a + b;
      }
    }
    cnt >>= 1;
  } else {
    float a = p[0], b = p[0];
    permlane16_swap(a, b);
    p[0] = a + b;
  }
  // mask 8 (row_ror:8 is lane ^ 8), then 4 (half mirror flips bit 2; the
  // quad steps after it cover the partner's quad), 2, 1
  auto step = [&](auto dppfn, int m) {
    if (cnt > 1) {
      const bool h = (lane & m) != 0;
#pragma unroll
      for (int i = 0; i < RM / 2; i++) {
        if (i < cnt / 2) {
          const float a = p[i], b = p[i + cnt / 2];
          const float send = h ? a : b, keep = h ? b : a;
          p[i] = keep + dppfn(send);
        }
      }
      cnt >>= 1;
    } else {
      p[0] += dppfn(p[0]);
    }
  };
  step([](float v) { return dpp_mov<kDppRor8>(v); }, 8);
  step([](float v) { return dpp_mov<kDppHalfMirror>(v); }, 4);
  step([](float v) { return dpp_mov<kDppXor2>(v); }, 2);
  step([](float v) { return dpp_mov<kDppXor1>(v); }, 1);
}

__device__ __forceinline__ float silu_mul(float h1, float h3) {
  return (h1 / (1.f + expf(-h1))) * h3;
}

// Split-attention partials as x (CMB), in the arithmetic of the decode's
// combine kernel: per head, M = max_s m_s, e_s = e^(m_s - M), 1/L with
// L = sum_s e_s l_s; x = (sum_s e_s o_s) * (1/L).  The first kCmbRegs chunks
// of the thread's elements are requested at kernel start with the heads'
// statistics (one round trip); further chunks (contexts past 4 * 64) are
// read when combined.
constexpr int kCmbRegs = 4;
// C chunks per lane, KT waves per row, NW waves per block (NW / KT teams),
// D rows in flight per team, MULTI: more than one segment (a single segment
// reads every argument at a fixed offset, one round of scalar loads),
// NORM: x = x0 * nw / rms, OUT: 0 store,
// 1 accumulate, 2 pairs (W1 row i, W3 row i) -> silu(h1) * h3 into seg 0.
// MX x vectors (rows of x ldx apart, of out ldo apart; a.mx of them are real):
// each weight dword meets the limbs of every vector, so the weights are read
// once for all of them.
// Units are rows (pairs of rows in mode 2); the blocks of a segment split its
// units evenly, team t of a block takes the block's units t, t + teams, ...
// UZ: unsigned nibbles with zeros (every segment's Z set).  CMB: x from
// split-attention partials (a.cws), combined after the first weight rows are
// requested.
template <int C, int KT, int NW, int D, int RM, bool NORM, int OUT, bool MULTI, int MX, bool UZ,
          bool CMB = false>
__global__ void __launch_bounds__(64 * NW) w4d8_gemv(W4D8Args a) {
  constexpr int NT = 64 * NW, NTM = NW / KT, UPR = OUT == 2 ? 2 : 1;
  static_assert(RM % UPR == 0 && RM >= D, "rows");
  static_assert(MX == 1 || (OUT == 0 && !NORM && !MULTI), "several x vectors: plain stores");
  static_assert(MX == 1 || !UZ, "zeros: one x vector");
  static_assert(!CMB || (MX == 1 && !NORM && !MULTI && OUT == 1), "partials: plain accumulate");
  extern __shared__ __align__(16) uint32_t sm[];
  const int K = a.K, nchunk = K >> 5, ngrp8 = K >> 3;
  const int cpg = a.gs >> 5, cps = cpg_log2(cpg);
  uint32_t *xl = sm;                            // [MX][nchunk][6 limbs][4 dwords]
  float *xf = (float *)(sm + MX * 24 * nchunk); // [MX][nchunk] 2^(e-22)
  float *xs = xf + MX * nchunk;                 // [MX][nchunk] sum of the chunk's x (UZ)
  float *ssq = xs + (UZ ? MX * nchunk : 0);     // [NW]
  float *red = ssq + NW;                        // [NW][MX][RM] row totals per wave
  float *cef = red + NW * MX * RM;              // CMB: [heads][cn] e_s, then [heads] 1/L
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int team = wave / KT, kw = wave - team * KT;
  // x first, before anything else reads the arguments (the weight requests of
  // every wave queue behind it otherwise):
  // one k-group of 8 elements per thread per pass; a config covers at most
  // 64*C*KT chunks, so XP passes cover K, all requested before any weight
  constexpr int XP = (4 * C * KT + NW - 1) / NW;
  float4 xa[MX][XP], xb[MX][XP], na[XP], nb[XP];
  // CMB: chunks 0 .. kCmbRegs-1 of the thread's 2 x XP groups of 4 elements
  float4 cov[CMB ? XP : 1][2][CMB ? kCmbRegs : 1];
  float2 cml[CMB ? kCmbRegs : 1];
  if constexpr (CMB) {
    const int st = a.chs + 4;
#pragma unroll
    for (int ps = 0; ps < XP; ps++)
#pragma unroll
      for (int hf = 0; hf < 2; hf++) {
        const int e0 = 8 * min((int)threadIdx.x + NT * ps, ngrp8 - 1) + 4 * hf;
        const int h = e0 / a.chs;
        const float *w = a.cws + (int64_t)h * a.cmax * st + (e0 - h * a.chs);
#pragma unroll
        for (int s = 0; s < kCmbRegs; s++)
          cov[ps][hf][s] = s < a.cn ? *(const float4 *)(w + s * st) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    // the heads' statistics (m, l) of chunks 0 .. kCmbRegs-1: thread h < heads
    const int h = min((int)threadIdx.x, K / a.chs - 1);
    const float *w = a.cws + (int64_t)h * a.cmax * st + a.chs;
#pragma unroll
    for (int s = 0; s < kCmbRegs; s++)
      cml[s] = s < a.cn ? *(const float2 *)(w + s * st) : make_float2(-INFINITY, 0.f);
  }
#pragma unroll
  for (int ps = 0; ps < XP && !CMB; ps++) {
    const int g8 = min((int)threadIdx.x + NT * ps, ngrp8 - 1);
#pragma unroll
    for (int m = 0; m < MX; m++) {
      const float *xr = a.x0 + (int64_t)min(m, a.mx - 1) * a.ldx;  // vectors past mx repeat the last
      xa[m][ps] = *(const float4 *)(xr + 8 * g8);
      xb[m][ps] = *(const float4 *)(xr + 8 * g8 + 4);
    }
    if constexpr (NORM) {
      na[ps] = *(const float4 *)(a.nw + 8 * g8);
      nb[ps] = *(const float4 *)(a.nw + 8 * g8 + 4);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  const int lpw = (nchunk + KT * C - 1) / (KT * C);  // lanes per wave that own chunks
  int cj[C];
  bool aj[C];
#pragma unroll
  for (int j = 0; j < C; j++) {
    const int cc = j * KT * lpw + kw * lpw + lane;
    cj[j] = min(cc, nchunk - 1);
    aj[j] = lane < lpw && cc < nchunk;
  }
  int sgo[C];  // scale index of the lane's chunks
#pragma unroll
  for (int j = 0; j < C; j++) sgo[j] = chunk_group(cj[j], cpg, cps);
  // the block's segment (blocks [bstart[s], bstart[s+1]) take segment s; in
  // the paired mode all blocks take the pairs of segments 0 and 1) and its units
  const int bx = (int)blockIdx.x;
  const int sg = (OUT == 2 || !MULTI) ? 0 : (bx >= a.bstart[1]) + (bx >= a.bstart[2]);
  const int bs0 = !MULTI ? 0 : (sg == 0 ? 0 : (sg == 1 ? a.bstart[1] : a.bstart[2]));
  const int bs1 = !MULTI ? (int)gridDim.x
                         : (sg == 0 ? min(a.bstart[1], (int)gridDim.x)
                                    : (sg == 1 ? min(a.bstart[2], (int)gridDim.x) : (int)gridDim.x));
  const int seg_units = sg == 0 ? a.s[0].rows : (sg == 1 ? a.s[1].rows : a.s[2].rows);
  const int ub = (int)((int64_t)(bx - bs0) * seg_units / (bs1 - bs0));
  const int ue = (int)((int64_t)(bx - bs0 + 1) * seg_units / (bs1 - bs0));
  const int cnt = max(ue - ub - team + NTM - 1, 0) / NTM * UPR;  // rows of this team

  uint4 w[D][C];
  float s[D][C];
  float z[UZ ? D : 1][UZ ? C : 1];
  // Row pointers of the team, stepped row by row (the team's rows are units
  // ub + team, + NTM, ... of one segment): a 64-bit add per row and matrix.
  // Past its last row a team repeats the last row's requests (cache hits), so
  // every load is unconditional and the compiler's wait counts stay exact.
  const int unit0 = min(ub + team, seg_units - 1);
  const int64_t ldw = sg == 0 ? a.s[0].ldw : (sg == 1 ? a.s[1].ldw : a.s[2].ldw);
  const int64_t lds = sg == 0 ? a.s[0].lds : (sg == 1 ? a.s[1].lds : a.s[2].lds);
  const uint8_t *wp = (sg == 0 ? a.s[0].W : (sg == 1 ? a.s[1].W : a.s[2].W)) + (int64_t)unit0 * ldw;
  const float *sp = (sg == 0 ? a.s[0].S : (sg == 1 ? a.s[1].S : a.s[2].S)) + (int64_t)unit0 * lds;
  const float *zp = UZ ? (sg == 0 ? a.s[0].Z : (sg == 1 ? a.s[1].Z : a.s[2].Z)) + (int64_t)unit0 * lds
                       : nullptr;
  // paired mode: the W3 row of the same unit
  const uint8_t *wp3 = OUT == 2 ? a.s[1].W + (int64_t)unit0 * a.s[1].ldw : nullptr;
  const float *sp3 = OUT == 2 ? a.s[1].S + (int64_t)unit0 * a.s[1].lds : nullptr;
  const float *zp3 = OUT == 2 && UZ ? a.s[1].Z + (int64_t)unit0 * a.s[1].lds : nullptr;
  auto advance = [&]() {  // to the team's next unit
    wp += NTM * ldw;
    sp += NTM * lds;
    if constexpr (UZ) zp += NTM * lds;
    if constexpr (OUT == 2) {
      wp3 += NTM * a.s[1].ldw;
      sp3 += NTM * a.s[1].lds;
      if constexpr (UZ) zp3 += NTM * a.s[1].lds;
    }
  };
  // row i of the team into a window slot; rows are requested in order
  auto issue = [&](int slot, int i) {
    const bool odd = OUT == 2 && (i & 1);
    const float *srow = odd ? sp3 : sp;
    const uint8_t *wrow = odd ? wp3 : wp;
#pragma unroll
    for (int j = 0; j < C; j++) s[slot][j] = *(const float *)((const char *)srow + (uint32_t)(4u * (uint32_t)sgo[j]));
    if constexpr (UZ) {
      const float *zrow = odd ? zp3 : zp;
#pragma unroll
      for (int j = 0; j < C; j++) z[slot][j] = *(const float *)((const char *)zrow + (uint32_t)(4u * (uint32_t)sgo[j]));
    }
#pragma unroll
    for (int j = 0; j < C; j++) w[slot][j] = *(const uint4 *)(wrow + (uint32_t)(16u * (uint32_t)cj[j]));
    if (i + 1 < cnt && (OUT != 2 || odd)) advance();
  };
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int d = 0; d < D; d++) {
    issue(d, d);
    __builtin_amdgcn_sched_barrier(0);
  }
  if constexpr (CMB) {
    const int st = a.chs + 4, heads = K / a.chs;
    if ((int)threadIdx.x < heads) {  // e_s and 1/L of head threadIdx.x
      const int h = threadIdx.x;
      const float *w = a.cws + (int64_t)h * a.cmax * st + a.chs;
      float M = -INFINITY;
#pragma unroll
      for (int s = 0; s < kCmbRegs; s++)
        if (s < a.cn) M = fmaxf(M, cml[s].x);
      for (int s = kCmbRegs; s < a.cn; s++) M = fmaxf(M, w[s * st]);
      float L = 0.f;
#pragma unroll
      for (int s = 0; s < kCmbRegs; s++)
        if (s < a.cn) {
          const float e = expf(cml[s].x - M);
          L += e * cml[s].y;
          cef[h * a.cn + s] = e;
        }
      for (int s = kCmbRegs; s < a.cn; s++) {
        const float e = expf(w[s * st] - M);
        L += e * w[s * st + 1];
        cef[h * a.cn + s] = e;
      }
      cef[heads * a.cn + h] = 1.f / L;
    }
    lds_barrier();
#pragma unroll
    for (int ps = 0; ps < XP; ps++)
#pragma unroll
      for (int hf = 0; hf < 2; hf++) {
        const int e0 = 8 * min((int)threadIdx.x + NT * ps, ngrp8 - 1) + 4 * hf;
        const int h = e0 / a.chs;
        const float *ef = cef + h * a.cn;
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
        auto acc4 = [&](float e, float4 v) {
          o.x = fmaf(e, v.x, o.x);
          o.y = fmaf(e, v.y, o.y);
          o.z = fmaf(e, v.z, o.z);
          o.w = fmaf(e, v.w, o.w);
        };
#pragma unroll
        for (int s = 0; s < kCmbRegs; s++)
          if (s < a.cn) acc4(ef[s], cov[ps][hf][s]);
        const float *w = a.cws + (int64_t)h * a.cmax * st + (e0 - h * a.chs);
        for (int s = kCmbRegs; s < a.cn; s++) acc4(ef[s], *(const float4 *)(w + s * st));
        const float il = cef[heads * a.cn + h];
        const float4 x = make_float4(o.x * il, o.y * il, o.z * il, o.w * il);
        if (hf == 0) xa[0][ps] = x;
        else xb[0][ps] = x;
      }
  }

  // x -> limbs in LDS, one k-group of 8 elements per thread per pass
  float ss = 0.f;
#pragma unroll
  for (int pass = 0; pass < XP; pass++)
#pragma unroll
  for (int mv = 0; mv < MX; mv++) {
    const int g8 = (int)threadIdx.x + NT * pass;
    const float4 ya = xa[mv][pass], yb = xb[mv][pass];
    float4 ma = make_float4(0.f, 0.f, 0.f, 0.f), mb = ma;
    if constexpr (NORM) {
      ma = na[pass];
      mb = nb[pass];
    }
    float v[8] = {ya.x, ya.y, ya.z, ya.w, yb.x, yb.y, yb.z, yb.w};
    if constexpr (NORM) {
      if (g8 < ngrp8) {
#pragma unroll
        for (int k = 0; k < 8; k++) ss = fmaf(v[k], v[k], ss);
      }
      const float nv[8] = {ma.x, ma.y, ma.z, ma.w, mb.x, mb.y, mb.z, mb.w};
#pragma unroll
      for (int k = 0; k < 8; k++) v[k] *= nv[k];
    }
    // chunk maximum of |v| as an integer maximum of the magnitude bits: NaN
    // sorts above Inf above every finite value, so a NaN anywhere in the chunk
    // survives into m (fmaxf would drop it) and turns the chunk's factor into
    // NaN below, as the fp32 product of the reference propagates it
    uint32_t mbits = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) mbits = max(mbits, __float_as_uint(v[k]) & 0x7fffffffu);
    // the 4 k-groups of a chunk are lanes 4c..4c+3 of one wave
    mbits = max(mbits, (uint32_t)__builtin_amdgcn_mov_dpp((int)mbits, kDppXor1, 0xF, 0xF, false));
    mbits = max(mbits, (uint32_t)__builtin_amdgcn_mov_dpp((int)mbits, kDppXor2, 0xF, 0xF, false));
    const float m = __uint_as_float(mbits);
    int e;
    frexpf(m, &e);       // m < 2^e (e = 0 for m = 0)
    e = max(e, -100);    // chunks below 2^-101 keep fewer bits; 2^(e-22) stays normal
    const float sc = ldexpf(1.f, 22 - e);
    uint32_t u[8];
#pragma unroll
    for (int k = 0; k < 8; k++)  // fp32 bits of v*2^(22-e) + 1.5*2^23 hold round(v*2^(22-e)) + 2^22
      u[k] = __float_as_uint(fmaf(v[k], sc, 12582912.f)) - 0x4AB77778u;
    uint32_t L[6];
    limbs8(u, L);
    int si = 0;  // sum of the chunk's integers I (UZ): u = I + 0x888888
    if constexpr (UZ) {
#pragma unroll
      for (int k = 0; k < 8; k++) si += (int)u[k];
      si -= 8 * 0x888888;
      si += __builtin_amdgcn_mov_dpp(si, kDppXor1, 0xF, 0xF, false);
      si += __builtin_amdgcn_mov_dpp(si, kDppXor2, 0xF, 0xF, false);
    }
    if (g8 < ngrp8) {
      const int ch = g8 >> 2, dd = g8 & 3;
#pragma unroll
      for (int j = 0; j < 6; j++) xl[(mv * nchunk + ch) * 24 + 4 * j + dd] = L[j];
      if (dd == 0) {
        // Inf or NaN in the chunk: NaN (the limbs of such a chunk are meaningless)
        const float fe = (m <= 3.4e38f) ? ldexpf(1.f, e - 22) : __int_as_float(0x7fc00000);
        xf[mv * nchunk + ch] = fe;
        if constexpr (UZ) xs[mv * nchunk + ch] = (float)si * fe;
      }
    }
  }
  if constexpr (NORM) {
    ss = wave_sum_dpp(ss);
    if (lane == 0) ssq[wave] = ss;
  }
  lds_barrier();
  float rs = 1.f;
  if constexpr (NORM) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < NW; i++) t += ssq[i];
    rs = 1.f / sqrtf(t / (float)K + a.eps);
  }
  uint32_t L[MX][C][6][4];
  float f[MX][C];
  float fs[UZ ? MX : 1][UZ ? C : 1];
#pragma unroll
  for (int mv = 0; mv < MX; mv++)
#pragma unroll
  for (int j = 0; j < C; j++) {
#pragma unroll
    for (int q = 0; q < 6; q++) {
      const uint4 t = *(const uint4 *)&xl[(mv * nchunk + cj[j]) * 24 + 4 * q];
      L[mv][j][q][0] = t.x;
      L[mv][j][q][1] = t.y;
      L[mv][j][q][2] = t.z;
      L[mv][j][q][3] = t.w;
    }
    f[mv][j] = xf[mv * nchunk + cj[j]];
    if constexpr (UZ) fs[mv][j] = xs[mv * nchunk + cj[j]];
  }

  // rows 0 .. RM-1 unrolled (cnt <= RM); row i + D is requested right after
  // row i is consumed; requests past cnt repeat the last row (cache hits)
  float p[MX][RM];
#pragma unroll
  for (int i = 0; i < RM; i++) {
    const int slot = i % D;
    float acc[MX];
#pragma unroll
    for (int mv = 0; mv < MX; mv++) acc[mv] = 0.f;
    if (i < cnt) {
#pragma unroll
      for (int j = 0; j < C; j++)
#pragma unroll
      for (int mv = 0; mv < MX; mv++) {
        uint4 wd = w[slot][j];
        if constexpr (UZ) {  // unsigned u -> signed u - 8
          wd.x ^= 0x88888888u;
          wd.y ^= 0x88888888u;
          wd.z ^= 0x88888888u;
          wd.w ^= 0x88888888u;
        }
        // Horner over the limbs, most significant first
        int T = 0;
#pragma unroll
        for (int q = 5; q >= 0; q--) {
          if (q < 5) T = (int)((uint32_t)T << 4);
          T = __builtin_amdgcn_sdot8((int)wd.x, (int)L[mv][j][q][0], T, false);
          T = __builtin_amdgcn_sdot8((int)wd.y, (int)L[mv][j][q][1], T, false);
          T = __builtin_amdgcn_sdot8((int)wd.z, (int)L[mv][j][q][2], T, false);
          T = __builtin_amdgcn_sdot8((int)wd.w, (int)L[mv][j][q][3], T, false);
        }
        acc[mv] = fmaf(aj[j] ? s[slot][j] * f[mv][j] : 0.f, (float)T, acc[mv]);
        if constexpr (UZ)
          acc[mv] = fmaf(aj[j] ? fmaf(8.f, s[slot][j], z[slot][j]) : 0.f, fs[mv][j], acc[mv]);
      }
    }
#pragma unroll
    for (int mv = 0; mv < MX; mv++) p[mv][i] = acc[mv];
    if (i + D < RM) {
      __builtin_amdgcn_sched_barrier(0);
      issue(slot, i + D);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int mv = 0; mv < MX; mv++) rows_reduce<RM>(p[mv], lane);
  // lanes (64/RM)*i .. hold the wave's total of row i of the team
  constexpr int LB = RM >= 64 ? 6 : RM >= 32 ? 5 : RM >= 16 ? 4 : RM >= 8 ? 3 : RM >= 4 ? 2 : 1;
  constexpr int GL = 1 << (6 - LB);  // lanes per row after the reduction
  const int ir = lane >> (6 - LB);
  if constexpr (MX > 1 && KT == 1) {
    if ((lane & (GL - 1)) == 0 && ir < cnt) {
#pragma unroll
      for (int mv = 0; mv < MX; mv++)
        if (mv < a.mx) a.s[0].out[mv * a.ldo + ub + team + NTM * ir] = p[mv][0];
    }
    return;
  } else if constexpr (KT == 1) {
    // one wave per row: the writer lanes store the outputs directly (stored
    // after the loop, so no store waits on a weight load in flight)
    const float v = p[0][0] * rs;
    if constexpr (OUT == 2) {
      const float h3 = __shfl_down(v, GL);  // row ir + 1: the W3 half of the pair
      if ((lane & (2 * GL - 1)) == 0 && ir < cnt)
        a.s[0].out[ub + team + NTM * (ir >> 1)] = silu_mul(v, h3);
    } else if ((lane & (GL - 1)) == 0 && ir < cnt) {
      float *o = (sg == 0 ? a.s[0].out : (sg == 1 ? a.s[1].out : a.s[2].out)) + ub + team + NTM * ir;
      *o = OUT == 1 ? *o + v : v;
    }
    return;
  }
  // KT waves per row: the wave totals meet in LDS, summed in wave order
  if ((lane & (GL - 1)) == 0 && ir < cnt) {
#pragma unroll
    for (int mv = 0; mv < MX; mv++) red[(wave * MX + mv) * RM + ir] = p[mv][0];
  }
  lds_barrier();
  const int nu = ue - ub;
  if constexpr (MX > 1) {
    for (int q = threadIdx.x; q < nu * MX; q += NT) {
      const int mv = q / nu, qq = q - mv * nu;
      const int t = qq % NTM, iu = qq / NTM, unit = ub + qq;
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < KT; k++) acc += red[((t * KT + k) * MX + mv) * RM + iu];
      if (mv < a.mx) a.s[0].out[mv * a.ldo + unit] = acc;
    }
    return;
  }
  for (int q = threadIdx.x; q < nu; q += NT) {
    const int t = q % NTM, iu = q / NTM, unit = ub + q;
    float h[UPR];
#pragma unroll
    for (int sub = 0; sub < UPR; sub++) {
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < KT; k++) acc += red[(t * KT + k) * MX * RM + iu * UPR + sub];
      h[sub] = acc * rs;
    }
    if constexpr (OUT == 2) {
      a.s[0].out[unit] = silu_mul(h[0], h[UPR - 1]);
    } else {
      float *o = (sg == 0 ? a.s[0].out : (sg == 1 ? a.s[1].out : a.s[2].out)) + unit;
      *o = OUT == 1 ? *o + h[0] : h[0];
    }
  }
}

template <int C, int KT, int NW, int D, int RM, bool UZ>
void launch_modes(const W4D8Args &a, int G, size_t shm, hipStream_t st) {
  if (a.cws) {  // x from attention partials (checked by launch_w4d8: plain accumulate)
    hipLaunchKernelGGL((w4d8_gemv<C, KT, NW, D, RM, false, 1, false, 1, UZ, true>), dim3((unsigned)G),
                       dim3(64 * NW), shm, st, a);
    return;
  }
  const bool norm = a.nw != nullptr;
#define L8(NORMV, OUTV, MV)                                                                       \
  hipLaunchKernelGGL((w4d8_gemv<C, KT, NW, D, RM, NORMV, OUTV, MV, 1, UZ>), dim3((unsigned)G), dim3(64 * NW), \
                     shm, st, a)
  const bool multi = a.out_mode != 2 && a.n > 1;
  if (norm) {
    if (a.out_mode == 2) L8(true, 2, false);
    else if (multi) L8(true, 0, true);
    else L8(true, 0, false);
  } else {
    if (a.out_mode == 1) L8(false, 1, false);
    else if (multi) L8(false, 0, true);
    else L8(false, 0, false);
  }
#undef L8
}

template <int C, int KT, int NW, int D, int RM, int MX = 1>
int launch_rm(const W4D8Args &a, int G, hipStream_t st) {
  const int nchunk = a.K / 32;
  const bool uz = a.s[0].Z != nullptr;
  const size_t cmb = a.cws ? (size_t)(a.K / a.chs) * (a.cn + 1) : 0;  // e_s and 1/L per head
  const size_t shm = sizeof(float) * ((size_t)(uz ? 26 : 25) * MX * nchunk + NW + (size_t)NW * MX * RM + cmb);
  if (shm > 160 * 1024) return set_error(SIMP_RT_EUNSUPPORTED, "w4d8: K=%d too large", a.K);
  KernelTimer kt(st, "w4s_gemv_d8");
  if constexpr (MX > 1) {
    hipLaunchKernelGGL((w4d8_gemv<C, KT, NW, D, RM, false, 0, false, MX, false>), dim3((unsigned)G),
                       dim3(64 * NW), shm, st, a);
  } else if (uz) {
    launch_modes<C, KT, NW, D, RM, true>(a, G, shm, st);
  } else {
    launch_modes<C, KT, NW, D, RM, false>(a, G, shm, st);
  }
  SIMP_HIP(hipGetLastError());
  return SIMP_RT_OK;
}

// Blocks: at least one per CU, and enough that a team has at most 16 rows
// (about 16 rows per team streams best; caps of 24 and 32 with fewer blocks
// measured 2-3% slower on the 3B W4 decode, and a cap of 8 with more blocks
// slower too: 3200->8640 6.7 against 6.1 us).
template <int C, int KT, int NW, int D, int MX = 1>
int launch_cfg(W4D8Args a, hipStream_t st) {
  constexpr int teams = NW / KT;
  const int upr = a.out_mode == 2 ? 2 : 1;
  const int nseg = a.out_mode == 2 ? 1 : a.n;
  int64_t total = 0;
  for (int i = 0; i < nseg; i++) total += a.s[i].rows;
  // Whole rounds of blocks: a count just past a multiple of the CU count
  // leaves a few CUs with one block more than the rest, and the launch lasts
  // as long as they do (3B W4 decode: W1|W3 at 270 and QKV at 258 blocks;
  // 966 -> 1047 tok/s with 512 and 256; at least two rounds measured slower).
  // Segments take blocks in proportion to their rows, at least enough for 16
  // rows per team; the remainder goes one by one to the segments in order.
  const int64_t cus = num_cus();
  int64_t G0 = std::max<int64_t>(cus, cdiv(total * upr, (int64_t)teams * 16));
  G0 = cdiv(G0, cus) * cus;
  int nb[3] = {0, 0, 0}, G = 0;
  int64_t rows = 0;  // rows per team at most
  int64_t rem = G0;
  for (int i = 0; i < nseg; i++) {
    const int64_t u = a.s[i].rows;
    int64_t b = std::max<int64_t>(G0 * u / total, cdiv(u * upr, (int64_t)teams * 16));
    b = std::max<int64_t>(1, std::min<int64_t>(b, u));
    nb[i] = (int)b;
    rem -= b;
  }
  for (bool more = true; rem > 0 && more;) {
    more = false;
    for (int i = 0; i < nseg && rem > 0; i++)
      if (nb[i] < a.s[i].rows) {
        nb[i]++;
        rem--;
        more = true;
      }
  }
  for (int i = 0; i < nseg; i++) {
    G += nb[i];
    rows = std::max<int64_t>(rows, cdiv(cdiv((int64_t)a.s[i].rows, nb[i]), teams) * upr);
  }
  a.bstart[0] = 0;
  a.bstart[1] = nseg > 1 ? nb[0] : INT32_MAX;
  a.bstart[2] = nseg > 2 ? nb[0] + nb[1] : INT32_MAX;
  if (rows <= 8) return launch_rm<C, KT, NW, D, 8, MX>(a, G, st);
  if (rows <= 16) return launch_rm<C, KT, NW, D, 16, MX>(a, G, st);
  return set_error(SIMP_RT_EUNSUPPORTED, "w4d8: %lld rows per team", (long long)rows);
}

}  // namespace

bool w4d8_supported(int K, int gs, const void *x0, const void *nw) {
  return K > 0 && K % 32 == 0 && gs > 0 && gs % 32 == 0 && K % gs == 0 && K / 32 <= 640 &&
         ((uintptr_t)x0 & 15) == 0 && ((uintptr_t)nw & 15) == 0;
}

int launch_w4d8(const W4D8Args &a, hipStream_t st) {
  if (!w4d8_supported(a.K, a.gs, a.x0, a.nw) || a.n < 1 || a.n > 3 ||
      (a.out_mode == 2 && a.n != 2))
    return set_error(SIMP_RT_EINVAL, "w4d8: unsupported arguments (K=%d gs=%d)", a.K, a.gs);
  for (int i = 0; i < (a.out_mode == 2 ? 1 : a.n); i++)
    if (a.s[i].rows <= 0) return set_error(SIMP_RT_EINVAL, "w4d8: empty segment");
  for (int i = 1; i < a.n; i++)
    if ((a.s[i].Z != nullptr) != (a.s[0].Z != nullptr))
      return set_error(SIMP_RT_EINVAL, "w4d8: zeros on some segments only");
  if (a.s[0].Z && a.mx > 1) return set_error(SIMP_RT_EINVAL, "w4d8: zeros with several x vectors");
  if (a.cws && (a.n != 1 || a.out_mode != 1 || a.nw || a.mx > 1 || a.chs <= 0 || a.chs % 4 ||
                a.K % a.chs || a.K / a.chs > 256 || a.cn < 1 || a.cn > a.cmax))
    return set_error(SIMP_RT_EINVAL, "w4d8: attention partials need one accumulating segment");
  const int nchunk = a.K / 32;
  if (a.mx > 1) {
    // several x vectors: one chunk per lane (the limbs of every vector stay in
    // registers), more waves per row instead
    if (a.n != 1 || a.out_mode != 0 || a.nw || a.mx > 4 || (a.ldx & 3) != 0)
      return set_error(SIMP_RT_EINVAL, "w4d8: several x vectors need one plain segment");
    // (8 rows in flight per team measured slower at every shape)
    if (a.mx == 2) {
      if (nchunk <= 64) return launch_cfg<1, 1, 4, 4, 2>(a, st);
      if (nchunk <= 128) return launch_cfg<1, 2, 8, 4, 2>(a, st);
      if (nchunk <= 192) return launch_cfg<1, 3, 6, 4, 2>(a, st);
      if (nchunk <= 320) return launch_cfg<1, 5, 10, 4, 2>(a, st);
      return launch_cfg<1, 10, 10, 4, 2>(a, st);
    }
    if (nchunk <= 64) return launch_cfg<1, 1, 4, 4, 4>(a, st);
    if (nchunk <= 128) return launch_cfg<1, 2, 8, 4, 4>(a, st);
    if (nchunk <= 192) return launch_cfg<1, 3, 6, 4, 4>(a, st);
    if (nchunk <= 320) return launch_cfg<1, 5, 10, 4, 4>(a, st);
    return launch_cfg<1, 10, 10, 4, 4>(a, st);
  }
  // x from attention partials: twice the waves per block, so each thread
  // combines half as many x elements in the prologue (3B W4 decode Wo:
  // 1068 -> 1087 tok/s; the same form for the other K = 3200 GEMVs measured
  // equal or slower, and 2-6 rows in flight or 16 waves slower here)
  if (a.cws && nchunk > 64 && nchunk <= 128) return launch_cfg<1, 2, 8, 4>(a, st);
  if (nchunk <= 64) return launch_cfg<1, 1, 4, 4>(a, st);
  if (nchunk <= 128) return launch_cfg<2, 1, 4, 4>(a, st);
  if (nchunk <= 192) return launch_cfg<1, 3, 6, 4>(a, st);
  if (nchunk <= 320) return launch_cfg<1, 5, 10, 4>(a, st);
  return launch_cfg<2, 5, 10, 4>(a, st);
}

}  // namespace simp
