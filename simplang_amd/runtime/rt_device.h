// rt_device.h -- device helpers shared by the kernels of libsimp_hip.so.
#pragma once

#include <hip/hip_runtime.h>

namespace simp {

// Sum over the 64 lanes of a wave (result in every lane).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = fmaxf(v, __shfl_xor(v, d));
  return v;
}

// Cross-lane moves that stay in the VALU (no LDS round trip, unlike
// __shfl_xor's ds_bpermute): DPP quad permutes and row mirrors/rotations, and
// gfx950's v_permlane{16,32}_swap.  Lane layouts were checked on the device.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppHalfMirror = 0x141; // within 8 lanes: i <-> 7 - i (= lane ^ 7)
constexpr int kDppMirror = 0x140;     // within 16 lanes: i <-> 15 - i
constexpr int kDppRor8 = 0x128;       // within 16 lanes: i <- i + 8 (= lane ^ 8)
// a' = rows (a0, b0, a2, b2), b' = rows (a1, b1, a3, b3) of 16 lanes
__device__ __forceinline__ void permlane16_swap(float &a, float &b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
// a' = halves (a_lo, b_lo), b' = halves (a_hi, b_hi) of 32 lanes
__device__ __forceinline__ void permlane32_swap(float &a, float &b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
// Sum / max over the 64 lanes, every lane gets the result (VALU only).
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_mov<kDppXor1>(v);
  v += dpp_mov<kDppXor2>(v);
  v += dpp_mov<kDppHalfMirror>(v);
  v += dpp_mov<kDppMirror>(v);
  float a = v, b = v;
  permlane16_swap(a, b);
  v = a + b;
  a = v;
  b = v;
  permlane32_swap(a, b);
  return a + b;
}
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_mov<kDppXor1>(v));
  v = fmaxf(v, dpp_mov<kDppXor2>(v));
  v = fmaxf(v, dpp_mov<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_mov<kDppMirror>(v));
  float a = v, b = v;
  permlane16_swap(a, b);
  v = fmaxf(a, b);
  a = v;
  b = v;
  permlane32_swap(a, b);
  return fmaxf(a, b);
}

// Workgroup barrier for LDS traffic only: this wave's LDS operations complete
// (lgkmcnt(0)), then s_barrier.  __syncthreads() also waits for every
// outstanding global load of the wave (its fence drains vmcnt), which would
// stall loads a kernel issued early on purpose; this one leaves them in flight.
// It orders LDS only: global memory written before it is not made visible to
// the other waves.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt untouched
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ---- LDS-DMA rings (the int8 and fp32 GEMM kernels)

// s_waitcnt immediate that waits for vmcnt <= n only (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima).
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
// s_waitcnt immediate that waits for lgkmcnt == 0 only.
constexpr int waitcnt_lgkm0 = 15 | (3 << 14) | (7 << 4);

// s_waitcnt vmcnt(D * n) for a run-time n in 0..Q (the immediate must be a constant)
template <int D, int Q>
__device__ __forceinline__ void wait_vm_le(int n) {
  if constexpr (Q >= 0) {
    if (n == Q) __builtin_amdgcn_s_waitcnt(waitcnt_vm(D * Q));
    else wait_vm_le<D, Q - 1>(n);
  }
}

// One global_load_lds_dwordx4: each lane's 16 bytes at `src` land in LDS at
// lds_off + 16*lane.  Issued as asm because the compiler, seeing the builtin's
// LDS write, waits for every outstanding load before any later LDS read; the
// kernels count these loads with their own s_waitcnt instead.
__device__ __forceinline__ void dma16(const void *src, uint32_t lds_off) {
  uint32_t saved;
  // M0 is saved and restored around the load (the compiler owns it); one wait
  // state separates the M0 write from the LDS-DMA load that reads it.
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(__builtin_amdgcn_readfirstlane(lds_off)), "v"(src)
      : "memory");
}

// LDS byte offset of a shared-memory pointer.
__device__ __forceinline__ uint32_t lds_offset(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)p;
}

// s_barrier alone: no wait for this wave's outstanding loads or LDS operations
// (the caller's s_waitcnt says which must have landed).
__device__ __forceinline__ void block_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Maps the hardware workgroup id to a C tile: XCD-contiguous (workgroups are
// dispatched round-robin over the 8 XCDs), then in groups of 8 tile rows so
// that co-resident tiles share operand lines in their XCD's L2.  (int8 GEMM,
// 256x256 tiles, 8192^3: groups of 4 ran level with 8, groups of 2, 16 and 32
// 2-5% slower.)
__device__ __forceinline__ void tile_of_block(int bid, int nb, int tiles_m, int tiles_n,
                                              int &tm, int &tn) {
  const int q = nb >> 3, r = nb & 7, xcd = bid & 7, local = bid >> 3;
  const int t = xcd * q + min(xcd, r) + local;
  constexpr int G = 8;
  const int gsz = G * tiles_n;
  const int g = t / gsz, first = g * G;
  const int gm = min(tiles_m - first, G);
  const int w = t - g * gsz;
  tm = first + w % gm;
  tn = w / gm;
}

// block_sum through LDS with lds_barrier(): global loads stay in flight.
// DPP: the wave sums by DPP and permlane swaps (VALU only) instead of
// __shfl_xor; a different summation order, so each caller keeps the one its
// tests pin.
template <bool DPP = false>
__device__ __forceinline__ float block_sum_lds(float v, float *scratch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  v = DPP ? wave_sum_dpp(v) : wave_sum(v);
  lds_barrier();  // scratch may still be read by a previous call
  if (lane == 0) scratch[wave] = v;
  lds_barrier();
  float t = 0.f;
  for (int i = 0; i < nw; i++) t += scratch[i];
  return t;
}
template <bool DPP = false>
__device__ __forceinline__ float block_max_lds(float v, float *scratch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  v = DPP ? wave_max_dpp(v) : wave_max(v);
  lds_barrier();
  if (lane == 0) scratch[wave] = v;
  lds_barrier();
  float t = scratch[0];
  for (int i = 1; i < nw; i++) t = fmaxf(t, scratch[i]);
  return t;
}

// Block-wide sum for blockDim.x <= 1024 (multiple of 64); every thread gets the
// result.  `scratch` holds at least 16 floats of LDS; it is reused on return.
__device__ __forceinline__ float block_sum(float v, float *scratch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  v = wave_sum(v);
  __syncthreads();  // scratch may still be read by a previous call
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; i++) t += scratch[i];
  return t;
}

__device__ __forceinline__ float block_max(float v, float *scratch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  v = wave_max(v);
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float t = scratch[0];
  for (int i = 1; i < nw; i++) t = fmaxf(t, scratch[i]);
  return t;
}

// Byte I of x as float in one v_cvt_f32_ubyte{I} (the compiler would emit a
// bitfield extract plus ubyte0 for the equivalent shift-and-mask).
template <int I>
__device__ __forceinline__ float ubyte(uint32_t x) {
  float r;
  if constexpr (I == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(x));
  else if constexpr (I == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(x));
  else if constexpr (I == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(x));
  else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(x));
  return r;
}

// Streaming (nontemporal) 16-byte loads for data read once per call (weight
// streams), so they do not displace reused data in the caches.
__device__ __forceinline__ uint4 ntload16(const void *p) {
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load((const u32x4 *)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 ntload_f4(const float4 *p) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const f32x4 v = __builtin_nontemporal_load((const f32x4 *)p);
  return make_float4(v.x, v.y, v.z, v.w);
}

// Group index of 32-weight chunk c for a group size of 32 * cpg: a shift when
// cpg is a power of two (cpg_shift = log2(cpg), else -1), since a 32-bit
// integer division costs about twenty VALU instructions per use.
__device__ __forceinline__ int chunk_group(int c, int cpg, int cpg_shift) {
  return cpg_shift >= 0 ? c >> cpg_shift : c / cpg;
}
__device__ __forceinline__ int cpg_log2(int cpg) {
  return (cpg & (cpg - 1)) == 0 ? __builtin_ctz((unsigned)cpg) : -1;
}

// Unpacks the 32 nibbles of a 16-byte chunk into u[0..31] (u[k] = nibble k).
__device__ __forceinline__ void unpack32(uint4 w, float (&u)[32]) {
  const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t lo = d[i] & 0x0F0F0F0Fu, hi = (d[i] >> 4) & 0x0F0F0F0Fu;
    u[8 * i + 0] = ubyte<0>(lo);
    u[8 * i + 1] = ubyte<0>(hi);
    u[8 * i + 2] = ubyte<1>(lo);
    u[8 * i + 3] = ubyte<1>(hi);
    u[8 * i + 4] = ubyte<2>(lo);
    u[8 * i + 5] = ubyte<2>(hi);
    u[8 * i + 6] = ubyte<3>(lo);
    u[8 * i + 7] = ubyte<3>(hi);
  }
}

}  // namespace simp
