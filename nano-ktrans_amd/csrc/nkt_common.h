// Device helpers shared by the MoE kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nkt {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr int kMaxExperts = 256;  // router: at most 4 logits per lane
constexpr int kMaxTopK = 16;
// route + group in one workgroup up to this many tokens / (token, slot) pairs
constexpr int kFusedRouteMaxTokens = 64;
constexpr int kFusedRouteMaxPairs = 1024;

// Weight formats (values match NKT_WEIGHT_* in include/nkt_moe.h).
enum WeightFormat : int { WF_F32 = 0, WF_BF16 = 1, WF_I8 = 2, WF_I4 = 3 };

// ---------------------------------------------------------------------------
// bf16 <-> fp32
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u | 0x00400000u) >> 16;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ float bf16_round(float f) {
  return __uint_as_float(f32_to_bf16_bits(f) << 16);
}

// Two floats -> packed bf16 pair (lo = a, hi = b), round to nearest even.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return f32_to_bf16_bits(a) | (f32_to_bf16_bits(b) << 16);
}

// ---------------------------------------------------------------------------
// Router exp.  x = n*ln2 + r with a Cody & Waite two-constant reduction
// (fused multiply-adds), exp(r) by the degree-7 Taylor polynomial 1/k! in
// Horner form (|r| <= ln2/2, truncation below 0.1 ulp), then an exact
// power-of-two scaling; below 2^-126 the scaling is split in two so a
// subnormal result is rounded once.  Every operation is a single IEEE
// operation, so the host oracle reproduces the result bit for bit.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float route_expf(float x) {
#pragma clang fp contract(off)
  if (x != x) return x;
  if (x > 89.0f) return __builtin_huge_valf();
  if (x < -110.0f) x = -110.0f;
  const float t = x * 0x1.715476p+0f;
  const float n = __builtin_rintf(t);
  float r = __builtin_fmaf(-n, 0x1.62e430p-1f, x);
  r = __builtin_fmaf(-n, -0x1.05c610p-29f, r);
  float p = 0x1.a01a02p-13f;
  p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
  p = __builtin_fmaf(p, r, 0x1.111112p-7f);
  p = __builtin_fmaf(p, r, 0x1.555556p-5f);
  p = __builtin_fmaf(p, r, 0x1.555556p-3f);
  p = __builtin_fmaf(p, r, 0x1.000000p-1f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const int ni = (int)n;
  if (ni > 127) return (p * __uint_as_float(254u << 23)) * 2.0f;
  if (ni >= -126) return p * __uint_as_float((uint32_t)(ni + 127) << 23);
  return (p * __uint_as_float((uint32_t)(ni + 127 + 64) << 23)) *
         __uint_as_float((uint32_t)(127 - 64) << 23);
}

// ---------------------------------------------------------------------------
// wave reductions (64 lanes, xor butterfly)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

__device__ __forceinline__ float wave_sum_butterfly(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    uint32_t lo = __shfl_xor((uint32_t)v, off);
    uint32_t hi = __shfl_xor((uint32_t)(v >> 32), off);
    uint64_t o = ((uint64_t)hi << 32) | lo;
    v = o > v ? o : v;
  }
  return v;
}

// Inclusive prefix sum over the 64 lanes (Hillis-Steele).
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    int o = __shfl_up(v, off);
    if (lane >= off) v += o;
  }
  return v;
}

// ---------------------------------------------------------------------------
// weight dequantisation into MFMA A operands (exact bf16 integers)
//   int4: one u32 holds 8 nibbles in MFMA column order (nibble j<4 -> column
//         2j, j>=4 -> 2(j-4)+1); step s of dq_i4(w >> 4s) gives bf16 128 + n
//         for columns 2s', 2s'+1 pairs (n = stored nibble = q + 8).
//   int8: two u32 hold 8 bytes (stored q + 128) -> 8 bf16 values 0..255.
// ---------------------------------------------------------------------------
__device__ __forceinline__ u32x4 dq_i4(uint32_t w) {
  u32x4 a;
  a[0] = (w & 0x000F000Fu) | 0x43004300u;
  a[1] = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
  a[2] = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
  a[3] = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
  return a;
}

__device__ __forceinline__ uint32_t bf16pair_u8(uint32_t w, int lo_byte) {
  const float f0 = (float)((w >> (8 * lo_byte)) & 0xffu);
  const float f1 = (float)((w >> (8 * lo_byte + 8)) & 0xffu);
  return __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
}

__device__ __forceinline__ u32x4 dq_i8(uint32_t w0, uint32_t w1) {
  u32x4 a;
  a[0] = bf16pair_u8(w0, 0);
  a[1] = bf16pair_u8(w0, 2);
  a[2] = bf16pair_u8(w1, 0);
  a[3] = bf16pair_u8(w1, 2);
  return a;
}

__device__ __forceinline__ f32x4 bf16x4_to_f32(u32x2 v) {
  return f32x4{__uint_as_float(v[0] << 16), __uint_as_float(v[0] & 0xffff0000u),
               __uint_as_float(v[1] << 16), __uint_as_float(v[1] & 0xffff0000u)};
}

__device__ __forceinline__ float silu_f32(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS
// operations, not for its outstanding global loads (a full __syncthreads
// fence would also drain the weight prefetch).
__device__ __forceinline__ void lds_barrier() {
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt, expcnt untouched
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}

// ---------------------------------------------------------------------------
// MFMA wrappers (gfx950)
//   16x16x32 bf16: lane l supplies A[l%16][8*(l/16) .. +7] and
//   B[8*(l/16) .. +7][l%16]; D[4*(l/16)+v][l%16] lands in register v.
//   16x16x4 f32:   lane l supplies A[l%16][l/16] and B[l/16][l%16].
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x4 mfma_bf16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

}  // namespace nkt
