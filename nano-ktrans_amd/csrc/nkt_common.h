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

// round to nearest even; NaN stays NaN (quiet bit set); both results are
// formed and one selected (no branch)
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t quiet = (u | 0x00400000u) >> 16;
  return (u & 0x7fffffffu) > 0x7f800000u ? quiet : rounded;
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
  // every case is computed and one selected (no divergent branches); the
  // argument is kept finite where its result is selected away
  const bool nan = x != x;
  const bool big = x > 89.0f;
  float xc = x < -110.0f ? -110.0f : x;
  xc = (nan || big) ? 0.0f : xc;
  const float t = xc * 0x1.715476p+0f;
  const float n = __builtin_rintf(t);
  float r = __builtin_fmaf(-n, 0x1.62e430p-1f, xc);
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
  const float hi = (p * __uint_as_float(254u << 23)) * 2.0f;                       // ni > 127
  const float mid = p * __uint_as_float((uint32_t)(ni + 127) << 23);               // -126 <= ni <= 127
  const float lo = (p * __uint_as_float((uint32_t)(ni + 127 + 64) << 23)) *        // ni < -126
                   __uint_as_float((uint32_t)(127 - 64) << 23);
  float y = ni > 127 ? hi : (ni >= -126 ? mid : lo);
  y = big ? __builtin_huge_valf() : y;
  return nan ? x : y;
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

// ---------------------------------------------------------------------------
// Lane moves without the LDS crossbar: DPP within 16-lane rows and the
// gfx950 half / row swaps (a few cycles each instead of a ds_bpermute).
// DPP controls used: row_shl:n = 0x100 + n (lane i reads lane i + n of its
// row), row_shr:n = 0x110 + n (reads i - n), row_bcast:15 = 0x142 (lane 15
// of each row to the next row), row_bcast:31 = 0x143 (lane 31 to rows 2, 3).
// Lanes with no source lane, or in rows outside ROW_MASK, read 0.
// ---------------------------------------------------------------------------
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xf, false);
}

// v(l) + v(l ^ 32) and v(l) + v(l ^ 16) in every lane (a swap of the wave's
// halves / of neighbouring rows puts each lane's partner beside it).
__device__ __forceinline__ float add_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum of the 64 lanes by the halving tree: level off = 32, 16, ..., 1 adds
// lane l + off into lane l (l < off); the total of lane 0, as a uniform
// value.  (The same order as wave_sum_butterfly's lane 0.)
__device__ __forceinline__ float wave_sum_tree(float v) {
  v = add_xor32(v);
  v = add_xor16(v);
  v = v + __uint_as_float(dpp_u32<0x108>(__float_as_uint(v)));
  v = v + __uint_as_float(dpp_u32<0x104>(__float_as_uint(v)));
  v = v + __uint_as_float(dpp_u32<0x102>(__float_as_uint(v)));
  v = v + __uint_as_float(dpp_u32<0x101>(__float_as_uint(v)));
  return __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 0));
}

// Maximum over the 64 lanes (fmaxf: NaN inputs are ignored unless all are
// NaN), as a uniform value.
__device__ __forceinline__ float wave_max_tree(float v) {
  {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  // within the row: lanes past the row's end read 0, which only reaches
  // lanes whose result is not used (lane 0 always reads real lanes)
  v = fmaxf(v, __uint_as_float(dpp_u32<0x108>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<0x104>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<0x102>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<0x101>(__float_as_uint(v))));
  return __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 0));
}

// Inclusive prefix sum over the 64 lanes: shifted adds inside each row, then
// the row totals carried across rows (row_bcast).
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  v += (int)dpp_u32<0x111>((uint32_t)v);
  v += (int)dpp_u32<0x112>((uint32_t)v);
  v += (int)dpp_u32<0x114>((uint32_t)v);
  v += (int)dpp_u32<0x118>((uint32_t)v);
  v += (int)dpp_u32<0x142, 0xa>((uint32_t)v);
  v += (int)dpp_u32<0x143, 0xc>((uint32_t)v);
  return v;
}

// ---------------------------------------------------------------------------
// weight dequantisation into MFMA A operands (exact bf16 integers)
//   int4: one u32 holds 8 nibbles in MFMA column order (nibble j<4 -> column
//         2j, j>=4 -> 2(j-4)+1); step s of dq_i4(w >> 4s) gives bf16 128 + n
//         for columns 2s', 2s'+1 pairs (n = stored nibble = q + 8).
//   int8: two u32 hold 8 bytes (stored q + 128) -> 8 bf16 values 0..255.
// ---------------------------------------------------------------------------
// int4 dequantisation with v_and_or_b32: (w >> 4j) & 0x000F000F | 0x43004300
// in one instruction after the shift (the mask comes from an SGPR, the bf16
// exponent bits from a VGPR: one constant-bus read per instruction).
struct DqConst {
  uint32_t mask;  // SGPR: 0x000F000F
  uint32_t bits;  // VGPR: 0x43004300
};

__device__ __forceinline__ DqConst dq_const() {
  DqConst k;
  __asm__ volatile("s_mov_b32 %0, 0xf000f" : "=s"(k.mask));
  __asm__ volatile("v_mov_b32 %0, 0x43004300" : "=v"(k.bits));
  return k;
}

// (w >> SH) & mask | bits; the shift sits inside the same statement so that
// nothing of the dequantisation can move away from the constants' block
template <int SH>
__device__ __forceinline__ uint32_t dq_word(uint32_t w, const DqConst& k) {
  uint32_t r;
  if (SH == 0)
    __asm__("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(w), "s"(k.mask), "v"(k.bits));
  else
    __asm__("v_lshrrev_b32 %0, %4, %1\n\tv_and_or_b32 %0, %0, %2, %3"
            : "=&v"(r)
            : "v"(w), "s"(k.mask), "v"(k.bits), "i"(SH));
  return r;
}

__device__ __forceinline__ u32x4 dq_i4_k(uint32_t w, const DqConst& k) {
  return u32x4{dq_word<0>(w, k), dq_word<4>(w, k), dq_word<8>(w, k), dq_word<12>(w, k)};
}

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

// int8 for the fp16 matrix cores: stored byte u -> fp16 1024 + u (bits
// 0x6400 | u, exact), one byte permute per pair; same element order as dq_i8.
__device__ __forceinline__ u32x4 dq_i8_f16(uint32_t w0, uint32_t w1) {
  return u32x4{__builtin_amdgcn_perm(0x64646464u, w0, 0x04010400u), __builtin_amdgcn_perm(0x64646464u, w0, 0x04030402u),
               __builtin_amdgcn_perm(0x64646464u, w1, 0x04010400u), __builtin_amdgcn_perm(0x64646464u, w1, 0x04030402u)};
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

// Direct-to-LDS loads (global_load_lds): lane l's 16 (4) bytes from src land
// at dst + 16 l (dst + 4 l); dst must be the same in every lane.  Waited for
// with the vector-memory counter.
__device__ __forceinline__ void load16_to_lds(const void* src, uint8_t* dst) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
}
__device__ __forceinline__ void load4_to_lds(const void* src, uint8_t* dst) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)dst, 4, 0, 0);
}

// Waits for every vector-memory load of this wave (direct-to-LDS ones
// included) before the LDS is read.
__device__ __forceinline__ void wait_vmem() {
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
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

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f32x4 mfma_f16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                 0, 0);
}

__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// K4 for token t by one whole wave: sigmoid(x[t] . g) (fp32 products and
// sums in a fixed order: each lane's strided share, then the butterfly), the
// value in every lane.  The shared-gate kernel and the single-token layer's
// gate_up launch both call it, so they give the same bits.
__device__ __forceinline__ float shared_gate_value(const void* __restrict__ x, const void* __restrict__ gw,
                                                   int act_bf16, int t, int H, int lane) {
  float s = 0.f;
  if (act_bf16 && H % 8 == 0) {
    // 8 bf16 per lane per 16-byte load, four loads of x and of g in flight
    const uint16_t* xr = (const uint16_t*)x + (int64_t)t * H;
    const uint16_t* g = (const uint16_t*)gw;
    for (int c0 = lane * 8; c0 < H; c0 += 4 * 512) {
      u32x4 xv[4], gv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int c = c0 + u * 512;
        xv[u] = c < H ? *(const u32x4*)(xr + c) : u32x4{0u, 0u, 0u, 0u};
        gv[u] = c < H ? *(const u32x4*)(g + c) : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          s += __uint_as_float(xv[u][h] << 16) * __uint_as_float(gv[u][h] << 16);
          s += __uint_as_float(xv[u][h] & 0xffff0000u) * __uint_as_float(gv[u][h] & 0xffff0000u);
        }
    }
  } else if (act_bf16) {
    const uint16_t* xr = (const uint16_t*)x + (int64_t)t * H;
    const uint16_t* g = (const uint16_t*)gw;
    for (int i = lane; i < H; i += 64) s += bf16_bits_to_f32(xr[i]) * bf16_bits_to_f32(g[i]);
  } else {
    const float* xr = (const float*)x + (int64_t)t * H;
    const float* g = (const float*)gw;
    for (int i = lane; i < H; i += 64) s += xr[i] * g[i];
  }
  s = wave_sum_butterfly(s);
  return 1.0f / (1.0f + __expf(-s));
}

}  // namespace nkt
