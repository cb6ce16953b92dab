// K1 device code shared by the routing kernels and the single-token gate_up
// GEMV: router softmax + top-k + renormalise for one token, one wavefront.
//
// Routing semantics follow nano_ktrans/layers/hybrid_moe.py:3321-3329:
//   softmax arches: p = softmax_fp32(logits) rounded to the logits dtype,
//                   top-k of p, optional w / sum(w) in the logits dtype;
//   Mixtral:        top-k of the logits, softmax over the k selected values.
// The order of every floating-point operation is fixed (route_expf, the
// lane/butterfly layout of the softmax sum, slot-order k-way sums) so the
// result is reproducible bit for bit.
#pragma once

#include "nkt_common.h"

namespace nkt {

__device__ __forceinline__ uint32_t ordered_bits(float v) {
  v = v + 0.0f;  // -0.0 -> +0.0
  uint32_t u = __float_as_uint(v);
  if (v != v) u = 0x7fc00000u;  // NaN ranks above everything
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float from_ordered_bits(uint32_t o) {
  uint32_t u = (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o;
  return __uint_as_float(u);
}

// number of set bits of m below this lane
__device__ __forceinline__ int lanes_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                        __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__device__ __forceinline__ uint64_t ballot64(bool p) { return __ballot(p); }

// LDS writes of this wave visible to its other lanes (no workgroup barrier)
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The selection of one token with the whole wavefront: lane l's values
// v[j] (expert l + 64 j; the rounded probabilities for softmax arches, else
// the logits) and whether that expert is among the token's k.
template <int VPL, bool BF16>
__device__ __forceinline__ void route_select(const void* __restrict__ logits, int t, int E, int k, unsigned flags,
                                             float (&v)[VPL], bool (&sel)[VPL]) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  bool valid[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = lane + 64 * j;
    valid[j] = e < E;
    const int64_t idx = (int64_t)t * E + (valid[j] ? e : 0);
    float x;
    if (BF16)
      x = bf16_bits_to_f32(((const uint16_t*)logits)[idx]);
    else
      x = ((const float*)logits)[idx];
    v[j] = valid[j] ? x : -__builtin_huge_valf();
  }

  const bool use_softmax = flags & 1u;
  if (use_softmax) {
    float m = v[0];
#pragma unroll
    for (int j = 1; j < VPL; ++j) m = (v[j] > m) ? v[j] : m;
    m = wave_max_tree(m);
    float ex[VPL];
    float part = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      ex[j] = valid[j] ? route_expf(v[j] - m) : 0.0f;
      part = (j == 0) ? ex[j] : part + ex[j];
    }
    const float s = wave_sum_tree(part);
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      float p = ex[j] / s;
      if (BF16) p = bf16_round(p);
      v[j] = p;
    }
  }

  // ---- radix select of the k-th largest key ------------------------------
  uint32_t key[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) key[j] = valid[j] ? ordered_bits(v[j]) : 0u;  // valid keys > 0
  // a bf16 value fixes the low 16 key bits (0 for values >= 0, ones below):
  // only the high 16 need rounds
  const int low_bit = BF16 ? 16 : 0;
  uint32_t tau = 0;
#pragma unroll 4
  for (int b = 31; b >= low_bit; --b) {
    const uint32_t cand = tau | (1u << b);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < VPL; ++j) cnt += __popcll(ballot64(key[j] >= cand));
    tau = (cnt >= k) ? cand : tau;
  }
  // the skipped low bits of a bf16 key: 0 for values >= 0, all ones below 0
  if (BF16 && !(tau & 0x80000000u)) tau |= 0xffffu;
  int above = 0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) above += __popcll(ballot64(key[j] > tau));
  const int need_eq = k - above;  // >= 1 ties at tau, lowest ids first
  int eq_before = 0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const uint64_t m = ballot64(key[j] == tau);
    const int r = eq_before + lanes_below(m);
    sel[j] = key[j] > tau || (key[j] == tau && r < need_eq);
    eq_before += __popcll(m);
  }
}

// The token's selected experts as a bit mask (bit e of 32-bit word e / 32,
// words 0 .. 2 VPL - 1), written to selmask (LDS) by lane 0: the selection of
// route_token without its slots and weights.
template <int VPL, bool BF16>
__device__ __forceinline__ void route_mask(const void* __restrict__ logits, int t, int E, int k, unsigned flags,
                                           uint32_t* selmask) {
  float v[VPL];
  bool sel[VPL];
  route_select<VPL, BF16>(logits, t, E, k, flags, v, sel);
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const uint64_t m = ballot64(sel[j]);
    if (lane == 0) {
      selmask[2 * j] = (uint32_t)m;
      selmask[2 * j + 1] = (uint32_t)(m >> 32);
    }
  }
}

// Route one token with the whole wavefront.  sv/si: this wave's 16-entry LDS
// scratch (selected values / ids in slot order).  Returns, in lanes < k, the
// slot's expert id and weight; lanes >= k return id -1.
// selmask (nullable, LDS): the token's selected experts as a bit mask, bit
// e of 32-bit word e / 32, written by lane 0.
template <int VPL, bool BF16>
__device__ __forceinline__ void route_token(const void* __restrict__ logits, int t, int E, int k,
                                            unsigned flags, float* sv, int* si, int* out_id,
                                            float* out_w, uint32_t* selmask = nullptr) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  float v[VPL];
  bool sel[VPL];
  route_select<VPL, BF16>(logits, t, E, k, flags, v, sel);
  const bool use_softmax = flags & 1u;
  const bool renorm = flags & 2u;

  // ---- the k selected elements into lanes 0..k-1, ascending id ----------
  int before = 0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const uint64_t m = ballot64(sel[j]);
    if (selmask && lane == 0) {
      selmask[2 * j] = (uint32_t)m;
      selmask[2 * j + 1] = (uint32_t)(m >> 32);
    }
    if (sel[j]) {
      const int c = before + lanes_below(m);
      sv[c] = v[j];
      si[c] = lane + 64 * j;
    }
    before += __popcll(m);
  }
  wave_lds_sync();
  const bool slot_lane = lane < k;
  const float cv = slot_lane ? sv[lane] : 0.0f;
  const int cid = slot_lane ? si[lane] : -1;
  const uint32_t ck = ordered_bits(cv);
  wave_lds_sync();  // every lane has read its element before the slots are rewritten

  // ---- slot = rank under (value desc, id asc); lanes are in id order, so an
  // equal key ranks first exactly when it sits in a lower lane
  int rank = 0;
  for (int j = 0; j < k; ++j) {
    const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)ck, j);
    rank += (kj > ck || (kj == ck && j < lane)) ? 1 : 0;
  }
  if (slot_lane) {
    sv[rank] = cv;
    si[rank] = cid;
  }
  wave_lds_sync();
  const float val = slot_lane ? sv[lane] : 0.0f;  // slot order from here on
  const int sid = slot_lane ? si[lane] : -1;

  // ---- weights, k-way sums in slot order (uniform, from lane reads) -------
  const float m0 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(val), 0));
  const float e = (!use_softmax && slot_lane) ? route_expf(val - m0) : 0.0f;
  const float term = use_softmax ? val : e;
  float s = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(term), 0));
  if (!use_softmax || renorm) {
    for (int jj = 1; jj < k; ++jj) s = s + __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(term), jj));
    if (use_softmax && BF16) s = bf16_round(s);
  }
  int id = -1;
  float w = 0.0f;
  if (slot_lane) {
    id = sid;
    if (use_softmax) {
      w = val;
      if (renorm) {
        const float q = val / s;
        w = BF16 ? bf16_round(q) : q;
      }
    } else {
      const float q = e / s;
      w = BF16 ? bf16_round(q) : q;
    }
  }
  *out_id = id;
  *out_w = w;
  __builtin_amdgcn_wave_barrier();  // sv/si are reused by this wave's next token
}

}  // namespace nkt
