// K1: router softmax + top-k + renormalise, one wavefront per token.
// K2: deterministic count / prefix-sum / permute of the (token, slot) pairs
//     by expert, plus the tile list the grouped expert GEMM walks.
//
// Routing semantics follow nano_ktrans/layers/hybrid_moe.py:3321-3329:
//   softmax arches: p = softmax_fp32(logits) rounded to the logits dtype,
//                   top-k of p, optional w / sum(w) in the logits dtype;
//   Mixtral:        top-k of the logits, softmax over the k selected values.
// Grouping follows hybrid_moe.py:3512-3526 / cpu_moe.py:515-523: experts in
// ascending id, tokens in ascending order within an expert.
// The order of every floating-point operation is fixed (see route_expf and
// the lane/butterfly layout below) so the result is reproducible bit for bit.
#include "nkt_common.h"
#include "nkt_internal.h"

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

template <int VPL, bool BF16>
__global__ void __launch_bounds__(256) route_kernel(const void* __restrict__ logits, int T, int E,
                                                    int k, unsigned flags,
                                                    int32_t* __restrict__ ids_out,
                                                    float* __restrict__ w_out) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;

  float v[VPL];
  bool valid[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = lane + 64 * j;
    valid[j] = e < E;
    float x = -__builtin_huge_valf();
    if (valid[j]) {
      const int64_t idx = (int64_t)t * E + e;
      if (BF16)
        x = bf16_bits_to_f32(((const uint16_t*)logits)[idx]);
      else
        x = ((const float*)logits)[idx];
    }
    v[j] = x;
  }

  const bool use_softmax = flags & 1u;
  const bool renorm = flags & 2u;

  if (use_softmax) {
    float m = v[0];
#pragma unroll
    for (int j = 1; j < VPL; ++j) m = (v[j] > m) ? v[j] : m;
    m = wave_max(m);
    float ex[VPL];
    float part = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      ex[j] = valid[j] ? route_expf(v[j] - m) : 0.0f;
      part = (j == 0) ? ex[j] : part + ex[j];
    }
    const float s = wave_sum_butterfly(part);
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      float p = ex[j] / s;
      if (BF16) p = bf16_round(p);
      v[j] = p;
    }
  }

  // top-k by repeated wave-wide maximum of (value desc, id asc)
  uint32_t taken = 0;
  int sel_id[kMaxTopK];
  float sel_val[kMaxTopK];
#pragma unroll
  for (int jj = 0; jj < kMaxTopK; ++jj) {
    sel_id[jj] = 0;
    sel_val[jj] = 0.0f;
    if (jj < k) {
      uint64_t best = 0;
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        const int e = lane + 64 * j;
        if (valid[j] && !(taken & (1u << j))) {
          const uint64_t key = ((uint64_t)ordered_bits(v[j]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)e);
          best = key > best ? key : best;
        }
      }
      best = wave_max_u64(best);
      const int id = (int)(0xffffffffu - (uint32_t)best);
      if ((id & 63) == lane) taken |= 1u << (id >> 6);
      sel_id[jj] = id;
      sel_val[jj] = from_ordered_bits((uint32_t)(best >> 32));
    }
  }

  float w[kMaxTopK];
  if (use_softmax) {
#pragma unroll
    for (int jj = 0; jj < kMaxTopK; ++jj) w[jj] = sel_val[jj];
    if (renorm) {
      float s = sel_val[0];
#pragma unroll
      for (int jj = 1; jj < kMaxTopK; ++jj)
        if (jj < k) s = s + sel_val[jj];
      if (BF16) s = bf16_round(s);
#pragma unroll
      for (int jj = 0; jj < kMaxTopK; ++jj) {
        float q = sel_val[jj] / s;
        w[jj] = BF16 ? bf16_round(q) : q;
      }
    }
  } else {
    const float m = sel_val[0];
    float ex[kMaxTopK];
    float s = 0.0f;
#pragma unroll
    for (int jj = 0; jj < kMaxTopK; ++jj) {
      ex[jj] = 0.0f;
      if (jj < k) {
        ex[jj] = route_expf(sel_val[jj] - m);
        s = (jj == 0) ? ex[jj] : s + ex[jj];
      }
    }
#pragma unroll
    for (int jj = 0; jj < kMaxTopK; ++jj) {
      float q = ex[jj] / s;
      w[jj] = BF16 ? bf16_round(q) : q;
    }
  }

  // lane jj writes slot jj
  int my_id = 0;
  float my_w = 0.0f;
#pragma unroll
  for (int jj = 0; jj < kMaxTopK; ++jj) {
    if (lane == jj) {
      my_id = sel_id[jj];
      my_w = w[jj];
    }
  }
  if (lane < k) {
    ids_out[(int64_t)t * k + lane] = my_id;
    w_out[(int64_t)t * k + lane] = my_w;
  }
}

// ---------------------------------------------------------------------------
// K2: one workgroup of 16 waves.  Wave w owns a contiguous range of pairs (in
// pair order = token order).  Pass 1 counts per (wave, expert); a column scan
// gives each wave its starting slot inside every expert's segment; pass 2
// walks the range 64 pairs at a time and ranks equal experts inside the
// chunk with ballots, so the permutation is stable in token order and
// independent of scheduling.
// ---------------------------------------------------------------------------
constexpr int kGroupWaves = 16;

__global__ void __launch_bounds__(1024) group_kernel(const int32_t* __restrict__ ids, int T, int k,
                                                     int E, int bm, int max_tiles,
                                                     int32_t* __restrict__ counts,
                                                     int32_t* __restrict__ offsets,
                                                     int32_t* __restrict__ perm,
                                                     int32_t* __restrict__ inv,
                                                     int32_t* __restrict__ tiles,
                                                     int32_t* __restrict__ n_tiles) {
  __shared__ int32_t hist[kGroupWaves][kMaxExperts];
  __shared__ int32_t tot[kMaxExperts];
  __shared__ int32_t off_s[kMaxExperts + 1];
  __shared__ int32_t tile_off[kMaxExperts + 1];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int P = T * k;
  int ppw = (P + kGroupWaves - 1) / kGroupWaves;
  ppw = (ppw + 63) & ~63;
  const int pbeg = min(P, wave * ppw);
  const int pend = min(P, pbeg + ppw);

  for (int i = tid; i < kGroupWaves * kMaxExperts; i += blockDim.x) (&hist[0][0])[i] = 0;
  __syncthreads();

  for (int p = pbeg + lane; p < pend; p += 64) {
    const int e = ids[p];
    if (e >= 0 && e < E) atomicAdd(&hist[wave][e], 1);
  }
  __syncthreads();

  // column scan over waves -> per-wave start inside each expert
  if (tid < E) {
    int run = 0;
    for (int w = 0; w < kGroupWaves; ++w) {
      const int h = hist[w][tid];
      hist[w][tid] = run;
      run += h;
    }
    tot[tid] = run;
  }
  __syncthreads();

  // exclusive scan over experts (wave 0, 4 experts per lane)
  if (wave == 0) {
    int local[4];
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane * 4 + i;
      local[i] = (e < E) ? tot[e] : 0;
      sum += local[i];
    }
    const int incl = wave_inclusive_scan(sum);
    int run = incl - sum;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane * 4 + i;
      if (e < E) off_s[e] = run;
      run += local[i];
    }
    if (lane == 63) off_s[E] = incl;
  }
  __syncthreads();

  if (tid < E) {
    counts[tid] = tot[tid];
    offsets[tid] = off_s[tid];
    for (int w = 0; w < kGroupWaves; ++w) hist[w][tid] += off_s[tid];
  }
  if (tid == 0) offsets[E] = off_s[E];
  __syncthreads();

  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  for (int base = pbeg; base < pend; base += 64) {
    const int p = base + lane;
    const bool valid = p < pend;
    int e = valid ? ids[p] : 0;
    const bool ok = valid && e >= 0 && e < E;
    uint64_t same = __ballot(ok);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (e >> b) & 1;
      const uint64_t bb = __ballot(ok && bit);
      same &= bit ? bb : ~bb;
    }
    if (ok) {
      const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
      const int rank = __popcll(same & lt);
      const int cnt = __popcll(same);
      const int pos = hist[wave][e] + rank;
      perm[pos] = p;
      inv[p] = pos;
      __builtin_amdgcn_s_waitcnt(0);
      if (rank == cnt - 1) hist[wave][e] += cnt;
    }
  }
  __syncthreads();

  // tile list for the grouped GEMM: (expert, first position, rows)
  if (wave == 0) {
    int local[4];
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane * 4 + i;
      local[i] = (e < E) ? (tot[e] + bm - 1) / bm : 0;
      sum += local[i];
    }
    const int incl = wave_inclusive_scan(sum);
    int run = incl - sum;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane * 4 + i;
      if (e < E) tile_off[e] = run;
      run += local[i];
    }
    if (lane == 63) tile_off[E] = incl;
  }
  __syncthreads();
  if (tid < E) {
    const int c = tot[tid];
    const int nt = (c + bm - 1) / bm;
    for (int m = 0; m < nt; ++m) {
      const int ti = tile_off[tid] + m;
      if (ti < max_tiles) {
        tiles[4 * ti + 0] = tid;
        tiles[4 * ti + 1] = off_s[tid] + m * bm;
        tiles[4 * ti + 2] = min(bm, c - m * bm);
        tiles[4 * ti + 3] = 0;
      }
    }
  }
  if (tid == 0) n_tiles[0] = min(tile_off[E], max_tiles);
}

hipError_t launch_route(const void* logits, int act_bf16, int T, int E, int k, unsigned flags,
                        int32_t* ids, float* w, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  const int tokens_per_block = 4;
  dim3 grid((T + tokens_per_block - 1) / tokens_per_block), block(64 * tokens_per_block);
  const int vpl = (E + 63) / 64;
#define NKT_ROUTE_CASE(V)                                                                    \
  case V:                                                                                    \
    if (act_bf16)                                                                            \
      hipLaunchKernelGGL((route_kernel<V, true>), grid, block, 0, stream, logits, T, E, k,   \
                         flags, ids, w);                                                     \
    else                                                                                     \
      hipLaunchKernelGGL((route_kernel<V, false>), grid, block, 0, stream, logits, T, E, k,  \
                         flags, ids, w);                                                     \
    break;
  switch (vpl) {
    NKT_ROUTE_CASE(1)
    NKT_ROUTE_CASE(2)
    NKT_ROUTE_CASE(3)
    NKT_ROUTE_CASE(4)
    default:
      return hipErrorInvalidValue;
  }
#undef NKT_ROUTE_CASE
  return hipGetLastError();
}

hipError_t launch_group(const int32_t* ids, int T, int k, int E, int bm, int max_tiles,
                        int32_t* counts, int32_t* offsets, int32_t* perm, int32_t* inv,
                        int32_t* tiles, int32_t* n_tiles, hipStream_t stream) {
  hipLaunchKernelGGL(group_kernel, dim3(1), dim3(64 * kGroupWaves), 0, stream, ids, T, k, E, bm,
                     max_tiles, counts, offsets, perm, inv, tiles, n_tiles);
  return hipGetLastError();
}

}  // namespace nkt
