// K1: router softmax + top-k + renormalise, one wavefront per token.
// K2: deterministic count / prefix-sum / permute of the (token, slot) pairs
//     by expert, plus the tile list the grouped expert GEMMs walk.
//
// Routing semantics follow nano_ktrans/layers/hybrid_moe.py:3321-3329:
//   softmax arches: p = softmax_fp32(logits) rounded to the logits dtype,
//                   top-k of p, optional w / sum(w) in the logits dtype;
//   Mixtral:        top-k of the logits, softmax over the k selected values.
// Grouping follows hybrid_moe.py:3512-3526 / cpu_moe.py:515-523: experts in
// ascending id, tokens in ascending order within an expert.
// The order of every floating-point operation is fixed (route_expf, the
// lane/butterfly layout of the softmax sum, slot-order k-way sums) so the
// result is reproducible bit for bit.
//
// Top-k selection is a radix select over the 32-bit order-preserving keys:
// 32 ballot/popcount rounds find the k-th largest key, ties at that key are
// taken in ascending expert id, and each selected element's slot is its rank
// under (value descending, id ascending), counted with scalar broadcasts.  No
// cross-lane shuffles sit on the selection's critical path.
//
// Small batches run route and grouping in one launch (one workgroup of 16
// waves); large batches use a wave-per-token route launch and a grouping
// launch.
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

// number of set bits of m below this lane
__device__ __forceinline__ int lanes_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                        __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__device__ __forceinline__ uint64_t ballot64(bool p) { return __ballot(p); }

// Route one token with the whole wavefront.  sv/si: this wave's 16-entry LDS
// scratch (selected values / ids in slot order).  Returns, in lanes < k, the
// slot's expert id and weight; lanes >= k return id -1.
template <int VPL, bool BF16>
__device__ __forceinline__ void route_token(const void* __restrict__ logits, int t, int E, int k,
                                            unsigned flags, float* sv, int* si, int* out_id,
                                            float* out_w) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  float v[VPL];
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
  bool sel[VPL];
  int eq_before = 0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const uint64_t m = ballot64(key[j] == tau);
    const int r = eq_before + lanes_below(m);
    sel[j] = key[j] > tau || (key[j] == tau && r < need_eq);
    eq_before += __popcll(m);
  }

  // ---- slot = rank under (value desc, id asc) among the selected ---------
  int rank[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) rank[j] = 0;
#pragma unroll
  for (int j2 = 0; j2 < VPL; ++j2) {
    uint64_t m = ballot64(sel[j2]);
    while (m) {
      const int ln = __builtin_ctzll(m);
      m &= m - 1;
      const uint32_t ks = (uint32_t)__builtin_amdgcn_readlane((int)key[j2], ln);
      const int is = ln + 64 * j2;
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        const int id = lane + 64 * j;
        rank[j] += (ks > key[j] || (ks == key[j] && is < id)) ? 1 : 0;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    if (sel[j]) {
      sv[rank[j]] = v[j];
      si[rank[j]] = lane + 64 * j;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- weights, k-way sums in slot order ---------------------------------
  float s = 0.0f;
  float m0 = sv[0];
  if (use_softmax) {
    if (renorm) {
      for (int jj = 0; jj < k; ++jj) s = (jj == 0) ? sv[0] : s + sv[jj];
      if (BF16) s = bf16_round(s);
    }
  } else {
    for (int jj = 0; jj < k; ++jj) {
      const float e = route_expf(sv[jj] - m0);
      s = (jj == 0) ? e : s + e;
    }
  }
  int id = -1;
  float w = 0.0f;
  if (lane < k) {
    id = si[lane];
    const float val = sv[lane];
    if (use_softmax) {
      w = val;
      if (renorm) {
        const float q = val / s;
        w = BF16 ? bf16_round(q) : q;
      }
    } else {
      const float q = route_expf(val - m0) / s;
      w = BF16 ? bf16_round(q) : q;
    }
  }
  *out_id = id;
  *out_w = w;
  __builtin_amdgcn_wave_barrier();  // sv/si are reused by this wave's next token
}

template <int VPL, bool BF16>
__global__ void __launch_bounds__(256) route_kernel(const void* __restrict__ logits, int T, int E,
                                                    int k, unsigned flags,
                                                    int32_t* __restrict__ ids_out,
                                                    float* __restrict__ w_out) {
  __shared__ float sv[4][kMaxTopK];
  __shared__ int si[4][kMaxTopK];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  int id;
  float w;
  route_token<VPL, BF16>(logits, t, E, k, flags, sv[wave], si[wave], &id, &w);
  if (lane < k) {
    ids_out[(int64_t)t * k + lane] = id;
    w_out[(int64_t)t * k + lane] = w;
  }
}

// ---------------------------------------------------------------------------
// K2 body: one workgroup of 16 waves groups the P = T*k pairs whose expert
// ids sit in ids (global or LDS).  Wave w owns a contiguous range of pairs (in
// pair order = token order).  Pass 1 counts per (wave, expert); a column scan
// gives each wave its starting slot inside every expert's segment; pass 2
// walks the range 64 pairs at a time and ranks equal experts inside the chunk
// with ballots, so the permutation is stable in token order and independent
// of scheduling.  Then the tile list: (expert, first position, rows) for
// every BM-row slice of every expert's segment, experts ascending.
// ---------------------------------------------------------------------------
constexpr int kGroupWaves = 16;

struct GroupLds {
  int32_t hist[kGroupWaves][kMaxExperts];
  int32_t tot[kMaxExperts];
  int32_t off_s[kMaxExperts + 1];
  int32_t tile_off[kMaxExperts + 1];
};

__device__ __forceinline__ void group_body(const int32_t* ids, int T, int k, int E, int bm,
                                           int max_tiles, int32_t* __restrict__ counts,
                                           int32_t* __restrict__ offsets,
                                           int32_t* __restrict__ perm, int32_t* __restrict__ inv,
                                           int32_t* __restrict__ tiles,
                                           int32_t* __restrict__ n_tiles,
                                           int32_t* __restrict__ tile_src,
                                           const uint8_t* __restrict__ resident, GroupLds& L) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int P = T * k;
  int ppw = (P + kGroupWaves - 1) / kGroupWaves;
  ppw = (ppw + 63) & ~63;
  const int pbeg = min(P, wave * ppw);
  const int pend = min(P, pbeg + ppw);

  for (int i = tid; i < kGroupWaves * kMaxExperts; i += blockDim.x) (&L.hist[0][0])[i] = 0;
  __syncthreads();

  for (int p = pbeg + lane; p < pend; p += 64) {
    const int e = ids[p];
    if (e >= 0 && e < E) atomicAdd(&L.hist[wave][e], 1);
  }
  __syncthreads();

  // column scan over waves -> per-wave start inside each expert
  if (tid < E) {
    int run = 0;
    for (int w = 0; w < kGroupWaves; ++w) {
      const int h = L.hist[w][tid];
      L.hist[w][tid] = run;
      run += h;
    }
    L.tot[tid] = run;
  }
  __syncthreads();

  // exclusive scans over experts (wave 0, 4 experts per lane): positions and
  // tiles (experts that are not HBM-resident get no tiles)
  if (wave == 0) {
    int local[4], tl[4];
    int sum = 0, tsum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane * 4 + i;
      local[i] = (e < E) ? L.tot[e] : 0;
      tl[i] = (e < E && (!resident || resident[e])) ? (local[i] + bm - 1) / bm : 0;
      sum += local[i];
      tsum += tl[i];
    }
    const int incl = wave_inclusive_scan(sum);
    const int tincl = wave_inclusive_scan(tsum);
    int run = incl - sum, trun = tincl - tsum;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane * 4 + i;
      if (e < E) {
        L.off_s[e] = run;
        L.tile_off[e] = trun;
      }
      run += local[i];
      trun += tl[i];
    }
    if (lane == 63) {
      L.off_s[E] = incl;
      L.tile_off[E] = tincl;
    }
  }
  __syncthreads();

  if (tid < E) {
    counts[tid] = L.tot[tid];
    offsets[tid] = L.off_s[tid];
    for (int w = 0; w < kGroupWaves; ++w) L.hist[w][tid] += L.off_s[tid];
  }
  if (tid == 0) offsets[E] = L.off_s[E];
  __syncthreads();

  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  for (int base = pbeg; base < pend; base += 64) {
    const int p = base + lane;
    const bool valid = p < pend;
    const int e = valid ? ids[p] : 0;
    const bool ok = valid && e >= 0 && e < E;
    uint64_t same = __ballot(ok);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (e >> b) & 1;
      const uint64_t bb = __ballot(ok && bit);
      same &= bit ? bb : ~bb;
    }
    if (ok) {
      const int rank = lanes_below(same);
      const int cnt = __popcll(same);
      const int pos = L.hist[wave][e] + rank;
      perm[pos] = p;
      inv[p] = pos;
      if (tile_src && (!resident || resident[e])) {
        const int rel = pos - L.off_s[e];
        const int ti = L.tile_off[e] + rel / bm;
        if (ti < max_tiles) tile_src[ti * kTileSrcCols + rel % bm] = p / k;
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): every lane has read its start
      if (rank == cnt - 1) L.hist[wave][e] += cnt;
    }
  }

  // tile list for the grouped GEMMs: (expert, first position, rows); lane
  // group lane/16 takes a tile, its 16 lanes the tile's source-row padding
  for (int e = wave; e < E; e += kGroupWaves) {
    const int c = L.tot[e];
    const int nt = (!resident || resident[e]) ? (c + bm - 1) / bm : 0;
    for (int m = lane >> 4; m < nt; m += 4) {
      const int ti = L.tile_off[e] + m;
      if (ti < max_tiles) {
        const int rows = min(bm, c - m * bm);
        if ((lane & 15) == 0) *(int4*)(tiles + 4 * ti) = int4{e, L.off_s[e] + m * bm, rows, 0};
        if (tile_src && (lane & 15) >= rows) tile_src[ti * kTileSrcCols + (lane & 15)] = 0;
      }
    }
  }
  // records past the last tile say "no rows" (the decode form reads every record up to max_tiles)
  for (int ti = L.tile_off[E] + tid; ti < max_tiles; ti += blockDim.x) *(int4*)(tiles + 4 * ti) = int4{0, 0, 0, 0};
  if (tid == 0) n_tiles[0] = min(L.tile_off[E], max_tiles);
}

// ---------------------------------------------------------------------------
// K2 for large batches, over many workgroups: count_kernel writes one
// histogram per block of kPairsPerBlock consecutive pairs; scatter_kernel
// (same blocks) turns the histograms into each block's start inside every
// expert's segment, ranks its pairs with ballots (stable in pair order) and
// writes perm / inv; block 0 also writes counts, offsets and the tile list.
// ---------------------------------------------------------------------------
constexpr int kScatterWaves = 16;
constexpr int kPairsPerWave = 128;
constexpr int kPairsPerBlock = kScatterWaves * kPairsPerWave;

__global__ void __launch_bounds__(1024) count_kernel(const int32_t* __restrict__ ids, int P, int E,
                                                     int32_t* __restrict__ hist) {
  __shared__ int32_t h[kMaxExperts];
  const int tid = threadIdx.x;
  if (tid < E) h[tid] = 0;
  __syncthreads();
  const int p0 = blockIdx.x * kPairsPerBlock;
  for (int p = p0 + tid; p < min(P, p0 + kPairsPerBlock); p += 1024) {
    const int e = ids[p];
    if (e >= 0 && e < E) atomicAdd(&h[e], 1);
  }
  __syncthreads();
  if (tid < E) hist[(int64_t)blockIdx.x * E + tid] = h[tid];
}

__global__ void __launch_bounds__(1024) scatter_kernel(const int32_t* __restrict__ ids, int P, int k, int E, int bm,
                                                       int max_tiles, const int32_t* __restrict__ hist,
                                                       int32_t* __restrict__ counts,
                                                       int32_t* __restrict__ offsets,
                                                       int32_t* __restrict__ perm, int32_t* __restrict__ inv,
                                                       int32_t* __restrict__ tiles,
                                                       int32_t* __restrict__ n_tiles,
                                                       int32_t* __restrict__ tile_src,
                                                       const uint8_t* __restrict__ resident) {
  __shared__ int32_t tot[kMaxExperts], pre[kMaxExperts], off_s[kMaxExperts + 1], tile_off[kMaxExperts + 1];
  __shared__ int32_t whist[kScatterWaves][kMaxExperts];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int nb = gridDim.x;
  const int b = blockIdx.x;
  // totals per expert and the pairs of earlier blocks, blocks in order
  if (tid < E) {
    int t = 0, q = 0;
#pragma unroll 8
    for (int bb = 0; bb < nb; ++bb) {
      const int c = hist[(int64_t)bb * E + tid];
      q += bb < b ? c : 0;
      t += c;
    }
    tot[tid] = t;
    pre[tid] = q;
  }
  for (int i = tid; i < kScatterWaves * kMaxExperts; i += 1024) (&whist[0][0])[i] = 0;
  __syncthreads();
  // exclusive scans over experts (wave 0, 4 experts per lane): positions and
  // tiles (experts that are not HBM-resident get no tiles)
  if (wave == 0) {
    int local[4], tl[4];
    int sum = 0, tsum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane * 4 + i;
      local[i] = (e < E) ? tot[e] : 0;
      tl[i] = (e < E && (!resident || resident[e])) ? (local[i] + bm - 1) / bm : 0;
      sum += local[i];
      tsum += tl[i];
    }
    const int incl = wave_inclusive_scan(sum);
    const int tincl = wave_inclusive_scan(tsum);
    int run = incl - sum, trun = tincl - tsum;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane * 4 + i;
      if (e < E) {
        off_s[e] = run;
        tile_off[e] = trun;
      }
      run += local[i];
      trun += tl[i];
    }
    if (lane == 63) {
      off_s[E] = incl;
      tile_off[E] = tincl;
    }
  }
  // per-wave histogram of this block's pairs (wave w: kPairsPerWave consecutive pairs)
  const int pbeg = min(P, b * kPairsPerBlock + wave * kPairsPerWave);
  const int pend = min(P, pbeg + kPairsPerWave);
  for (int p = pbeg + lane; p < pend; p += 64) {
    const int e = ids[p];
    if (e >= 0 && e < E) atomicAdd(&whist[wave][e], 1);
  }
  __syncthreads();
  // each wave's start inside every expert's segment
  if (tid < E) {
    int run = off_s[tid] + pre[tid];
#pragma unroll
    for (int w = 0; w < kScatterWaves; ++w) {
      const int c = whist[w][tid];
      whist[w][tid] = run;
      run += c;
    }
  }
  if (b == 0) {
    if (tid < E) {
      counts[tid] = tot[tid];
      offsets[tid] = off_s[tid];
    }
    if (tid == 0) {
      offsets[E] = off_s[E];
      n_tiles[0] = min(tile_off[E], max_tiles);
    }
    // records past the last tile say "no rows" (the decode form reads every record up to max_tiles)
    for (int ti = tile_off[E] + tid; ti < max_tiles; ti += 1024) *(int4*)(tiles + 4 * ti) = int4{0, 0, 0, 0};
    for (int e = wave; e < E; e += kScatterWaves) {
      const int c = tot[e];
      const int nt = (!resident || resident[e]) ? (c + bm - 1) / bm : 0;
      for (int m = lane >> 4; m < nt; m += 4) {
        const int ti = tile_off[e] + m;
        if (ti < max_tiles) {
          const int rows = min(bm, c - m * bm);
          if ((lane & 15) == 0) *(int4*)(tiles + 4 * ti) = int4{e, off_s[e] + m * bm, rows, 0};
          if (tile_src && (lane & 15) >= rows) tile_src[ti * kTileSrcCols + (lane & 15)] = 0;
        }
      }
    }
  }
  __syncthreads();
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  for (int base = pbeg; base < pend; base += 64) {
    const int p = base + lane;
    const bool valid = p < pend;
    const int e = valid ? ids[p] : 0;
    const bool ok = valid && e >= 0 && e < E;
    uint64_t same = __ballot(ok);
    for (int bit = 0; bit < nbits; ++bit) {
      const bool on = (e >> bit) & 1;
      const uint64_t bb = __ballot(ok && on);
      same &= on ? bb : ~bb;
    }
    if (ok) {
      const int rank = lanes_below(same);
      const int cnt = __popcll(same);
      const int pos = whist[wave][e] + rank;
      perm[pos] = p;
      inv[p] = pos;
      if (tile_src && (!resident || resident[e])) {
        const int rel = pos - off_s[e];
        const int ti = tile_off[e] + rel / bm;
        if (ti < max_tiles) tile_src[ti * kTileSrcCols + rel % bm] = p / k;
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): every lane has read its start
      if (rank == cnt - 1) whist[wave][e] += cnt;
    }
  }
}

int group_hist_blocks(int P) { return (P + kPairsPerBlock - 1) / kPairsPerBlock; }

hipError_t launch_group_multi(const int32_t* ids, int T, int k, int E, int bm, int max_tiles, int32_t* hist,
                              int32_t* counts, int32_t* offsets, int32_t* perm, int32_t* inv, int32_t* tiles,
                              int32_t* n_tiles, int32_t* tile_src, const uint8_t* resident,
                              hipStream_t stream) {
  if (tile_src && bm != kTileSrcCols) return hipErrorInvalidValue;
  const int P = T * k;
  const int nb = group_hist_blocks(P);
  if (nb <= 0) return hipSuccess;
  hipLaunchKernelGGL(count_kernel, dim3(nb), dim3(1024), 0, stream, ids, P, E, hist);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(scatter_kernel, dim3(nb), dim3(1024), 0, stream, ids, P, k, E, bm, max_tiles, hist, counts,
                     offsets, perm, inv, tiles, n_tiles, tile_src, resident);
  return hipGetLastError();
}

// Route and group in one workgroup of 16 waves (small batches): wave w routes
// tokens w, w + 16, ...; the ids stay in LDS for the grouping.
template <int VPL, bool BF16>
__global__ void __launch_bounds__(1024) route_group_kernel(
    const void* __restrict__ logits, int T, int E, int k, unsigned flags, int bm, int max_tiles,
    int32_t* __restrict__ ids_out, float* __restrict__ w_out, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ perm, int32_t* __restrict__ inv,
    int32_t* __restrict__ tiles, int32_t* __restrict__ n_tiles, int32_t* __restrict__ tile_src,
    const uint8_t* __restrict__ resident) {
  __shared__ GroupLds L;
  __shared__ int32_t ids_s[kFusedRouteMaxPairs];
  __shared__ float sv[kGroupWaves][kMaxTopK];
  __shared__ int si[kGroupWaves][kMaxTopK];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  for (int t = wave; t < T; t += kGroupWaves) {
    int id;
    float w;
    route_token<VPL, BF16>(logits, t, E, k, flags, sv[wave], si[wave], &id, &w);
    if (lane < k) {
      ids_s[t * k + lane] = id;
      ids_out[(int64_t)t * k + lane] = id;
      w_out[(int64_t)t * k + lane] = w;
    }
  }
  __syncthreads();
  group_body(ids_s, T, k, E, bm, max_tiles, counts, offsets, perm, inv, tiles, n_tiles, tile_src, resident, L);
}

#define NKT_VPL_SWITCH(E, CASE) \
  switch ((E + 63) / 64) {      \
    CASE(1)                     \
    CASE(2)                     \
    CASE(3)                     \
    CASE(4)                     \
    default:                    \
      return hipErrorInvalidValue; \
  }

hipError_t launch_route(const void* logits, int act_bf16, int T, int E, int k, unsigned flags,
                        int32_t* ids, float* w, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  dim3 grid((T + 3) / 4), block(256);
#define NKT_ROUTE_CASE(V)                                                                    \
  case V:                                                                                    \
    if (act_bf16)                                                                            \
      hipLaunchKernelGGL((route_kernel<V, true>), grid, block, 0, stream, logits, T, E, k,   \
                         flags, ids, w);                                                     \
    else                                                                                     \
      hipLaunchKernelGGL((route_kernel<V, false>), grid, block, 0, stream, logits, T, E, k,  \
                         flags, ids, w);                                                     \
    break;
  NKT_VPL_SWITCH(E, NKT_ROUTE_CASE)
#undef NKT_ROUTE_CASE
  return hipGetLastError();
}

bool route_group_fused(int T, int k) { return T <= kFusedRouteMaxTokens && T * k <= kFusedRouteMaxPairs; }

hipError_t launch_route_group(const void* logits, int act_bf16, int T, int E, int k,
                              unsigned flags, int bm, int max_tiles, int32_t* ids, float* w,
                              int32_t* counts, int32_t* offsets, int32_t* perm, int32_t* inv,
                              int32_t* tiles, int32_t* n_tiles, int32_t* tile_src,
                              const uint8_t* resident, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  if (!route_group_fused(T, k)) return hipErrorInvalidValue;
  if (tile_src && bm != kTileSrcCols) return hipErrorInvalidValue;
  dim3 grid(1), block(64 * kGroupWaves);
#define NKT_RG_CASE(V)                                                                          \
  case V:                                                                                       \
    if (act_bf16)                                                                               \
      hipLaunchKernelGGL((route_group_kernel<V, true>), grid, block, 0, stream, logits, T, E, k, \
                         flags, bm, max_tiles, ids, w, counts, offsets, perm, inv, tiles,       \
                         n_tiles, tile_src, resident);                                          \
    else                                                                                        \
      hipLaunchKernelGGL((route_group_kernel<V, false>), grid, block, 0, stream, logits, T, E,  \
                         k, flags, bm, max_tiles, ids, w, counts, offsets, perm, inv, tiles,    \
                         n_tiles, tile_src, resident);                                          \
    break;
  NKT_VPL_SWITCH(E, NKT_RG_CASE)
#undef NKT_RG_CASE
  return hipGetLastError();
}

}  // namespace nkt
