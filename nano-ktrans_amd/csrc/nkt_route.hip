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

// LDS writes of this wave visible to its other lanes (no workgroup barrier)
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

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
  bool sel[VPL];
  int eq_before = 0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const uint64_t m = ballot64(key[j] == tau);
    const int r = eq_before + lanes_below(m);
    sel[j] = key[j] > tau || (key[j] == tau && r < need_eq);
    eq_before += __popcll(m);
  }

  // ---- the k selected elements into lanes 0..k-1, ascending id ----------
  int before = 0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const uint64_t m = ballot64(sel[j]);
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
// K2 for small batches: one workgroup of 16 waves groups the P = T*k pairs
// (P <= kFusedRouteMaxPairs) whose expert ids sit in LDS.  Thread t owns
// (expert e, part q) = (t / NP, t % NP): the pairs are cut into NP equal
// consecutive parts and the thread counts the pairs of its part that go to
// its expert.  An expert's NP counts sit in neighbouring lanes, so its total
// takes a few DPP adds; one workgroup prefix sum over the threads, in
// (expert, part) order, of count | tiles << 16 then gives every thread the
// first position of its pairs inside the expert's segment and every expert
// its first tile.  A second walk over the part writes perm / inv / tile
// sources in pair order (stable in token order, independent of scheduling);
// the expert's lanes write its tile records.  Two workgroup barriers in all.
// ---------------------------------------------------------------------------
constexpr int kGroupWaves = 16;
constexpr int kGroupThreads = 64 * kGroupWaves;

// parts per expert: NP lanes of one expert share a 16-lane row
__host__ __device__ constexpr int group_parts(int E) {
  int epad = 1;
  while (epad < E) epad <<= 1;
  const int np = kGroupThreads / epad;
  return np < 16 ? np : 16;
}

// Sum over the aligned group of NP (1, 2, 4, 8 or 16) neighbouring lanes,
// in every lane of the group.
__device__ __forceinline__ int group_lane_sum(int v, int np) {
  if (np >= 2) v += (int)dpp_u32<0xB1>((uint32_t)v);   // quad_perm [1,0,3,2]: lane ^ 1
  if (np >= 4) v += (int)dpp_u32<0x4E>((uint32_t)v);   // quad_perm [2,3,0,1]: lane ^ 2
  if (np >= 8) v += (int)dpp_u32<0x141>((uint32_t)v);  // row_half_mirror: the other quad
  if (np >= 16) v += (int)dpp_u32<0x140>((uint32_t)v); // row_mirror: the other half row
  return v;
}

// Bit i of the result: pair p + i (i < n <= 64) goes to expert e.
__device__ __forceinline__ uint64_t pair_match_mask(const int32_t* ids, int p, int n, int e) {
  uint32_t lo = 0, hi = 0;
  for (int i = 0; i < n; i += 4) {
    const int4 g = *(const int4*)(ids + p + i);
    const uint32_t b = (uint32_t)(g.x == e) | ((uint32_t)(g.y == e) << 1) | ((uint32_t)(g.z == e) << 2) |
                       ((uint32_t)(g.w == e) << 3);
    if (i < 32)
      lo |= b << i;
    else
      hi |= b << (i - 32);
  }
  const uint64_t m = ((uint64_t)hi << 32) | lo;
  return n >= 64 ? m : m & ((1ull << n) - 1);
}

// ids: LDS, 16-byte aligned, at least P rounded up to 4 entries readable.
// res_ok: this thread's expert is HBM-resident (loaded by the caller early).
// bm: a power of two (kTileSrcCols when tile_src is given).
__device__ __forceinline__ void group_small(const int32_t* ids, int T, int k, int E, int bm,
                                            int max_tiles, bool res_ok, int32_t* __restrict__ counts,
                                            int32_t* __restrict__ offsets, int32_t* __restrict__ perm,
                                            int32_t* __restrict__ inv, int32_t* __restrict__ tiles,
                                            int32_t* __restrict__ n_tiles, int32_t* __restrict__ tile_src,
                                            int32_t* wave_tot) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int P = T * k;
  const int np = group_parts(E);  // a power of two
  const int lg_np = __builtin_ctz(np);
  const int e = tid >> lg_np;
  const int q = tid & (np - 1);
  const bool own = e < E;
  const int chunk = (((P + np - 1) >> lg_np) + 3) & ~3;
  const int pb = min(P, q * chunk);
  const int pe = min(P, pb + chunk);

  // pass 1: pairs of this part that go to e, as bit masks of 64-pair windows
  // (the first window's mask is kept for pass 2)
  int cnt = 0;
  uint64_t m_first = 0;
  if (own) {
    for (int p = pb; p < pe; p += 64) {
      const uint64_t m = pair_match_mask(ids, p, min(64, pe - p), e);
      if (p == pb) m_first = m;
      cnt += __popcll(m);
    }
  }
  const int tot = group_lane_sum(cnt, np);
  const int nt = (own && res_ok) ? (tot + bm - 1) >> __builtin_ctz(bm) : 0;  // non-resident: no tiles

  // workgroup exclusive prefix of (pairs | tiles << 16) in (expert, part) order
  const int val = own ? (cnt | ((q == 0 ? nt : 0) << 16)) : 0;
  const int incl = wave_inclusive_scan(val);
  if (lane == 63) wave_tot[wave] = incl;
  __syncthreads();
  int base = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kGroupWaves; ++w) {
    const int x = wave_tot[w];
    base += (w < wave) ? x : 0;
    total += x;
  }
  const int excl = base + incl - val;
  const int pos0 = excl & 0xffff;                      // first position of this part's pairs
  const int off_e = __shfl(pos0, lane & ~(np - 1));    // the expert's first position
  const int toff_e = (excl >> 16) - (q > 0 ? nt : 0);  // the expert's first tile
  const int n_pairs = total & 0xffff;
  const int n_tile_all = total >> 16;

  // pass 2: positions in pair order, one iteration per matching pair; the
  // token of pair p is p / k = (p * ceil(2^32 / k)) >> 32 (exact for p < 2^16)
  if (cnt > 0) {
    const uint64_t kmagic = ((1ull << 32) + (uint64_t)k - 1) / (uint64_t)k;
    int pos = pos0;
    for (int p = pb; p < pe; p += 64) {
      uint64_t m = (p == pb) ? m_first : pair_match_mask(ids, p, min(64, pe - p), e);
      while (m) {
        const int pp = p + __builtin_ctzll(m);
        m &= m - 1;
        perm[pos] = pp;
        inv[pp] = pos;
        if (tile_src && nt > 0) {
          const int rel = pos - off_e;
          const int ti = toff_e + rel / kTileSrcCols;
          if (ti < max_tiles) tile_src[ti * kTileSrcCols + rel % kTileSrcCols] = (int)(((uint64_t)pp * kmagic) >> 32);
        }
        ++pos;
      }
    }
  }

  // the expert's tile records (expert, first position, rows); its lanes pad
  // the unused source columns of every tile
  if (own) {
    if (q == 0) {
      counts[e] = tot;
      offsets[e] = off_e;
    }
    for (int m = 0; m < nt; ++m) {
      const int ti = toff_e + m;
      if (ti >= max_tiles) break;
      const int rows = min(bm, tot - m * bm);
      if (q == 0) *(int4*)(tiles + 4 * ti) = int4{e, off_e + m * bm, rows, 0};
      if (tile_src)
        for (int c = q; c < kTileSrcCols; c += np)
          if (c >= rows) tile_src[ti * kTileSrcCols + c] = 0;
    }
  }
  if (tid == 0) {
    offsets[E] = n_pairs;
    n_tiles[0] = min(n_tile_all, max_tiles);
  }
  // records past the last tile say "no rows" (the decode form reads every record up to max_tiles)
  for (int ti = n_tile_all + tid; ti < max_tiles; ti += kGroupThreads) *(int4*)(tiles + 4 * ti) = int4{0, 0, 0, 0};
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
__global__ void __launch_bounds__(kGroupThreads) route_group_kernel(
    const void* __restrict__ logits, int T, int E, int k, unsigned flags, int bm, int max_tiles,
    int32_t* __restrict__ ids_out, float* __restrict__ w_out, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ perm, int32_t* __restrict__ inv,
    int32_t* __restrict__ tiles, int32_t* __restrict__ n_tiles, int32_t* __restrict__ tile_src,
    const uint8_t* __restrict__ resident) {
  __shared__ __attribute__((aligned(16))) int32_t ids_s[kFusedRouteMaxPairs];
  __shared__ int32_t wave_tot[kGroupWaves];
  __shared__ float sv[kGroupWaves][kMaxTopK];
  __shared__ int si[kGroupWaves][kMaxTopK];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  // the grouping thread's residency flag, read before routing so its latency hides
  const int ge = threadIdx.x / group_parts(E);
  const bool res_ok = !resident || (ge < E && resident[ge]);
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
  group_small(ids_s, T, k, E, bm, max_tiles, res_ok, counts, offsets, perm, inv, tiles, n_tiles, tile_src,
              wave_tot);
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
  if (bm <= 0 || (bm & (bm - 1)) != 0) return hipErrorInvalidValue;
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
