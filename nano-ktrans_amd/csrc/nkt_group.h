// K2 device code for small batches, shared by the routing kernels and the
// decode gate_up that routes its tokens itself: the grouping from the
// selection masks K1 leaves in LDS, and K1 + K2 of a few tokens in one
// workgroup.
//
// Grouping follows nano_ktrans/layers/hybrid_moe.py:3512-3526 /
// nano_ktrans/kernels/cpu_moe.py:515-523: experts in ascending id, tokens in
// ascending order within an expert.
#pragma once

#include "nkt_common.h"
#include "nkt_internal.h"
#include "nkt_route_token.h"

namespace nkt {

// ---------------------------------------------------------------------------
// K2 for small batches (T <= 64), from the selection masks K1 leaves in LDS
// (token t's experts as bits of selmask[t]).  A token picks an expert at most
// once, so expert e's pairs are the set bits of a 64-bit token mask M_e
// (bit t: token t picked e).  Two steps:
//   * group_scan, one wave, lane l owning the VPL consecutive experts
//     VPL l .. VPL l + VPL - 1: M_e by transposing the token masks (T words
//     read per lane, one bit field extract and insert per token and expert);
//     count_e = popcount(M_e), tiles_e = ceil(count_e / bm) (0 when e is not
//     HBM-resident); one wave scan of count | tiles << 16 in expert order
//     gives every expert its first position and first tile; M_e, the first
//     position and first tile, the count and the tile -> expert map go to LDS;
//   * group_write, the whole workgroup, one output element per thread:
//     counts, offsets, tile records; column r of an expert's tiles = its r-th
//     token = the r-th set bit of M_e (a six-step popcount select); pair
//     p = t k + slot with expert e lands at position
//     off_e + popcount(M_e & (2^t - 1)): tokens ascend within an expert, as
//     the reference's stable grouping orders them.
// ---------------------------------------------------------------------------
constexpr int kGroupWaves = 16;  // waves of the fused route + group workgroup
constexpr int kGroupThreads = 64 * kGroupWaves;
// tiles of the fused grouping: sum of ceil(count_e / bm) <= P / bm + min(P, E)
constexpr int kFusedMaxTiles = kFusedRouteMaxPairs + kMaxExperts;

// LDS the two grouping steps share
struct GroupLds {
  uint32_t mlo[kMaxExperts], mhi[kMaxExperts];  // M_e
  int32_t off[kMaxExperts];                     // first position of expert e
  int32_t toff[kMaxExperts];                    // first tile of expert e
  int32_t cnt[kMaxExperts];                     // count_e
  int32_t tmap[kFusedMaxTiles];                 // tile -> expert
  int32_t n_tile_all;
};

// selmask: [T][8] u32 words (LDS); res: this lane's experts are HBM-resident
// (bit i for expert VPL lane + i).  Runs in one wave.
template <int VPL>
__device__ __forceinline__ void group_scan(const uint32_t (*selmask)[8], int T, int E, int bm, unsigned res,
                                           GroupLds& g) {
  const int lane = threadIdx.x & 63;
  const int lg_bm = __builtin_ctz(bm);
  // token masks of this lane's experts
  uint32_t lo[VPL], hi[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) lo[i] = hi[i] = 0u;
  for (int t = 0; t < T; ++t) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int e = VPL * lane + i;
      const uint32_t b = (selmask[t][(e >> 5) & 7] >> (e & 31)) & 1u;
      if (t < 32)
        lo[i] |= b << t;
      else
        hi[i] |= b << (t - 32);
    }
  }
  int cnt[VPL], nt[VPL];
  int lane_val = 0;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int e = VPL * lane + i;
    const bool own = e < E;
    if (!own) lo[i] = hi[i] = 0u;
    cnt[i] = __popc(lo[i]) + __popc(hi[i]);
    nt[i] = (own && ((res >> i) & 1u)) ? (cnt[i] + bm - 1) >> lg_bm : 0;
    lane_val += cnt[i] | (nt[i] << 16);
  }
  const int incl = wave_inclusive_scan(lane_val);
  int run = incl - lane_val;  // this lane's first (position | tile << 16)
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int e = VPL * lane + i;
    const int off = run & 0xffff, toff = run >> 16;
    run += cnt[i] | (nt[i] << 16);
    if (e >= E) continue;
    g.mlo[e] = lo[i];
    g.mhi[e] = hi[i];
    g.off[e] = off;
    g.toff[e] = toff;
    g.cnt[e] = cnt[i];
    for (int m = 0; m < nt[i]; ++m) g.tmap[toff + m] = e;
  }
  if (lane == 0) g.n_tile_all = __builtin_amdgcn_readlane(incl, 63) >> 16;
}

// the position (0..63) of the r-th (from 0) set bit of m; r < popcount(m)
__device__ __forceinline__ int nth_set_bit(uint64_t m, int r) {
  int pos = 0;
#pragma unroll
  for (int w = 32; w >= 1; w >>= 1) {
    const int c = __popcll(m & ((1ull << w) - 1ull));
    const bool up = r >= c;
    r -= up ? c : 0;
    m = up ? (m >> w) : m;
    pos += up ? w : 0;
  }
  return pos;
}

// ids: the P = T k expert ids (LDS).  Every thread of the workgroup, after a
// barrier that follows group_scan.
// ws (LDS) / wpos (nullable): the pairs' routing weights, and their copy in
// position order.
template <int kThreads = kGroupThreads>
__device__ __forceinline__ void group_write(const GroupLds& g, const int32_t* ids, int T, int k, int E, int bm,
                                            int max_tiles, int32_t* __restrict__ counts,
                                            int32_t* __restrict__ offsets, int32_t* __restrict__ perm,
                                            int32_t* __restrict__ inv, int32_t* __restrict__ tiles,
                                            int32_t* __restrict__ n_tiles, int32_t* __restrict__ tile_src,
                                            const float* ws, float* __restrict__ wpos) {
  const int tid = threadIdx.x;
  const int P = T * k;
  const int n_tile_all = g.n_tile_all;
  const int nt_out = min(n_tile_all, max_tiles);
  for (int e = tid; e < E; e += kThreads) {
    counts[e] = g.cnt[e];
    offsets[e] = g.off[e];
  }
  if (tid == 0) {
    offsets[E] = P;
    n_tiles[0] = nt_out;
  }
  // tile records; records past the last tile say "no rows" (the decode form
  // reads every record up to max_tiles)
  for (int ti = tid; ti < max_tiles; ti += kThreads) {
    int4 rec = int4{0, 0, 0, 0};
    if (ti < n_tile_all) {
      const int e = g.tmap[ti];
      const int m = ti - g.toff[e];
      rec = int4{e, g.off[e] + m * bm, min(bm, g.cnt[e] - m * bm), 0};
    }
    *(int4*)(tiles + 4 * ti) = rec;
  }
  if (tile_src) {
    // column c of tile ti: the expert's token of rank (ti - first tile) * 16 + c, unused columns 0
    for (int i = tid; i < nt_out * kTileSrcCols; i += kThreads) {
      const int ti = i / kTileSrcCols;
      const int e = g.tmap[ti];
      const int r = (ti - g.toff[e]) * kTileSrcCols + (i & (kTileSrcCols - 1));
      const uint64_t mm = ((uint64_t)g.mhi[e] << 32) | g.mlo[e];
      tile_src[i] = r < g.cnt[e] ? nth_set_bit(mm, r) : 0;
    }
  }
  // positions of the pairs; the token of pair p is p / k = (p ceil(2^32 / k)) >> 32
  const uint64_t kmagic = ((1ull << 32) + (uint64_t)k - 1) / (uint64_t)k;
  for (int p = tid; p < P; p += kThreads) {
    const int e = ids[p];
    const int t = (int)(((uint64_t)p * kmagic) >> 32);
    const uint32_t below_lo = t >= 32 ? 0xffffffffu : ((1u << t) - 1u);
    const uint32_t below_hi = t <= 32 ? 0u : ((1u << (t - 32)) - 1u);
    const int pos = g.off[e] + __popc(g.mlo[e] & below_lo) + __popc(g.mhi[e] & below_hi);
    perm[pos] = p;
    inv[p] = pos;
    if (wpos) wpos[pos] = ws[p];
  }
}


// LDS of route_group_body: the pairs' ids and weights, the token masks, the
// grouping's tables and each wave's K1 slot scratch.
template <int kMaxTok, int kMaxPairs, int kWaves>
struct RouteGroupLds {
  int32_t ids[kMaxPairs];
  float w[kMaxPairs];
  uint32_t selmask[kMaxTok][8];
  GroupLds g;
  float sv[kWaves][kMaxTopK];
  int si[kWaves][kMaxTopK];
};

// K1 + K2 for T <= kMaxTok tokens in one workgroup of kWaves waves: wave w
// routes tokens w, w + kWaves, ...; the ids stay in LDS for the grouping.
template <int VPL, bool BF16, int kWaves, int kMaxTok, int kMaxPairs>
__device__ __forceinline__ void route_group_body(
    const void* __restrict__ logits, int T, int E, int k, unsigned flags, int bm, int max_tiles,
    int32_t* __restrict__ ids_out, float* __restrict__ w_out, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ perm, int32_t* __restrict__ inv,
    int32_t* __restrict__ tiles, int32_t* __restrict__ n_tiles, int32_t* __restrict__ tile_src,
    const uint8_t* __restrict__ resident, float* __restrict__ wpos, RouteGroupLds<kMaxTok, kMaxPairs, kWaves>& L) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  // the grouping lane's residency flags, read before routing so their latency hides
  unsigned res = 0;
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int e = VPL * lane + i;
      res |= (unsigned)(!resident || (e < E && resident[e])) << i;
    }
  }
  for (int t = wave; t < T; t += kWaves) {
    int id;
    float w;
    route_token<VPL, BF16>(logits, t, E, k, flags, L.sv[wave], L.si[wave], &id, &w, L.selmask[t]);
    if (lane < k) {
      L.ids[t * k + lane] = id;
      L.w[t * k + lane] = w;
      ids_out[(int64_t)t * k + lane] = id;
      w_out[(int64_t)t * k + lane] = w;
    }
  }
  __syncthreads();
  if (wave == 0) group_scan<VPL>(L.selmask, T, E, bm, res, L.g);
  __syncthreads();
  group_write<64 * kWaves>(L.g, L.ids, T, k, E, bm, max_tiles, counts, offsets, perm, inv, tiles, n_tiles, tile_src,
                           L.w, wpos);
}

}  // namespace nkt
