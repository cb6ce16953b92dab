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
// waves routes the tokens, then one wave groups them from the selection
// masks); large batches use a wave-per-token route launch and a grouping
// launch over many workgroups.
#include "nkt_common.h"
#include "nkt_internal.h"
#include "nkt_group.h"
#include "nkt_route_token.h"

namespace nkt {

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
  if (hist) {
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
  } else {
    // no count launch (few pairs): every block counts all pairs itself
    if (tid < E) {
      tot[tid] = 0;
      pre[tid] = 0;
    }
    __syncthreads();
    const int pstart = b * kPairsPerBlock;
    for (int p = tid; p < P; p += 1024) {
      const int e = ids[p];
      if (e >= 0 && e < E) {
        atomicAdd(&tot[e], 1);
        if (p < pstart) atomicAdd(&pre[e], 1);
      }
    }
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

constexpr int kSelfCountMaxPairs = 8192;

hipError_t launch_group_multi(const int32_t* ids, int T, int k, int E, int bm, int max_tiles, int32_t* hist,
                              int32_t* counts, int32_t* offsets, int32_t* perm, int32_t* inv, int32_t* tiles,
                              int32_t* n_tiles, int32_t* tile_src, const uint8_t* resident,
                              hipStream_t stream) {
  if (tile_src && bm != kTileSrcCols) return hipErrorInvalidValue;
  const int P = T * k;
  const int nb = group_hist_blocks(P);
  if (nb <= 0) return hipSuccess;
  // up to kSelfCountMaxPairs pairs every scatter block reads all ids itself
  // (at most 64 KiB each), which costs less than a count launch
  const bool self_count = P <= kSelfCountMaxPairs;
  if (!self_count) {
    hipLaunchKernelGGL(count_kernel, dim3(nb), dim3(1024), 0, stream, ids, P, E, hist);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(scatter_kernel, dim3(nb), dim3(1024), 0, stream, ids, P, k, E, bm, max_tiles,
                     self_count ? nullptr : hist, counts, offsets, perm, inv, tiles, n_tiles, tile_src, resident);
  return hipGetLastError();
}

// Route and group in one workgroup of 16 waves (small batches).
template <int VPL, bool BF16>
__global__ void __launch_bounds__(kGroupThreads) route_group_kernel(
    const void* __restrict__ logits, int T, int E, int k, unsigned flags, int bm, int max_tiles,
    int32_t* __restrict__ ids_out, float* __restrict__ w_out, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ perm, int32_t* __restrict__ inv,
    int32_t* __restrict__ tiles, int32_t* __restrict__ n_tiles, int32_t* __restrict__ tile_src,
    const uint8_t* __restrict__ resident, float* __restrict__ wpos) {
  __shared__ RouteGroupLds<kFusedRouteMaxTokens, kFusedRouteMaxPairs, kGroupWaves> lds;
  route_group_body<VPL, BF16, kGroupWaves>(logits, T, E, k, flags, bm, max_tiles, ids_out, w_out, counts, offsets,
                                          perm, inv, tiles, n_tiles, tile_src, resident, wpos, lds);
}

// ---------------------------------------------------------------------------
// Router (optionally RMSNorm + GEMV), K1 and K2 for up to 64 tokens in one
// launch of several workgroups that pass their results on without waiting
// for each other ("last arriver"): a workgroup publishes its part, then
// counts itself in on an agent-scope counter; the one that arrives last --
// the returned count says so -- has every part and goes on with the next
// step; the others end.  Nothing polls, so nothing can wait for ever.
//
// Grid: token blocks of 4 tokens (one wave each) x expert blocks of 16 router
// rows (1 when the logits are given):
//   A (router GEMV, bf16): workgroup (tb, eb) computes the logits of experts
//     16 eb .. 16 eb + 15 for the tokens of block tb: the 4 rows of x (with
//     NORM first RMS-normalised as nano_ktrans/layers/norm.py:11-17 computes
//     it, the same arithmetic and order as rmsnorm_kernel; block eb == 0
//     writes the normalised rows out) sit in LDS as the B operand, the gate
//     rows are the A operand of v_mfma_f32_16x16x32_bf16, the 4 waves split
//     K and their partial tiles are added in wave order, rounded once to bf16
//     and stored (nano_ktrans/models/mixtral.py:127, 212).  Last arriver of
//     block tb's counter goes on to B.
//   B (K1): one wave per token, route_token on the block's rows of logits;
//     ids, weights and the selection mask are published.  Last arriver of the
//     all-blocks counter goes on to C.
//   C (K2): the selection masks, ids and weights of every token into LDS,
//     group_scan and group_write as route_group_kernel; the counters and the
//     published masks are reset to zero for the next call (so a graph replay
//     finds them as every call does).
// Data that crosses workgroups (logits, ids, weights, masks) moves by
// agent-scope stores and loads (coherent across the XCDs' L2s); a workgroup's
// waves wait for their stores to complete (vmcnt(0)) and meet at a barrier
// before its one counter increment, so a count that names the last arriver is
// only returned after every part it counts is readable.
// ---------------------------------------------------------------------------
constexpr int kSpTokens = 4;                  // tokens per token block: one wave each
constexpr int kSpThreads = 64 * kSpTokens;
constexpr int kSpExperts = 16;                // router rows per GEMV workgroup (one MFMA row tile)
constexpr int kSpMaxBlocks = kFusedRouteMaxTokens / kSpTokens;
constexpr int kSpMaxH = 8192;                 // rows of x held in LDS: 4 x 8192 bf16
constexpr int kSpKbBatch = 16;                // K blocks of gate weights in flight per wave

enum SpreadMode : int { SP_LOGITS = 0, SP_GEMV = 1, SP_GEMV_NORM = 2 };

struct SpreadArgs {
  const void* logits_in;    // SP_LOGITS: [T, E] act dtype
  const uint16_t* x;        // SP_GEMV*: hidden states [T, H] bf16
  const uint8_t* gate;      // SP_GEMV*: the packed router rows (bf16 blocks)
  const uint16_t* norm_w;   // SP_GEMV_NORM: RMSNorm weight [H] bf16
  float eps;
  uint16_t* normed;         // SP_GEMV_NORM: normalised rows [T, H]
  uint16_t* logits_out;     // SP_GEMV*: [T, E] bf16
  int T, E, k, H;
  unsigned flags;
  int bm, max_tiles;
  int32_t* ids;
  float* w;
  int32_t* counts;
  int32_t* offsets;
  int32_t* perm;
  int32_t* inv;
  int32_t* tiles;
  int32_t* n_tiles;
  int32_t* tile_src;
  const uint8_t* resident;
  float* wpos;
  uint32_t* cnt;      // sync words: [0, kSpMaxBlocks) per token block, [kSpMaxBlocks] all blocks
  uint32_t* masks;    // [T][8] published selection masks (zero between calls)
  int gemv_only;      // SP_GEMV*: phase A alone (logits, normalised rows); no sync words touched
};

template <typename Tv>
__device__ __forceinline__ void agent_store(Tv* p, Tv v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename Tv>
__device__ __forceinline__ Tv agent_load(const Tv* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Every wave's stores complete, the workgroup meets, thread 0 counts it in on
// *c; returns (to every thread) whether this workgroup arrived last of n.
__device__ __forceinline__ bool arrive_last(uint32_t* c, uint32_t n, uint32_t* flag_lds) {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's stores are complete
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag_lds = old == n - 1 ? 1u : 0u;
  }
  __syncthreads();
  return *flag_lds != 0u;
}

// RMSNorm of one bf16 row with the whole wave (rmsnorm_kernel's order: lane
// l adds its 8-column chunks l, l + 64, ... in order, then a fixed
// butterfly); the result to dst0 (LDS) and, when non-null, dst1.  The first
// kNormKept chunks of the lane (H <= 4096) stay in registers for the second
// pass, so it reads x only once (further chunks are read again), and their
// norm weights are loaded with them, before the reduction.
constexpr int kNormKept = 8;

__device__ __forceinline__ void rms_norm_row(const uint16_t* __restrict__ xr, const uint16_t* __restrict__ wr,
                                             float eps, int H, uint16_t* dst0, uint16_t* dst1) {
  const int lane = threadIdx.x & 63;
  u32x4 kept[kNormKept], gk[kNormKept];
#pragma unroll
  for (int i = 0; i < kNormKept; ++i) {
    const int c = lane * 8 + 512 * i;
    kept[i] = c < H ? *(const u32x4*)(xr + c) : u32x4{0u, 0u, 0u, 0u};
    gk[i] = c < H ? *(const u32x4*)(wr + c) : u32x4{0u, 0u, 0u, 0u};
  }
  auto add_sq = [](float ss, u32x4 v) {
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const float a = __uint_as_float(v[h] << 16), b = __uint_as_float(v[h] & 0xffff0000u);
      ss += a * a;
      ss += b * b;
    }
    return ss;
  };
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kNormKept; ++i)
    if (lane * 8 + 512 * i < H) ss = add_sq(ss, kept[i]);
  for (int c = lane * 8 + 512 * kNormKept; c < H; c += 512) ss = add_sq(ss, *(const u32x4*)(xr + c));
  ss = wave_sum_butterfly(ss);
  const float inv = 1.0f / sqrtf(ss / (float)H + eps);
  auto put = [&](int c, u32x4 v, u32x4 g) {
    u32x4 o;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const float a = bf16_round(__uint_as_float(v[h] << 16) * inv);
      const float b = bf16_round(__uint_as_float(v[h] & 0xffff0000u) * inv);
      o[h] = pack_bf16x2(a * __uint_as_float(g[h] << 16), b * __uint_as_float(g[h] & 0xffff0000u));
    }
    *(u32x4*)(dst0 + c) = o;
    if (dst1) *(u32x4*)(dst1 + c) = o;
  };
#pragma unroll
  for (int i = 0; i < kNormKept; ++i)
    if (lane * 8 + 512 * i < H) put(lane * 8 + 512 * i, kept[i], gk[i]);
  for (int c = lane * 8 + 512 * kNormKept; c < H; c += 512) put(c, *(const u32x4*)(xr + c), *(const u32x4*)(wr + c));
}

struct SpreadGemvLds {
  uint16_t xs[kSpTokens * kSpMaxH];  // the block's rows of x (normalised)
  f32x4 red[kSpTokens][64];          // the waves' partial logit tiles
};
struct SpreadRouteLds {
  uint32_t lg[kSpTokens * kMaxExperts / 2];  // the block's rows of bf16 logits
  float sv[kSpTokens][kMaxTopK];
  int si[kSpTokens][kMaxTopK];
  uint32_t sel[kSpTokens][8];
};
struct SpreadGroupLds {
  int32_t ids_s[kFusedRouteMaxPairs];
  float w_s[kFusedRouteMaxPairs];
  uint32_t selmask[kFusedRouteMaxTokens][8];
  GroupLds g;
};

template <int VPL, int MODE, bool BF16>
__global__ void __launch_bounds__(kSpThreads) route_spread_kernel(SpreadArgs a) {
  constexpr int kBytes = sizeof(SpreadGemvLds) > sizeof(SpreadGroupLds) ? sizeof(SpreadGemvLds) : sizeof(SpreadGroupLds);
  __shared__ __attribute__((aligned(16))) uint8_t smem[kBytes > sizeof(SpreadRouteLds) ? kBytes : sizeof(SpreadRouteLds)];
  __shared__ uint32_t flag;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int n_tb = (a.T + kSpTokens - 1) / kSpTokens;
  const int n_eb = MODE == SP_LOGITS ? 1 : (a.E + kSpExperts - 1) / kSpExperts;
  const int tb = blockIdx.x / n_eb;
  const int t0 = tb * kSpTokens;
  const int nt = min(kSpTokens, a.T - t0);

  if (MODE != SP_LOGITS) {
    // ---- A: logits of experts 16 eb .. for the block's tokens -----------
    SpreadGemvLds& L = *(SpreadGemvLds*)smem;
    const int eb = blockIdx.x - tb * n_eb;
    const int H = a.H;
    const int NKB = H / 32;
    const int nkbw = (NKB - wave + kSpTokens - 1) / kSpTokens;  // this wave's K blocks: wave, wave + 4, ...
    const uint8_t* ablk = a.gate + (size_t)eb * NKB * 1024 + lane * 16;
    // the first batch of gate blocks before anything else (HBM latency)
    u32x4 av[kSpKbBatch];
#pragma unroll
    for (int i = 0; i < kSpKbBatch; ++i)
      av[i] = i < nkbw ? *(const u32x4*)(ablk + (size_t)(wave + kSpTokens * i) * 1024) : u32x4{0u, 0u, 0u, 0u};
    if (wave < nt) {
      const uint16_t* xr = a.x + (size_t)(t0 + wave) * H;
      uint16_t* xl = L.xs + wave * H;
      if (MODE == SP_GEMV_NORM) {
        rms_norm_row(xr, a.norm_w, a.eps, H, xl, eb == 0 ? a.normed + (size_t)(t0 + wave) * H : nullptr);
      } else {
        for (int c = lane * 8; c < H; c += 512) *(u32x4*)(xl + c) = *(const u32x4*)(xr + c);
      }
    }
    __syncthreads();
    const int col = lane & 15;
    const uint16_t* xcol = L.xs + col * H + 8 * (lane >> 4);
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int b0 = 0; b0 < nkbw; b0 += kSpKbBatch) {
      if (b0 > 0) {
#pragma unroll
        for (int i = 0; i < kSpKbBatch; ++i)
          av[i] = b0 + i < nkbw ? *(const u32x4*)(ablk + (size_t)(wave + kSpTokens * (b0 + i)) * 1024)
                                : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int i = 0; i < kSpKbBatch; ++i) {
        const int kb = wave + kSpTokens * (b0 + i);
        // columns past the block's tokens multiply zeros (their sums are never stored)
        const u32x4 bv = (col < nt && b0 + i < nkbw) ? *(const u32x4*)(xcol + kb * 32) : u32x4{0u, 0u, 0u, 0u};
        acc = mfma_bf16(av[i], bv, acc);
      }
    }
    L.red[wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
      f32x4 s = L.red[0][lane];
#pragma unroll
      for (int w2 = 1; w2 < kSpTokens; ++w2) s += L.red[w2][lane];
      const int e0 = eb * kSpExperts + 4 * (lane >> 4);
      if (col < nt && e0 < a.E) {  // E % 4 == 0: the four experts are all real
        uint32_t* dst = (uint32_t*)(a.logits_out + (size_t)(t0 + col) * a.E + e0);
        agent_store(dst, pack_bf16x2(s[0], s[1]));
        agent_store(dst + 1, pack_bf16x2(s[2], s[3]));
      }
    }
    if (a.gemv_only) return;  // a later launch reads the logits
    if (!arrive_last(a.cnt + tb, (uint32_t)n_eb, &flag)) return;
  }

  // ---- B: K1 for the block's tokens ----------------------------------------
  {
    SpreadRouteLds& R = *(SpreadRouteLds*)smem;
    if (MODE != SP_LOGITS) {
      const int nw = nt * a.E / 2;
      const uint32_t* src = (const uint32_t*)(a.logits_out + (size_t)t0 * a.E);
      for (int i = threadIdx.x; i < nw; i += kSpThreads) R.lg[i] = agent_load(src + i);
      __syncthreads();
    }
    if (wave < nt) {
      int id;
      float wt;
      if (MODE != SP_LOGITS)
        route_token<VPL, true>(R.lg, wave, a.E, a.k, a.flags, R.sv[wave], R.si[wave], &id, &wt, R.sel[wave]);
      else
        route_token<VPL, BF16>(a.logits_in, t0 + wave, a.E, a.k, a.flags, R.sv[wave], R.si[wave], &id, &wt,
                               R.sel[wave]);
      const int t = t0 + wave;
      if (lane < a.k) {
        agent_store(a.ids + (size_t)t * a.k + lane, id);
        agent_store((uint32_t*)(a.w + (size_t)t * a.k + lane), __float_as_uint(wt));
      }
      wave_lds_sync();
      if (lane < 2 * VPL) agent_store(a.masks + t * 8 + lane, R.sel[wave][lane]);
    }
    if (!arrive_last(a.cnt + kSpMaxBlocks, (uint32_t)n_tb, &flag)) return;
  }

  // ---- C: K2 over every token --------------------------------------------
  SpreadGroupLds& G = *(SpreadGroupLds*)smem;
  unsigned res = 0;
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int e = VPL * lane + i;
      res |= (unsigned)(!a.resident || (e < a.E && a.resident[e])) << i;
    }
  }
  const int P = a.T * a.k;
  for (int i = threadIdx.x; i < P; i += kSpThreads) {
    G.ids_s[i] = agent_load(a.ids + i);
    G.w_s[i] = __uint_as_float(agent_load((const uint32_t*)(a.w + i)));
  }
  for (int i = threadIdx.x; i < a.T * 2 * VPL; i += kSpThreads) {
    const int t = i / (2 * VPL), j = i - t * (2 * VPL);
    G.selmask[t][j] = agent_load(a.masks + t * 8 + j);
    agent_store(a.masks + t * 8 + j, 0u);
  }
  if (threadIdx.x < n_tb) agent_store(a.cnt + threadIdx.x, 0u);
  if (threadIdx.x == 0) agent_store(a.cnt + kSpMaxBlocks, 0u);
  __syncthreads();
  if (wave == 0) group_scan<VPL>(G.selmask, a.T, a.E, a.bm, res, G.g);
  __syncthreads();
  group_write<kSpThreads>(G.g, G.ids_s, a.T, a.k, a.E, a.bm, a.max_tiles, a.counts, a.offsets, a.perm, a.inv, a.tiles,
                          a.n_tiles, a.tile_src, G.w_s, a.wpos);
}

// ---------------------------------------------------------------------------
// K2 from routing the caller computed: the expert side of the reference's
// offload contract (ExpertOffloadBackend.submit_forward(hidden_states,
// topk_ids, topk_weights, stream), nano_ktrans/kernels/offload_backend.py:
// 40-52; kt-kernel's forward_task(bsz, k, expert_ids int64*, weights fp32*,
// input, output, ...), nano_ktrans/kernels/cpu_moe.py:570-592).  Slot j of
// token t names expert ids[t k + j] with weight w[t k + j]; K1 is not run.
// Every later kernel takes a token's k experts to be distinct ids in [0, E),
// as top-k leaves them.  A slot whose id is outside [0, E) or repeats an
// earlier slot's id of the same token is dropped: it takes the smallest
// expert id the token leaves unused, with weight 0 (so the selection stays k
// distinct experts and every later access stays in bounds), and the status
// word gets 1 (it is never cleared here).
// ---------------------------------------------------------------------------

// One wave per token.  Lanes < k return the slot's (sanitised) id and weight;
// *dropped (uniform) says whether a slot was dropped.  selmask (nullable,
// LDS): the token's experts as bits, bit e of word e / 32, words < 2 VPL
// written by lane 0.
template <int VPL>
__device__ __forceinline__ void given_token(const int64_t* __restrict__ ids_in, const float* __restrict__ w_in, int t,
                                            int E, int k, int* out_id, float* out_w, bool* dropped,
                                            uint32_t* selmask = nullptr) {
  const int lane = threadIdx.x & 63;
  int64_t v = -1;
  float w = 0.f;
  if (lane < k) {
    v = ids_in[(int64_t)t * k + lane];
    w = w_in[(int64_t)t * k + lane];
  }
  int id = (v >= 0 && v < E) ? (int)v : -1;
  bool dup = false;
  for (int i = 0; i < k; ++i) {
    const int o = __builtin_amdgcn_readlane(id, i);
    dup = dup || (i < lane && o == id);
  }
  const uint64_t dm = ballot64(lane < k && (id < 0 || dup));
  if (dm) {
    // the kept ids as a 256-bit set, then the dropped slots in slot order each
    // take the smallest free id (at most k - 1 ids are taken and k <= E, so
    // it is below E)
    uint64_t u[4] = {0ull, 0ull, 0ull, 0ull};
    for (int i = 0; i < k; ++i) {
      const int e = __builtin_amdgcn_readlane(id, i);
      if (!((dm >> i) & 1ull)) {
#pragma unroll
        for (int q = 0; q < 4; ++q) u[q] |= (e >> 6) == q ? 1ull << (e & 63) : 0ull;
      }
    }
    for (int i = 0; i < k; ++i) {
      if (!((dm >> i) & 1ull)) continue;
      int f = 0;
#pragma unroll
      for (int q = 3; q >= 0; --q)
        if (~u[q]) f = 64 * q + __builtin_ctzll(~u[q]);
#pragma unroll
      for (int q = 0; q < 4; ++q) u[q] |= (f >> 6) == q ? 1ull << (f & 63) : 0ull;
      if (lane == i) {
        id = f;
        w = 0.f;
      }
    }
  }
  if (selmask) {
#pragma unroll
    for (int wi = 0; wi < 2 * VPL; ++wi) {
      uint32_t word = 0u;
      for (int i = 0; i < k; ++i) {
        const int e = __builtin_amdgcn_readlane(id, i);
        word |= (e >> 5) == wi ? 1u << (e & 31) : 0u;
      }
      if (lane == 0) selmask[wi] = word;
    }
  }
  *out_id = lane < k ? id : -1;
  *out_w = w;
  *dropped = dm != 0ull;
}

// large batches: one wave per token writes the sanitised ids and weights
template <int VPL>
__global__ void __launch_bounds__(256) given_kernel(const int64_t* __restrict__ ids_in, const float* __restrict__ w_in,
                                                    int T, int E, int k, int32_t* __restrict__ ids_out,
                                                    float* __restrict__ w_out, uint32_t* __restrict__ status) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  int id;
  float w;
  bool dropped;
  given_token<VPL>(ids_in, w_in, t, E, k, &id, &w, &dropped);
  if (lane < k) {
    ids_out[(int64_t)t * k + lane] = id;
    w_out[(int64_t)t * k + lane] = w;
  }
  if (dropped && lane == 0) __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// small batches (route_group_fused): the given routing and K2 in one
// workgroup, as route_group_kernel does from logits
template <int VPL>
__global__ void __launch_bounds__(kGroupThreads) given_group_kernel(
    const int64_t* __restrict__ ids_in, const float* __restrict__ w_in, int T, int E, int k, int bm, int max_tiles,
    int32_t* __restrict__ ids_out, float* __restrict__ w_out, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ perm, int32_t* __restrict__ inv,
    int32_t* __restrict__ tiles, int32_t* __restrict__ n_tiles, int32_t* __restrict__ tile_src,
    const uint8_t* __restrict__ resident, float* __restrict__ wpos, uint32_t* __restrict__ status) {
  __shared__ int32_t ids_s[kFusedRouteMaxPairs];
  __shared__ float w_s[kFusedRouteMaxPairs];
  __shared__ uint32_t selmask[kFusedRouteMaxTokens][8];
  __shared__ GroupLds g;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  unsigned res = 0;
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int e = VPL * lane + i;
      res |= (unsigned)(!resident || (e < E && resident[e])) << i;
    }
  }
  bool any_dropped = false;
  for (int t = wave; t < T; t += kGroupWaves) {
    int id;
    float w;
    bool dropped;
    given_token<VPL>(ids_in, w_in, t, E, k, &id, &w, &dropped, selmask[t]);
    any_dropped = any_dropped || dropped;
    if (lane < k) {
      ids_s[t * k + lane] = id;
      w_s[t * k + lane] = w;
      ids_out[(int64_t)t * k + lane] = id;
      w_out[(int64_t)t * k + lane] = w;
    }
  }
  if (any_dropped && lane == 0) __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (wave == 0) group_scan<VPL>(selmask, T, E, bm, res, g);
  __syncthreads();
  group_write(g, ids_s, T, k, E, bm, max_tiles, counts, offsets, perm, inv, tiles, n_tiles, tile_src, w_s, wpos);
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

bool route_spread_ok(int T, int k, int E, int H, bool gemv) {
  if (!route_group_fused(T, k) || E > kMaxExperts) return false;
  return !gemv || (E % 4 == 0 && H % 128 == 0 && H <= kSpMaxH);
}

hipError_t launch_route_spread(const void* logits_in, int act_bf16, const void* x, const void* gate_packed,
                               const void* norm_w, float eps, void* normed, int H, int T, int E, int k,
                               unsigned flags, int bm, int max_tiles, void* logits_out, uint32_t* sync,
                               uint32_t* masks, int32_t* ids, float* w, int32_t* counts, int32_t* offsets,
                               int32_t* perm, int32_t* inv, int32_t* tiles, int32_t* n_tiles, int32_t* tile_src,
                               const uint8_t* resident, float* wpos, hipStream_t stream, bool gemv_only) {
  if (T <= 0) return hipSuccess;
  const bool gemv = x != nullptr;
  if (!route_spread_ok(T, k, E, H, gemv) || (gemv_only && !gemv)) return hipErrorInvalidValue;
  if (gemv ? (!gate_packed || !logits_out || (norm_w && !normed)) : !logits_in) return hipErrorInvalidValue;
  if (!gemv_only) {
    if (bm <= 0 || (bm & (bm - 1)) != 0) return hipErrorInvalidValue;
    if (tile_src && bm != kTileSrcCols) return hipErrorInvalidValue;
    if (!sync || !masks) return hipErrorInvalidValue;
  }
  SpreadArgs a;
  a.logits_in = logits_in;
  a.x = (const uint16_t*)x;
  a.gate = (const uint8_t*)gate_packed;
  a.norm_w = (const uint16_t*)norm_w;
  a.eps = eps;
  a.normed = (uint16_t*)normed;
  a.logits_out = (uint16_t*)logits_out;
  a.T = T;
  a.E = E;
  a.k = k;
  a.H = H;
  a.flags = flags;
  a.bm = bm;
  a.max_tiles = max_tiles;
  a.ids = ids;
  a.w = w;
  a.counts = counts;
  a.offsets = offsets;
  a.perm = perm;
  a.inv = inv;
  a.tiles = tiles;
  a.n_tiles = n_tiles;
  a.tile_src = tile_src;
  a.resident = resident;
  a.wpos = wpos;
  a.cnt = sync;
  a.masks = masks;
  a.gemv_only = gemv_only ? 1 : 0;
  const int n_tb = (T + kSpTokens - 1) / kSpTokens;
  const int n_eb = gemv ? (E + kSpExperts - 1) / kSpExperts : 1;
  dim3 grid(n_tb * n_eb), block(kSpThreads);
#define NKT_SP_CASE(V)                                                                                       \
  case V:                                                                                                    \
    if (!gemv && act_bf16)                                                                                   \
      hipLaunchKernelGGL((route_spread_kernel<V, SP_LOGITS, true>), grid, block, 0, stream, a);              \
    else if (!gemv)                                                                                          \
      hipLaunchKernelGGL((route_spread_kernel<V, SP_LOGITS, false>), grid, block, 0, stream, a);             \
    else if (norm_w)                                                                                         \
      hipLaunchKernelGGL((route_spread_kernel<V, SP_GEMV_NORM, true>), grid, block, 0, stream, a);           \
    else                                                                                                     \
      hipLaunchKernelGGL((route_spread_kernel<V, SP_GEMV, true>), grid, block, 0, stream, a);                \
    break;
  NKT_VPL_SWITCH(E, NKT_SP_CASE)
#undef NKT_SP_CASE
  return hipGetLastError();
}

hipError_t launch_route_group(const void* logits, int act_bf16, int T, int E, int k,
                              unsigned flags, int bm, int max_tiles, int32_t* ids, float* w,
                              int32_t* counts, int32_t* offsets, int32_t* perm, int32_t* inv,
                              int32_t* tiles, int32_t* n_tiles, int32_t* tile_src,
                              const uint8_t* resident, float* wpos, hipStream_t stream) {
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
                         n_tiles, tile_src, resident, wpos);                                    \
    else                                                                                        \
      hipLaunchKernelGGL((route_group_kernel<V, false>), grid, block, 0, stream, logits, T, E,  \
                         k, flags, bm, max_tiles, ids, w, counts, offsets, perm, inv, tiles,    \
                         n_tiles, tile_src, resident, wpos);                                    \
    break;
  NKT_VPL_SWITCH(E, NKT_RG_CASE)
#undef NKT_RG_CASE
  return hipGetLastError();
}

hipError_t launch_given_group(const int64_t* ids_in, const float* w_in, int T, int E, int k, int bm, int max_tiles,
                              int32_t* hist, int32_t* ids, float* w, int32_t* counts, int32_t* offsets, int32_t* perm,
                              int32_t* inv, int32_t* tiles, int32_t* n_tiles, int32_t* tile_src,
                              const uint8_t* resident, float* wpos, uint32_t* status, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  if (bm <= 0 || (bm & (bm - 1)) != 0) return hipErrorInvalidValue;
  if (tile_src && bm != kTileSrcCols) return hipErrorInvalidValue;
  if (!ids_in || !w_in || !status) return hipErrorInvalidValue;
  if (route_group_fused(T, k)) {
#define NKT_GG_CASE(V)                                                                                          \
  case V:                                                                                                       \
    hipLaunchKernelGGL((given_group_kernel<V>), dim3(1), dim3(kGroupThreads), 0, stream, ids_in, w_in, T, E, k, \
                       bm, max_tiles, ids, w, counts, offsets, perm, inv, tiles, n_tiles, tile_src, resident,   \
                       wpos, status);                                                                           \
    break;
    NKT_VPL_SWITCH(E, NKT_GG_CASE)
#undef NKT_GG_CASE
    return hipGetLastError();
  }
#define NKT_GV_CASE(V)                                                                                      \
  case V:                                                                                                   \
    hipLaunchKernelGGL((given_kernel<V>), dim3((T + 3) / 4), dim3(256), 0, stream, ids_in, w_in, T, E, k, ids, \
                       w, status);                                                                          \
    break;
  NKT_VPL_SWITCH(E, NKT_GV_CASE)
#undef NKT_GV_CASE
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_group_multi(ids, T, k, E, bm, max_tiles, hist, counts, offsets, perm, inv, tiles, n_tiles, tile_src,
                            resident, stream);
}

}  // namespace nkt
