// K3, prefill form: grouped SwiGLU expert GEMM for tiles of up to 64
// positions of one expert (prefill-sized groups), on the matrix cores.
//
// Replaces, for large batches, the per-routed-expert loop of
// nano_ktrans/layers/hybrid_moe.py:3501-3533 (SparseExpertMLP /
// PackedSparseExpertMLP.forward, nano_ktrans/layers/expert_mlp.py:20-41) and
// the quantized loop of nano_ktrans/kernels/cpu_moe.py:419-450.
//
// Three kernels share the work order, tile record and epilogue:
//   * gemm2_i8_kernel (int8): 4 waves, three-stage pipeline of 64-wide K
//     stages (tokens direct-to-LDS, weights in a register ring), gate_up on
//     the fp16 matrix cores;
//   * gemm2_i4_kernel (int4 g128): 8 waves, three-stage pipeline of 128-wide
//     K stages (tokens, scales and group sums direct-to-LDS, weights in a
//     register ring);
//   * gemm2_kernel (bf16 weights, and int8 / int4 operands past the
//     pipelines' 32-bit buffer offsets): the register-staged form below.
// The two pipelines also hold copies that compute only the first 16 / 32
// positions of a tile, taken by tiles with no more (an expert's last or
// only tile): the matrix-core work of empty column tiles is skipped, and an
// expert's only tile loads its weights non-temporally.
// Tile = 64 positions x 256 weight rows.  gate_up: the 256 rows are 128 gate
// rows and the 128 matching up rows (a wave holds gate and up rows for the
// same h columns, so SwiGLU is wave-local); down: 256 output rows split over
// the waves.  In gemm2_kernel K advances one 128-wide group per step:
//   * the token tile (64 positions x 128 K, bf16, gathered through the
//     permutation for gate_up) is staged in LDS, double-buffered: the next
//     group's rows load into registers while this group computes;
//   * each wave streams its own weight blocks from HBM into registers (one
//     16-byte load per lane per 1 KiB block), one group ahead;
//   * per group a wave runs 4 (or 2) row tiles x 4 column tiles x 4 K steps of
//     v_mfma_f32_16x16x32_bf16, dequantising each weight fragment once.
// Codes enter the matrix core as exact integers with an offset (int4: bf16
// 136 + q, int8: bf16 128 + q, or fp16 1152 + q in the int8 gate_up); the
// offset times the group's activation sum (precomputed per source row and
// group, fp32) is removed per group for int4, whose group scale then
// multiplies the group's fp32 partial; for int8 the offset times the row's
// total sum is removed once and the per-row scale multiplies the total.
// gate_up also writes the per-position group sums of the bf16 h it stores,
// which the down projection consumes.
#include "nkt_common.h"
#include "nkt_internal.h"
#include "nkt_route_token.h"

namespace nkt {

namespace {

constexpr int kBM = 64;           // positions per tile
constexpr int kCT = kBM / 16;     // 16-position MFMA column tiles

constexpr int kXcds = 8;          // MI355X: accelerator complex dies, each with its own L2

template <int WF, int kRT>
struct ARegs {
  static constexpr int NBLK = 128 / block_k(WF);
  u32x4 w[kRT][NBLK];
  u32x2 s[kRT];
};


}  // namespace

// One workgroup's work item: (token tile, weight slab) and the tile record.
// XCD-aware work order: workgroup b runs on XCD b % 8, so XCD x takes the
// x-th contiguous eighth of the item list, and the items one XCD runs side
// by side share its L2.  The list runs over groups of sg slabs, tile-major
// inside a group.  For small experts (one group of all slabs) the slabs of
// one token tile and the tiles of one expert run together: token rows and
// weight slabs are read from HBM about once.  For experts larger than the
// L2 (sg = 4: Mixtral's 58.7 MB gate_up, Qwen1.5's shared expert) a group
// of 4 slabs runs over the expert's tiles, so a slab's weights are fetched
// once per group instead of once per tile; a last, smaller group takes the
// remaining slabs.  (The 1-D grid is a multiple of 8 and at least
// 8 * per_xcd, so every item below n_items has exactly one workgroup.)
// Returns false for a workgroup without an item.
// slabs per group: all of them unless one expert's weights pass 4 MiB
int slab_group(int n_slabs, int64_t expert_bytes) { return expert_bytes > (4 << 20) ? min(4, n_slabs) : n_slabs; }

struct TileItem {
  int expert, row0, rows, slab;
  bool only;  // the expert's only tile: no other item reads this slab
};

__device__ __forceinline__ bool gemm2_item(const GemmArgs& a, int n_slabs, int sg, TileItem& it) {
  const int n_tiles = a.n_tiles ? a.n_tiles[0] : (a.num_rows + kBM - 1) / kBM;
  const int n_items = n_tiles * n_slabs;
  const int b = blockIdx.x;
  const int per_xcd = (n_items + kXcds - 1) / kXcds;
  const int j = b / kXcds;
  if (j >= per_xcd) return false;
  const int item = (b % kXcds) * per_xcd + j;
  if (item >= n_items) return false;
  const int full = (n_slabs / sg) * n_tiles * sg;  // items in full groups
  int tile;
  if (item < full) {
    const int g = item / (n_tiles * sg);
    const int rem = item - g * n_tiles * sg;
    tile = rem / sg;
    it.slab = g * sg + (rem - tile * sg);
  } else {
    const int last = n_slabs % sg;  // slabs of the last group
    const int rem = item - full;
    tile = rem / last;
    it.slab = (n_slabs / sg) * sg + (rem - tile * last);
  }
  if (a.n_tiles) {
    const int4 rec = *(const int4*)(a.tiles + 4 * tile);
    // an expert's tiles are consecutive records, its full ones first
    const int prev = tile > 0 ? a.tiles[4 * (tile - 1)] : -1;
    it.expert = rec.x;
    it.row0 = rec.y;
    it.rows = rec.z;
    it.only = rec.z < kBM && prev != rec.x;
  } else {
    it.expert = 0;
    it.row0 = tile * kBM;
    it.rows = min(kBM, a.num_rows - it.row0);
    it.only = a.num_rows <= kBM;
  }
  return true;
}

// Source row of each tile position (positions past the tile's rows repeat
// the first) and its output row (down: the pair, so y is in pair order),
// into LDS; the caller's barrier publishes them.
__device__ __forceinline__ void gemm2_sources(const GemmArgs& a, const TileItem& it, int* srcl, int* orow_l) {
  const int tid = threadIdx.x;
  if (tid < kBM) {
    const int p = it.row0 + (tid < it.rows ? tid : 0);
    srcl[tid] = a.perm ? a.perm[p] / a.topk : p;
    orow_l[tid] = a.out_rows ? a.out_rows[p] : p;
  }
}

// Epilogue of the prefill form (shared by its kernels): int8 code offset,
// per-row scales, then gate_up SwiGLU -> bf16 h (+ h's group sums) or down
// fp32 y.  acc[r][c]: this wave's row tile r x column tile c.
// XS (int8 gate_up on the fp16 matrix cores): acc holds sum (1024 + u) x / s
// for the input rows scaled by s; it is rescaled per position and the code
// offset is 1152 (1024 + 128).
template <int kRT>
struct EpiPre {
  bool valid;
  u32x2 s[kRT];
};

// g0, G: the item's K groups [g0, g0 + G) of the a.K / 128 per input row
template <bool XS>
__device__ __forceinline__ bool i8_row_terms(const GemmArgs& a, const int* srcl, float (&v)[16], float& xi, int g0,
                                             int G) {
  if (G > 16) return false;
  const int tid = threadIdx.x;
  if (tid < kBM) {
    const float* xr = a.xsum + (int64_t)srcl[tid] * (a.K / 128) + g0;
#pragma unroll
    for (int g = 0; g < 16; ++g) v[g] = g < G ? xr[g] : 0.f;
    if (XS) xi = a.xinv[srcl[tid]];
  }
  return true;
}

__device__ __forceinline__ void i8_row_terms_store(int G, float* xtot_l, float* xinv_l, const float (&v)[16], float xi,
                                                   bool xs) {
  const int tid = threadIdx.x;
  if (tid < kBM) {
    float t = 0.f;
#pragma unroll
    for (int g = 0; g < 16; ++g)
      if (g < G) t += v[g];
    xtot_l[tid] = t;
    if (xs) xinv_l[tid] = xi;
  }
}

// LDS writes of this wave visible to its other lanes (no workgroup barrier)
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Stores one column tile's rows of 16-bit output through this wave's LDS
// staging rows: lane l holds, for position l % 16, the four columns
// 16 r + 4 (l / 16) .. + 3 of each of its NR row tiles (pk[r]); the 16
// positions' NR x 16 contiguous columns then leave as 16-byte pieces, so a
// store instruction writes whole row segments instead of 16 scattered
// 8-byte pieces.  dst(p): the output row of position p (0..15) at the
// wave's first column; positions >= n_rows are not stored.
template <int NR, typename Dst>
__device__ __forceinline__ void staged_rows_store(uint8_t* stage, const u32x2 (&pk)[NR], int lane, int n_rows, Dst dst) {
  constexpr int RB = NR * 32, SB = RB + 16, LPP = RB / 16, PPI = 64 / LPP;
  const int rq = 4 * (lane >> 4);
#pragma unroll
  for (int r = 0; r < NR; ++r) *(u32x2*)(stage + (lane & 15) * SB + (r * 16 + rq) * 2) = pk[r];
  wave_lds_fence();
#pragma unroll
  for (int i = 0; i < 16 / PPI; ++i) {
    const int pp = i * PPI + lane / LPP;
    const u32x4 v = *(const u32x4*)(stage + pp * SB + (lane % LPP) * 16);
    if (pp < n_rows) *(u32x4*)(dst(pp) + (lane % LPP) * 8) = v;
  }
  wave_lds_fence();  // read before the next column tile rewrites the rows
}

template <int WF, int PHASE, int kWaves, bool XS = false>
__device__ __forceinline__ void gemm2_epilogue(const GemmArgs& a, f32x4 (&acc)[16 / kWaves][kCT], const int* srcl,
                                               const int* orow_l,
                                               float (*hpart)[kBM], float* xtot_l, float* xinv_l, const int* wrow,
                                               const uint16_t* sexp, int row0, int rows, int slab,
                                               const EpiPre<16 / kWaves>* pre = nullptr, uint8_t* stage = nullptr,
                                               int64_t out_off = 0) {
  constexpr int kRT = 16 / kWaves;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int G = a.K / 128;
  const int rq = 4 * (lane >> 4);
  const bool have = pre && pre->valid;
  auto scale_of = [&](int r) -> u32x2 { return have ? pre->s[r] : *(const u32x2*)(sexp + wrow[r] + rq); };
  if (WF == WF_I8) {
    if (!have) {
      if (tid < kBM) {
        const float* xr = a.xsum + (int64_t)srcl[tid] * G;
        float t = 0.f;
        for (int g = 0; g < G; ++g) t += xr[g];
        xtot_l[tid] = t;
        if (XS) xinv_l[tid] = a.xinv[srcl[tid]];
      }
      lds_barrier();
    }
#pragma unroll
    for (int c = 0; c < kCT; ++c) {
      const float cv = (XS ? -1152.0f : -128.0f) * xtot_l[c * 16 + (lane & 15)];
      const float xi = XS ? xinv_l[c * 16 + (lane & 15)] : 1.0f;
#pragma unroll
      for (int r = 0; r < kRT; ++r) {
        if (XS)
          acc[r][c] = acc[r][c] * xi + f32x4{cv, cv, cv, cv};
        else
          acc[r][c] += f32x4{cv, cv, cv, cv};
      }
    }
  }
  if (PHASE == PHASE_GATE_UP) {
    const int hcol0 = slab * 128 + wave * (128 / kWaves);
    constexpr int HR = kRT / 2;
    f32x4 sg[HR], su[HR];
    if (WF == WF_I8) {
#pragma unroll
      for (int r = 0; r < HR; ++r) {
        sg[r] = bf16x4_to_f32(scale_of(r));
        su[r] = bf16x4_to_f32(scale_of(r + HR));
      }
    }
#pragma unroll
    for (int c = 0; c < kCT; ++c) {
      const int pl = c * 16 + (lane & 15);
      float part = 0.f;
#pragma unroll
      for (int r = 0; r < HR; ++r) {
        f32x4 gv = acc[r][c], uv = acc[r + HR][c];
        if (WF == WF_I8) {
          gv *= sg[r];
          uv *= su[r];
        }
        u32x2 pk;
        pk[0] = pack_bf16x2(silu_f32(gv[0]) * uv[0], silu_f32(gv[1]) * uv[1]);
        pk[1] = pack_bf16x2(silu_f32(gv[2]) * uv[2], silu_f32(gv[3]) * uv[3]);
        const f32x4 hb = bf16x4_to_f32(pk);
        part += hb[0];
        part += hb[1];
        part += hb[2];
        part += hb[3];
        // h goes out directly: staged like y below it measured ~2 % slower
        if (pl < rows) *(u32x2*)((uint16_t*)a.out + (int64_t)(row0 + pl) * a.I + hcol0 + r * 16 + rq) = pk;
      }
      // the 4 lanes holding one position's columns: fixed-order butterfly
      part += __shfl_xor(part, 16);
      part += __shfl_xor(part, 32);
      if (lane < 16) hpart[wave][pl] = part;
    }
    if (a.hsum) {
      lds_barrier();
      if (tid < kBM && tid < rows) {
        float s = hpart[0][tid];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) s += hpart[w][tid];
        a.hsum[(int64_t)(row0 + tid) * (a.I / 128) + slab] = s;
      }
    }
  } else if (a.y16) {
    // compact y: per position, the slab's 256 rows as fp16 times 2^sh, sh
    // from the largest |y| of the position in the slab (lanes l, l ^ 16,
    // l ^ 32, l ^ 48 hold one position's rows of this wave; the waves meet
    // in LDS), so that largest value lands in [2^14, 2^15); 2^-sh goes to
    // yscale [position][slab]
    float m[kCT];
#pragma unroll
    for (int c = 0; c < kCT; ++c) m[c] = 0.f;
#pragma unroll
    for (int r = 0; r < kRT; ++r) {
      f32x4 sr = f32x4{1.f, 1.f, 1.f, 1.f};
      if (WF == WF_I8) sr = bf16x4_to_f32(scale_of(r));
#pragma unroll
      for (int c = 0; c < kCT; ++c) {
        if (WF == WF_I8) acc[r][c] *= sr;
#pragma unroll
        for (int v = 0; v < 4; ++v) m[c] = fmaxf(m[c], fabsf(acc[r][c][v]));
      }
    }
#pragma unroll
    for (int c = 0; c < kCT; ++c) {
      m[c] = fmaxf(m[c], __shfl_xor(m[c], 16));
      m[c] = fmaxf(m[c], __shfl_xor(m[c], 32));
      if (lane < 16) hpart[wave][c * 16 + lane] = m[c];
    }
    lds_barrier();
    const int n_slabs = a.N / 256;
#pragma unroll
    for (int c = 0; c < kCT; ++c) {
      const int pl = c * 16 + (lane & 15);
      float mx = hpart[0][pl];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) mx = fmaxf(mx, hpart[w][pl]);
      int sh = 0;
      if (mx > 0.f && mx <= 3.402823466e38f) {
        int e;
        frexpf(mx, &e);
        sh = min(max(15 - e, -126), 126);
      }
      const float sc = __builtin_ldexpf(1.0f, sh);
      u32x2 pk[kRT];
#pragma unroll
      for (int r = 0; r < kRT; ++r)
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const _Float16 lo = (_Float16)(acc[r][c][2 * q] * sc), hi = (_Float16)(acc[r][c][2 * q + 1] * sc);
          pk[r][q] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
        }
      if (pl < rows && wave == 0 && lane < 16) a.yscale[(int64_t)orow_l[pl] * n_slabs + slab] = __builtin_ldexpf(1.0f, -sh);
      if (stage) {
        staged_rows_store(stage, pk, lane, rows - c * 16,
                          [&](int p) { return a.y16 + (int64_t)orow_l[c * 16 + p] * a.N + wrow[0]; });
      } else if (pl < rows) {
        const int64_t orow = orow_l[pl];
#pragma unroll
        for (int r = 0; r < kRT; ++r) *(u32x2*)(a.y16 + orow * a.N + wrow[r] + rq) = pk[r];
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < kRT; ++r) {
      f32x4 sr = f32x4{1.f, 1.f, 1.f, 1.f};
      if (WF == WF_I8) sr = bf16x4_to_f32(scale_of(r));
#pragma unroll
      for (int c = 0; c < kCT; ++c) {
        const int pl = c * 16 + (lane & 15);
        f32x4 v = acc[r][c];
        if (WF == WF_I8) v *= sr;
        if (pl < rows) *(f32x4*)((float*)a.out + out_off + (int64_t)orow_l[pl] * a.N + wrow[r] + rq) = v;
      }
    }
  }
}

template <int WF, int PHASE, int kWaves>
__global__ void __launch_bounds__(64 * kWaves, 2) gemm2_kernel(GemmArgs a, int n_slabs, int sg) {
  constexpr int kRT = 16 / kWaves;  // 16-row weight tiles per wave
  constexpr int NBLK = 128 / block_k(WF);
  // two separate LDS objects (not one array) so the compiler can tell a
  // direct-to-LDS load into one buffer from reads of the other
  __shared__ __attribute__((aligned(1024))) uint8_t bt0[kBM * 256];
  __shared__ __attribute__((aligned(1024))) uint8_t bt1[kBM * 256];
  __shared__ float xsl0[256];  // int4: group sums of the tile rows (each wave loads all; [0, kBM) used)
  __shared__ float xsl1[256];
  __shared__ int srcl[kBM];
  __shared__ int orow_l[kBM];
  __shared__ float hpart[kWaves][kBM];
  __shared__ float xtot_l[kBM];

  TileItem it;
  if (!gemm2_item(a, n_slabs, sg, it)) return;
  const int expert = it.expert, row0 = it.row0, rows = it.rows, slab = it.slab;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int G = a.K / 128;
  const int NKB = a.K / block_k(WF);
  gemm2_sources(a, it, srcl, orow_l);
  __syncthreads();

  // ---- this wave's weight rows ------------------------------------------
  const uint8_t* wexp = a.w + (int64_t)expert * a.w_expert_bytes;
  const uint16_t* sexp = a.scales + (int64_t)expert * a.s_expert_elems;
  int wrow[kRT];
  uint32_t woff[kRT], soff[kRT];
#pragma unroll
  for (int r = 0; r < kRT; ++r) {
    if (PHASE == PHASE_GATE_UP)
      wrow[r] = (r < kRT / 2 ? 0 : a.I) + slab * 128 + wave * (128 / kWaves) + (r % (kRT / 2)) * 16;
    else
      wrow[r] = slab * 256 + wave * (256 / kWaves) + r * 16;
    const uint32_t rb = (uint32_t)(wrow[r] >> 4);
    woff[r] = rb * (uint32_t)NKB * 1024u + (uint32_t)lane * 16u;
    soff[r] = rb * (uint32_t)G * 16u + 4u * (uint32_t)(lane >> 4);
  }

  // ---- token-tile staging: 16 / kWaves x 16 B per thread per group --------
  // A group's tile (kBM rows x 256 B) is stored in LDS unpadded with the
  // 16-byte chunks of row r XOR-swizzled by (r & 15), so the MFMA operand
  // reads below hit 16 distinct bank quads.  Pass i of thread t covers row
  // r = 4 kWaves i + t / 16, chunk t % 16 (so r & 15 = (t / 16) & 15).
  const uint8_t* inb = (const uint8_t*)a.in;
  constexpr int NST = kBM / (4 * kWaves);
  uint32_t boff[NST];
#pragma unroll
  for (int i = 0; i < NST; ++i)
    boff[i] = (uint32_t)srcl[i * 4 * kWaves + (tid >> 4)] * (uint32_t)a.K * 2u + (tid & 15) * 16u;
  const int xs_src = tid < kBM ? srcl[tid] : 0;
  auto load_b = [&](u32x4(&st)[NST], float& xsv, int g) {
#pragma unroll
    for (int i = 0; i < NST; ++i) st[i] = *(const u32x4*)(inb + (boff[i] + (uint32_t)g * 256u));
    if (WF == WF_I4) xsv = a.xsum[(int64_t)xs_src * G + g];
  };
  auto store_b = [&](const u32x4(&st)[NST], float xsv, uint8_t* bt, float* xsl) {
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      const int r = i * 4 * kWaves + (tid >> 4);
      *(u32x4*)(bt + r * 256 + (((tid & 15) ^ (r & 15)) * 16)) = st[i];
    }
    if (WF == WF_I4 && tid < kBM) xsl[tid] = xsv;
  };
  auto load_a = [&](ARegs<WF, kRT>& A, int g) {
#pragma unroll
    for (int r = 0; r < kRT; ++r) {
#pragma unroll
      for (int i = 0; i < NBLK; ++i) A.w[r][i] = *(const u32x4*)(wexp + (woff[r] + (uint32_t)(g * NBLK + i) * 1024u));
      if (WF == WF_I4) A.s[r] = *(const u32x2*)(sexp + (soff[r] + (uint32_t)g * 16u));
    }
  };

  f32x4 acc[kRT][kCT];
#pragma unroll
  for (int r = 0; r < kRT; ++r)
#pragma unroll
    for (int c = 0; c < kCT; ++c) acc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const ARegs<WF, kRT>& A, const uint8_t* bb, const float* xsl) {
    if (WF == WF_I4) {
      // per-group scale: each (row tile, column tile) sums its 4 steps in a
      // temporary that starts at the offset correction, then is scaled in
      u32x4 ad[kRT][4];
      f32x4 sc[kRT];
#pragma unroll
      for (int r = 0; r < kRT; ++r) {
        sc[r] = bf16x4_to_f32(A.s[r]);
#pragma unroll
        for (int s = 0; s < 4; ++s) ad[r][s] = dq_i4(A.w[r][0][s]);
      }
#pragma unroll
      for (int c = 0; c < kCT; ++c) {
        const int prow = c * 16 + (lane & 15);
        u32x4 bf[4];
#pragma unroll
        for (int s = 0; s < 4; ++s)
          bf[s] = *(const u32x4*)(bb + prow * 256 + (((4 * s + (lane >> 4)) ^ (lane & 15)) * 16));
        const float cv = -136.0f * xsl[prow];
#pragma unroll
        for (int r = 0; r < kRT; ++r) {
          f32x4 tmp = f32x4{cv, cv, cv, cv};
#pragma unroll
          for (int s = 0; s < 4; ++s) tmp = mfma_bf16(ad[r][s], bf[s], tmp);
          acc[r][c] += sc[r] * tmp;
        }
      }
    } else {
      // one 32-wide K step at a time: 4 dequantised A fragments and 8 B
      // fragments feed 32 independent accumulators; the next step's B
      // fragments load while this step's MFMAs run (two fragment sets live,
      // pinned by scheduling barriers so the compiler does not hoist more)
      u32x4 bf[2][kCT];
      auto read_b = [&](u32x4(&f)[kCT], int s) {
#pragma unroll
        for (int c = 0; c < kCT; ++c)
          f[c] = *(const u32x4*)(bb + (c * 16 + (lane & 15)) * 256 + (((4 * s + (lane >> 4)) ^ (lane & 15)) * 16));
      };
      read_b(bf[0], 0);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        if (s + 1 < 4) read_b(bf[(s + 1) & 1], s + 1);
        u32x4 ad[kRT];
#pragma unroll
        for (int r = 0; r < kRT; ++r)
          ad[r] = (WF == WF_I8) ? dq_i8(A.w[r][s >> 1][2 * (s & 1)], A.w[r][s >> 1][2 * (s & 1) + 1]) : A.w[r][s];
#pragma unroll
        for (int c = 0; c < kCT; ++c)
#pragma unroll
          for (int r = 0; r < kRT; ++r) acc[r][c] = mfma_bf16(ad[r], bf[s & 1][c], acc[r][c]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  // ---- pipeline ------------------------------------------------------------
  // Two stages: while group g computes from LDS buffer g & 1 and the weight
  // registers A_cur, group g+1's token rows load into staging registers and
  // its weights into A_next; the rows are then written to the other buffer
  // and the workgroup meets at an LDS-only barrier (the weight loads stay in
  // flight).  The loads are pinned above the MFMAs (the scheduler would sink
  // them to their use); past the last group they repeat it (no load behind a
  // branch).  The second workgroup on the CU computes while this one waits.
  ARegs<WF, kRT> A0, A1;
  u32x4 st[NST];
  float xsv = 0.f;
  load_b(st, xsv, 0);
  load_a(A0, 0);
  store_b(st, xsv, bt0, xsl0);
  __syncthreads();
  for (int g = 0; g < G; g += 2) {
    load_b(st, xsv, min(g + 1, G - 1));
    load_a(A1, min(g + 1, G - 1));
    __builtin_amdgcn_sched_barrier(0);
    compute(A0, bt0, xsl0);
    if (g + 1 >= G) break;
    store_b(st, xsv, bt1, xsl1);
    lds_barrier();
    load_b(st, xsv, min(g + 2, G - 1));
    load_a(A0, min(g + 2, G - 1));
    __builtin_amdgcn_sched_barrier(0);
    compute(A1, bt1, xsl1);
    if (g + 2 >= G) break;
    store_b(st, xsv, bt0, xsl0);
    lds_barrier();
  }
  __syncthreads();

  gemm2_epilogue<WF, PHASE, kWaves>(a, acc, srcl, orow_l, hpart, xtot_l, xtot_l, wrow, sexp, row0, rows, slab);
}

// ---------------------------------------------------------------------------
// int8 weights, three-stage pipeline.  Same tile, waves, work order, MFMA
// sequence and epilogue as gemm2_kernel<WF_I8, ...> (so the results are the
// same bit for bit); K advances in 64-wide stages:
//   * weights: each wave's own 4 row tiles, one 1 KiB block (16 rows x 64 K,
//     lane l's MFMA fragments at 16 l) per row tile, loaded by buffer loads
//     straight into a ring of three register stages (the weights are private
//     to the wave, so they never touch LDS);
//   * tokens: 64 positions x 128 B per stage reach one of three LDS buffers
//     by direct-to-LDS buffer loads (8 loads of 8 positions, 2 per wave);
//     lane l carries position 8 i + l / 8 into LDS slot l % 8 of that
//     position's row, fetched from source chunk (l % 8) ^ ((position / 2) % 8):
//     the MFMA operand reads of 16 consecutive positions cover all 64 LDS
//     banks;
//   * step x: wait for this wave's loads of stage x + 1's tokens and stage
//     x's weights, meet at one LDS-only barrier, start stage x + 3's tokens
//     (into the buffer stage x was read from) and stage x + 2's weights,
//     read stage x + 1's token fragments from LDS, run stage x's MFMAs.
// Three separate LDS objects: the compiler tells a direct-to-LDS load into
// one buffer from reads of another and waits only where they alias.  Loads
// past the last stage use an out-of-range buffer offset: they read nothing
// and keep the per-step load count (6) fixed, so the wait is always "all
// but the newest 6".
// ---------------------------------------------------------------------------
constexpr int kI8Stage = 64;                   // K per stage
constexpr int kI8TokBytes = kBM * kI8Stage * 2;
constexpr uint32_t kI8Skip = 0xFFFFFF00u;     // a buffer offset past every range the kernel is given

template <int PHASE, bool F16>
__global__ void __launch_bounds__(256, 2) gemm2_i8_kernel(GemmArgs a, int n_slabs, int sg) {
  constexpr int kWaves = 4;
  constexpr int kRT = 4;
  __shared__ __attribute__((aligned(1024))) uint8_t tb0[kI8TokBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t tb1[kI8TokBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t tb2[kI8TokBytes];
  __shared__ int srcl[kBM];
  __shared__ int orow_l[kBM];
  __shared__ float hpart[kWaves][kBM];
  __shared__ float xtot_l[kBM];
  __shared__ float xinv_l[kBM];

  TileItem it;
  if (!gemm2_item(a, n_slabs, sg, it)) return;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  gemm2_sources(a, it, srcl, orow_l);
  __syncthreads();

  // down in K parts: item slab s is K part s / (N / 256) of slab s % (N / 256)
  int kpart = 0;
  if (PHASE == PHASE_DOWN && a.k_parts > 1) {
    kpart = it.slab / (a.N / 256);
    it.slab -= kpart * (a.N / 256);
  }
  const int Kp = (PHASE == PHASE_DOWN && a.k_parts > 1) ? a.K / a.k_parts : a.K;  // this item's K range
  const uint16_t* sexp = a.scales + (int64_t)it.expert * a.s_expert_elems;
  const int NS = Kp / kI8Stage;         // stages this item runs
  const int NSrow = a.K / kI8Stage;     // 1 KiB blocks per 16-row block
  // buffer resources over this expert's weights and the activation rows; a
  // load at offset kI8Skip is out of range: it reads nothing (zeros)
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.w + (int64_t)it.expert * a.w_expert_bytes), (short)0, a.N * a.K, 0x00020000);
  const __amdgpu_buffer_rsrc_t tres = __builtin_amdgcn_make_buffer_rsrc((void*)a.in, (short)0, a.in_bytes, 0x00020000);
  int wrow[kRT];
  uint32_t wsrc[kRT];
#pragma unroll
  for (int r = 0; r < kRT; ++r) {
    if (PHASE == PHASE_GATE_UP)
      wrow[r] = (r < kRT / 2 ? 0 : a.I) + it.slab * 128 + wave * (128 / kWaves) + (r % (kRT / 2)) * 16;
    else
      wrow[r] = it.slab * 256 + wave * (256 / kWaves) + r * 16;
    wsrc[r] = ((uint32_t)(wrow[r] >> 4) * (uint32_t)NSrow + (uint32_t)(kpart * NS)) * 1024u + lane * 16u;
  }
  uint32_t tsrc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int p = 16 * wave + 8 * j + (lane >> 3);
    const int chunk = (lane & 7) ^ ((p >> 1) & 7);
    tsrc[j] = ((uint32_t)srcl[p] * (uint32_t)a.K + (uint32_t)(kpart * Kp)) * 2u + chunk * 16u;
  }
  const int tofs = wave * 2048;  // this wave's slice of a token buffer

  // stage st's 2 token loads into tb (st >= NS: out of range, no traffic)
  auto issue_tok = [&](int st, uint8_t* tb) {
    const bool live = st < NS;
#pragma unroll
    for (int j = 0; j < 2; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(tres, (__attribute__((address_space(3))) void*)(tb + tofs + j * 1024),
                                               16, live ? tsrc[j] + st * (kI8Stage * 2u) : kI8Skip, 0, 0, 0);
  };
  // stage st's 4 weight blocks into registers, with the copy's load policy
  // (nt for an expert's only tile: no other item reads its weights)
  auto issue_w = [&](auto nc, int st, u32x4 (&w)[kRT]) {
    constexpr int kPolicy = decltype(nc)::value >> 4;
    const bool live = st < NS;
#pragma unroll
    for (int r = 0; r < kRT; ++r)
      w[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wres, live ? wsrc[r] + st * 1024u : kI8Skip, 0, kPolicy));
  };

  f32x4 acc[kRT][kCT];
#pragma unroll
  for (int r = 0; r < kRT; ++r)
#pragma unroll
    for (int c = 0; c < kCT; ++c) acc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  // one stage's token fragments (2 K steps x the first NC of the 4 column
  // tiles: a tile of at most 16 / 32 / 48 positions, an expert's last or
  // only one, runs only 1 / 2 / 3 column tiles' fragment reads and
  // matrix-core work; the other sums stay zero and are never stored)
  typedef u32x4 TokFrags[2][kCT];
  auto read_tok = [&](auto nc, TokFrags& f, const uint8_t* tb) {
    constexpr int NC = decltype(nc)::value & 15;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int p = c * 16 + (lane & 15);
        const int chunk = 4 * s + (lane >> 4);
        f[s][c] = *(const u32x4*)(tb + p * (kI8Stage * 2) + ((chunk ^ ((p >> 1) & 7)) * 16));
      }
  };
  auto mma = [&](auto nc, const u32x4 (&w)[kRT], const TokFrags& f) {
    constexpr int NC = decltype(nc)::value & 15;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      u32x4 ad[kRT];
#pragma unroll
      for (int r = 0; r < kRT; ++r) ad[r] = F16 ? dq_i8_f16(w[r][2 * s], w[r][2 * s + 1]) : dq_i8(w[r][2 * s], w[r][2 * s + 1]);
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int r = 0; r < kRT; ++r)
          acc[r][c] = F16 ? mfma_f16(ad[r], f[s][c], acc[r][c]) : mfma_bf16(ad[r], f[s][c], acc[r][c]);
    }
  };

  TokFrags f0, f1;
  u32x4 w0[kRT], w1[kRT], w2[kRT];
  // issue order: T0, T1, W0, T2, W1, then per step x: T(x + 3), W(x + 2);
  // at step x the newest 6 loads are T(x + 2) and W(x + 1), so waiting for
  // all but 6 covers T(x + 1) and W(x)
  auto step = [&](auto nc, TokFrags& cur, TokFrags& nxt, const u32x4 (&wcur)[kRT], u32x4 (&wnew)[kRT],
                  uint8_t* tb_x, const uint8_t* tb_n, int x) {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0x0F76);  // vmcnt(6)
    lds_barrier();
    issue_tok(x + 3, tb_x);
    issue_w(nc, x + 2, wnew);
    read_tok(nc, nxt, tb_n);
    mma(nc, wcur, cur);
    __builtin_amdgcn_sched_barrier(0);
  };

  // the rest of the item for the first NC column tiles, one copy of the
  // pipeline per NC (a branch per column tile inside one copy cost more than
  // it saved on full tiles); measured against always 4: Qwen3 int8 T = 128
  // (even routing) 142.7 -> 134.2 us per layer, Qwen1.5-MoE T = 128 / 1024
  // 172.4 -> 163.3 / 243.5 -> 236.8, Qwen3 int8 Zipf T = 1024 / 4096
  // 176.2 -> 173.3 / 441.9 -> 433.5, T = 512 unchanged
  auto run = [&](auto nc) {
    EpiPre<kRT> pre;
    float rv[16], rxi = 0.f;
    pre.valid = i8_row_terms<F16>(a, srcl, rv, rxi, kpart * (Kp / 128), Kp / 128);
    if (pre.valid) {
#pragma unroll
      for (int r = 0; r < kRT; ++r) pre.s[r] = *(const u32x2*)(sexp + wrow[r] + 4 * (lane >> 4));
    }
    issue_tok(0, tb0);
    issue_tok(1, tb1);
    issue_w(nc, 0, w0);
    issue_tok(2, tb2);
    issue_w(nc, 1, w1);
    if (pre.valid) i8_row_terms_store(Kp / 128, xtot_l, xinv_l, rv, rxi, F16);
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0x0F7C);  // vmcnt(12): T0 landed
    lds_barrier();
    read_tok(nc, f0, tb0);
    // six steps per iteration return fragments, weight registers and buffers
    // to their starting roles; the last NS % 6 steps follow
    int x = 0;
    for (; x + 6 <= NS; x += 6) {
      step(nc, f0, f1, w0, w2, tb0, tb1, x);
      step(nc, f1, f0, w1, w0, tb1, tb2, x + 1);
      step(nc, f0, f1, w2, w1, tb2, tb0, x + 2);
      step(nc, f1, f0, w0, w2, tb0, tb1, x + 3);
      step(nc, f0, f1, w1, w0, tb1, tb2, x + 4);
      step(nc, f1, f0, w2, w1, tb2, tb0, x + 5);
    }
    const int rest = NS - x;
    if (rest >= 1) step(nc, f0, f1, w0, w2, tb0, tb1, x);
    if (rest >= 2) step(nc, f1, f0, w1, w0, tb1, tb2, x + 1);
    if (rest >= 3) step(nc, f0, f1, w2, w1, tb2, tb0, x + 2);
    if (rest >= 4) step(nc, f1, f0, w0, w2, tb0, tb1, x + 3);
    if (rest >= 5) step(nc, f0, f1, w1, w0, tb1, tb2, x + 4);
    wait_vmem();  // out-of-range loads past the last stage land before the LDS is reused
    __syncthreads();
    // down's compact y staging: 16 rows of 144 B per wave in the token
    // buffers, free once every wave has passed the barrier above
    uint8_t* stage = wave < 3 ? tb0 + wave * 2304 : tb1;
    gemm2_epilogue<WF_I8, PHASE, kWaves, F16>(a, acc, srcl, orow_l, hpart, xtot_l, xinv_l, wrow, sexp, it.row0, it.rows,
                                              it.slab, &pre, PHASE == PHASE_DOWN ? stage : nullptr,
                                              (int64_t)kpart * a.num_rows * a.N);
  };
  // copy tag: column tiles | weight load policy << 4.  Measured against
  // short-tile copies with the default policy throughout: Qwen3 int8 T =
  // 128 / 256 (even routing) 133 / 141 -> 126 / 131 us per layer, Qwen1.5-MoE
  // T = 128 / 320 163 / 153 -> 155 / 144, Zipf routing and Qwen1.5 T = 1024
  // level; the nt policy for every short tile (an expert's last of several
  // too) lost 5 - 8 % at Qwen1.5 T = 1024, whose experts end in such tiles.
  // The 3-column-tile copies (33 - 48 positions) then: Qwen3 int8 T = 512
  // (even routing) 151.3 -> 140.5 us, Qwen1.5-MoE T = 512 / 640 174 / 189.6
  // -> 165.3 / 183
  const int urows = __builtin_amdgcn_readfirstlane(it.rows);
  const bool only = __builtin_amdgcn_readfirstlane((int)it.only) != 0;
  if (urows <= 16) {
    if (only)
      run(std::integral_constant<int, 1 | 2 << 4>{});
    else
      run(std::integral_constant<int, 1>{});
  } else if (urows <= 32) {
    if (only)
      run(std::integral_constant<int, 2 | 2 << 4>{});
    else
      run(std::integral_constant<int, 2>{});
  } else if (urows <= 48) {
    if (only)
      run(std::integral_constant<int, 3 | 2 << 4>{});
    else
      run(std::integral_constant<int, 3>{});
  } else {
    run(std::integral_constant<int, kCT>{});
  }
}

// Per-row sums of each 128-wide K group of a bf16 matrix [rows, K] -> fp32
// [rows, K/128].  One wave per row; lane l adds its 8 consecutive values,
// then the 16 lanes of a group reduce by xor butterfly (8, 4, 2, 1).
__global__ void __launch_bounds__(256) group_sums_kernel(const uint16_t* __restrict__ x, int rows, int K,
                                                         float* __restrict__ out) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const uint16_t* xr = x + (int64_t)row * K;
  const int G = K / 128;
  for (int g0 = 0; g0 < G; g0 += 4) {
    const int g = g0 + (lane >> 4);
    float s = 0.f;
    if (g < G) {
      const u32x4 v = *(const u32x4*)(xr + g * 128 + (lane & 15) * 8);
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        s += __uint_as_float(v[h] << 16);
        s += __uint_as_float(v[h] & 0xffff0000u);
      }
    }
    s += __shfl_xor(s, 8);
    s += __shfl_xor(s, 4);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 1);
    if ((lane & 15) == 0 && g < G) out[(int64_t)row * G + g] = s;
  }
}

// the int8 pipeline addresses its operands with 32-bit buffer offsets
bool gemm2_i8_pipeline(const GemmArgs& a, int wf) {
  return wf == WF_I8 && a.in_bytes <= (int64_t)kI8Skip && (int64_t)a.N * a.K <= (int64_t)kI8Skip;
}

// the int4 pipeline addresses weights, scales, group sums and activations
// with 32-bit buffer offsets (bf16 activations)
bool gemm2_i4_pipeline(const GemmArgs& a, int wf) {
  if (wf != WF_I4 || !a.act_bf16 || a.in_bytes <= 0) return false;
  const int64_t rows_in = a.in_bytes / ((int64_t)a.K * 2);
  return a.in_bytes <= (int64_t)kI8Skip && a.w_expert_bytes <= (int64_t)kI8Skip &&
         a.s_expert_elems * 2 <= (int64_t)kI8Skip && rows_in * (a.K / 128) * 4 <= (int64_t)kI8Skip;
}

bool gemm2_supported(int wf, int phase, int N, int K, int I) {
  if (wf != WF_BF16 && wf != WF_I8 && wf != WF_I4) return false;
  if (K % 128 != 0) return false;
  return phase == PHASE_GATE_UP ? (I % 128 == 0) : (N % 256 == 0);
}

// ---------------------------------------------------------------------------
// int4 g128 weights, three-stage pipeline.  Same tile, waves (8, two 16-row
// tiles each), work order, MFMA and scaling sequence and epilogue as
// gemm2_kernel<WF_I4, ...> (so the results are the same bit for bit); K
// advances one 128-wide scale group per stage:
//   * tokens: 64 positions x 256 B per stage reach one of three LDS buffers
//     by direct-to-LDS buffer loads (16 loads of 4 positions, 2 per wave);
//     lane l carries position 4 i + l / 16 into slot l % 16 of that
//     position's row, fetched from chunk (l % 16) ^ (position % 16), so the
//     MFMA operand reads of 16 consecutive positions cover all 64 banks;
//   * each wave's two 1 KiB weight blocks go by buffer loads straight into a
//     three-deep register ring; their bf16 scales (lanes 0-15, 4 bytes
//     each) and the 64 positions' activation group sums (4 bytes per lane)
//     reach the wave's own slice of a small LDS buffer by direct-to-LDS
//     loads;
//   * step x: wait for this wave's loads of stage x (all but the newest 6,
//     the loads of stage x + 1), one LDS-only barrier (every wave is also
//     done reading stage x - 1's buffers), start stage x + 2's loads into
//     those buffers and that ring slot, then stage x: four MFMAs per (row
//     tile, column tile) into a temporary that starts at the code offset,
//     the 8 temporaries advancing together, then scaled into the
//     accumulators.
// Loads past the last stage take an out-of-range buffer offset (no
// traffic), so every step issues the same 6.  Six LDS objects: the compiler
// tells a direct-to-LDS load into one from reads of another.
// ---------------------------------------------------------------------------
constexpr int kI4TokBytes = kBM * 256;
constexpr int kI4SxBytes = 8 * 512;  // per wave: 256 B scales (64 used), 256 B group sums

template <int PHASE, bool NARROW>
__global__ void __launch_bounds__(512, 1) gemm2_i4_kernel(GemmArgs a, int n_slabs, int sg) {
  constexpr int kWaves = 8;
  constexpr int kRT = 2;
  __shared__ __attribute__((aligned(1024))) uint8_t tb0[kI4TokBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t tb1[kI4TokBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t tb2[kI4TokBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t sx0[kI4SxBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t sx1[kI4SxBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t sx2[kI4SxBytes];
  __shared__ int srcl[kBM];
  __shared__ int orow_l[kBM];
  __shared__ float hpart[kWaves][kBM];
  __shared__ float xtot_l[kBM];

  TileItem it;
  if (!gemm2_item(a, n_slabs, sg, it)) return;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  gemm2_sources(a, it, srcl, orow_l);
  __syncthreads();

  const uint16_t* sexp = a.scales + (int64_t)it.expert * a.s_expert_elems;
  const int G = a.K / 128;  // stages = scale groups = 1 KiB blocks per 16-row block
  const int rows_in = (int)(a.in_bytes / ((int64_t)a.K * 2));
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.w + (int64_t)it.expert * a.w_expert_bytes), (short)0, (int)a.w_expert_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t sres =
      __builtin_amdgcn_make_buffer_rsrc((void*)sexp, (short)0, (int)(a.s_expert_elems * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t xres =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.xsum, (short)0, rows_in * G * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t tres = __builtin_amdgcn_make_buffer_rsrc((void*)a.in, (short)0, (int)a.in_bytes, 0x00020000);
  int wrow[kRT];
  uint32_t wsrc[kRT];
#pragma unroll
  for (int r = 0; r < kRT; ++r) {
    if (PHASE == PHASE_GATE_UP)
      wrow[r] = (r == 0 ? 0 : a.I) + it.slab * 128 + wave * 16;
    else
      wrow[r] = it.slab * 256 + wave * 32 + r * 16;
    wsrc[r] = (uint32_t)(wrow[r] >> 4) * (uint32_t)G * 1024u + lane * 16u;
  }
  // scale lane (lanes 16-63 repeat lanes 0-15): row tile (l % 16) / 8, 4-byte piece l % 8
  const int sl = lane & 15;
  const uint32_t ssrc = ((uint32_t)(wrow[sl >> 3] >> 4) * (uint32_t)G * 16u) * 2u + (sl & 7) * 4u;
  const uint32_t xsrc = (uint32_t)srcl[lane] * (uint32_t)G * 4u;
  uint32_t tsrc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int p = 8 * wave + 4 * j + (lane >> 4);
    const int chunk = (lane & 15) ^ (p & 15);
    tsrc[j] = (uint32_t)srcl[p] * (uint32_t)a.K * 2u + chunk * 16u;
  }
  const int tofs = wave * 2048;  // this wave's slice of a token buffer
  const int sofs = wave * 512;   // and of a scale / group-sum buffer

  // stage st's 6 loads (st >= G: out of range, no traffic), the weights
  // with the copy's load policy (tag >> 4: nt for an expert's only tile)
  auto issue = [&](auto nc, int st, uint8_t* tb, uint8_t* sx, u32x4 (&w)[kRT]) {
    constexpr int kPolicy = decltype(nc)::value >> 4;
    const bool live = st < G;
#pragma unroll
    for (int j = 0; j < 2; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(tres, (__attribute__((address_space(3))) void*)(tb + tofs + j * 1024),
                                               16, live ? tsrc[j] + st * 256u : kI8Skip, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(sres, (__attribute__((address_space(3))) void*)(sx + sofs), 4,
                                             live ? ssrc + st * 32u : kI8Skip, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(xres, (__attribute__((address_space(3))) void*)(sx + sofs + 256), 4,
                                             live ? xsrc + st * 4u : kI8Skip, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < kRT; ++r)
      w[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wres, live ? wsrc[r] + st * 1024u : kI8Skip, 0, kPolicy));
  };

  f32x4 acc[kRT][kCT];
#pragma unroll
  for (int r = 0; r < kRT; ++r)
#pragma unroll
    for (int c = 0; c < kCT; ++c) acc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  // all (row tile, column tile) temporaries advance one K step at a time,
  // so no MFMA waits on the one before it; only the first NC column tiles
  auto compute = [&](auto nc, const u32x4 (&w)[kRT], const uint8_t* tb, const uint8_t* sx) {
    constexpr int NC = decltype(nc)::value & 15;
    u32x4 bf[kCT][4];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int p = c * 16 + (lane & 15);
#pragma unroll
      for (int s = 0; s < 4; ++s) bf[c][s] = *(const u32x4*)(tb + p * 256 + (((4 * s + (lane >> 4)) ^ (p & 15)) * 16));
    }
    u32x4 ad[kRT][4];
    f32x4 sc[kRT];
    const DqConst kdq = dq_const();
#pragma unroll
    for (int r = 0; r < kRT; ++r) {
      sc[r] = bf16x4_to_f32(*(const u32x2*)(sx + sofs + r * 32 + (lane >> 4) * 8));
#pragma unroll
      for (int s = 0; s < 4; ++s) ad[r][s] = dq_i4_k(w[r][s], kdq);
    }
    f32x4 tmp[kRT][kCT];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float cv = -136.0f * *(const float*)(sx + sofs + 256 + (c * 16 + (lane & 15)) * 4);
#pragma unroll
      for (int r = 0; r < kRT; ++r) tmp[r][c] = f32x4{cv, cv, cv, cv};
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int r = 0; r < kRT; ++r) tmp[r][c] = mfma_bf16(ad[r][s], bf[c][s], tmp[r][c]);
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int r = 0; r < kRT; ++r) acc[r][c] += sc[r] * tmp[r][c];
  };

  u32x4 w0[kRT], w1[kRT], w2[kRT];
  auto step = [&](auto nc, const u32x4 (&wcur)[kRT], u32x4 (&wn2)[kRT], const uint8_t* tb_x, const uint8_t* sx_x,
                  uint8_t* tb_n2, uint8_t* sx_n2, int x) {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0x0F76);  // vmcnt(6): stage x landed (stage x + 1's 6 may fly)
    lds_barrier();
    issue(nc, x + 2, tb_n2, sx_n2, wn2);
    compute(nc, wcur, tb_x, sx_x);
    __builtin_amdgcn_sched_barrier(0);
  };
  // the pipeline over the first NC column tiles, one copy per NC
  auto run = [&](auto nc) {
    issue(nc, 0, tb0, sx0, w0);
    issue(nc, 1, tb1, sx1, w1);
    // three steps per iteration return ring slots and buffers to their roles
    int x = 0;
    for (; x + 3 <= G; x += 3) {
      step(nc, w0, w2, tb0, sx0, tb2, sx2, x);
      step(nc, w1, w0, tb1, sx1, tb0, sx0, x + 1);
      step(nc, w2, w1, tb2, sx2, tb1, sx1, x + 2);
    }
    if (x < G) step(nc, w0, w2, tb0, sx0, tb2, sx2, x);
    if (x + 1 < G) step(nc, w1, w0, tb1, sx1, tb0, sx0, x + 1);
    wait_vmem();  // out-of-range loads past the last stage land before the LDS is reused
    __syncthreads();
    gemm2_epilogue<WF_I4, PHASE, kWaves>(a, acc, srcl, orow_l, hpart, xtot_l, xtot_l, wrow, sexp, it.row0, it.rows,
                                         it.slab);
  };
  // NARROW (experts average at most 48 positions): a tile of at most 16 / 32
  // / 48 positions, an expert's last or only one, runs 1 / 2 / 3 of its 4
  // column tiles (3: Qwen3 int4 T = 448 / 512 137.9 / 141.7 -> 129.1 / 133.3
  // us, Mixtral T = 128 284.8 -> 265.7), an only tile with nt weight loads (T = 300 / 384 a further 124.5 /
  // 130.9 -> 120.2 / 126.3 us with the nt copy; the 1-tile copy then T = 200
  // / 256 / 300 114.9 / 116 / 117.5 -> 104.8 / 112.1 / 114.1 us).
  // Measured: Qwen3 int4 T = 300 (even routing) 149 -> 124.6 us per layer;
  // with the 1- and 2-tile copies the switch at 32 positions per expert
  // measured best (Qwen3 int4 T = 448 / 512 153.6 / 147.6 -> 139 / 144 us,
  // Mixtral T = 128 307 -> 292.5 against 24; at 48 T = 768 173.5 -> 178.5),
  // with the 3-tile copies 48 (against 32: T = 640 / 768 154.5 / 172.6 ->
  // 148 / 169.8, Mixtral T = 160 / 192 305.4 / 299.6 -> 279.5 / 289); where
  // experts hold many full tiles the copies cost 1 - 5 % (Mixtral T = 2048,
  // Qwen3 int4 Zipf T = 2048), hence the launch-wide switch
  if constexpr (NARROW) {
    // copy tag: column tiles | weight load policy << 4
    const int urows = __builtin_amdgcn_readfirstlane(it.rows);
    const bool only = __builtin_amdgcn_readfirstlane((int)it.only) != 0;
    if (urows <= 16) {
      if (only)
        run(std::integral_constant<int, 1 | 2 << 4>{});
      else
        run(std::integral_constant<int, 1>{});
    } else if (urows <= 32) {
      if (only)
        run(std::integral_constant<int, 2 | 2 << 4>{});
      else
        run(std::integral_constant<int, 2>{});
    } else if (urows <= 48) {
      if (only)
        run(std::integral_constant<int, 3 | 2 << 4>{});
      else
        run(std::integral_constant<int, 3>{});
    } else {
      run(std::integral_constant<int, kCT>{});
    }
  } else {
    // (the same pipeline written out: a launch of full tiles keeps the
    // schedule the compiler gives it without the lambda, 1 - 2 % faster)
    const std::integral_constant<int, kCT> nc;
    issue(nc, 0, tb0, sx0, w0);
    issue(nc, 1, tb1, sx1, w1);
    int x = 0;
    for (; x + 3 <= G; x += 3) {
      step(nc, w0, w2, tb0, sx0, tb2, sx2, x);
      step(nc, w1, w0, tb1, sx1, tb0, sx0, x + 1);
      step(nc, w2, w1, tb2, sx2, tb1, sx1, x + 2);
    }
    if (x < G) step(nc, w0, w2, tb0, sx0, tb2, sx2, x);
    if (x + 1 < G) step(nc, w1, w0, tb1, sx1, tb0, sx0, x + 1);
    wait_vmem();
    __syncthreads();
    gemm2_epilogue<WF_I4, PHASE, kWaves>(a, acc, srcl, orow_l, hpart, xtot_l, xtot_l, wrow, sexp, it.row0, it.rows,
                                         it.slab);
  }
}

// Input of the int8 gate_up on the fp16 matrix cores, one wave per row: the
// group sums exactly as group_sums_kernel, and the row times s = 2^(15 - E)
// rounded to fp16, where the row's largest |x| is f 2^E with f in [0.5, 1)
// (s = 1 for an all-zero or non-finite row).  The scaled maximum lies in
// [2^14, 2^15), and every bf16 value down to 2^-32 of it is exact in fp16
// (normal down to 2^-14, subnormal with 8 significant bits down to 2^-17).
// xinv = 1 / s.  Lane l holds 8 values of group 4c + l / 16 per chunk c.
// block: this launch's index of the workgroup (four rows).
template <int NCH>
__device__ __forceinline__ void prep_f16_rows(const uint16_t* __restrict__ x, int rows, int K,
                                              float* __restrict__ sums, uint16_t* __restrict__ x16,
                                              float* __restrict__ xinv, int block) {
  const int row = block * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const uint16_t* xr = x + (int64_t)row * K;
  const int G = K / 128;
  u32x4 v[NCH];
  float m = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int g = 4 * c + (lane >> 4);
    v[c] = u32x4{0u, 0u, 0u, 0u};
    if (g < G) v[c] = *(const u32x4*)(xr + g * 128 + (lane & 15) * 8);
    float s = 0.f;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const float lo = __uint_as_float(v[c][h] << 16), hi = __uint_as_float(v[c][h] & 0xffff0000u);
      s += lo;
      s += hi;
      m = fmaxf(m, fmaxf(fabsf(lo), fabsf(hi)));
    }
    s += __shfl_xor(s, 8);
    s += __shfl_xor(s, 4);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 1);
    if ((lane & 15) == 0 && g < G) sums[(int64_t)row * G + g] = s;
  }
  m = wave_max(m);
  int e = 0;
  if (m > 0.f && m <= 3.402823466e38f) {
    int E;
    frexpf(m, &E);
    e = min(max(15 - E, -126), 126);
  }
  const float sc = __builtin_ldexpf(1.0f, e);
  uint16_t* xo = x16 + (int64_t)row * K;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int g = 4 * c + (lane >> 4);
    if (g >= G) continue;
    u32x4 o;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const _Float16 lo = (_Float16)(__uint_as_float(v[c][h] << 16) * sc);
      const _Float16 hi = (_Float16)(__uint_as_float(v[c][h] & 0xffff0000u) * sc);
      o[h] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
    }
    *(u32x4*)(xo + g * 128 + (lane & 15) * 8) = o;
  }
  if (lane == 0) xinv[row] = __builtin_ldexpf(1.0f, -e);
}

template <int NCH>
__global__ void __launch_bounds__(256) prep_f16_kernel(const uint16_t* __restrict__ x, int rows, int K,
                                                       float* __restrict__ sums, uint16_t* __restrict__ x16,
                                                       float* __restrict__ xinv) {
  prep_f16_rows<NCH>(x, rows, K, sums, x16, xinv, blockIdx.x);
}

// K1 (one wave per token, as route_kernel) and the fp16 input of the int8
// gate_up (as prep_f16_kernel) in one launch: workgroups 0 .. ceil(T / 4) - 1
// route four tokens each, the rest prepare four rows of x each.  The two
// are independent; one launch instead of two in the prefill layer.
template <int VPL, int NCH>
__global__ void __launch_bounds__(256) route_prep_f16_kernel(const uint16_t* __restrict__ logits, int T, int E,
                                                             int k, unsigned flags, int32_t* __restrict__ ids_out,
                                                             float* __restrict__ w_out, int route_blocks,
                                                             const uint16_t* __restrict__ x, int rows, int K,
                                                             float* __restrict__ sums, uint16_t* __restrict__ x16,
                                                             float* __restrict__ xinv) {
  __shared__ float sv[4][kMaxTopK];
  __shared__ int si[4][kMaxTopK];
  if ((int)blockIdx.x >= route_blocks) {
    prep_f16_rows<NCH>(x, rows, K, sums, x16, xinv, blockIdx.x - route_blocks);
    return;
  }
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  int id;
  float w;
  route_token<VPL, true>(logits, t, E, k, flags, sv[wave], si[wave], &id, &w);
  if (lane < k) {
    ids_out[(int64_t)t * k + lane] = id;
    w_out[(int64_t)t * k + lane] = w;
  }
}

hipError_t launch_route_prep_f16(const void* logits, int T, int E, int k, unsigned flags, int32_t* ids, float* w,
                                 const void* x, int rows, int K, float* sums, uint16_t* x16, float* xinv,
                                 hipStream_t stream) {
  if (T <= 0 || rows <= 0) return hipErrorInvalidValue;
  if (K % 128 != 0 || K > 4096 || E <= 0 || E > 256) return hipErrorInvalidValue;
  const int route_blocks = (T + 3) / 4;
  const dim3 grid(route_blocks + (rows + 3) / 4), block(256);
  const uint16_t* lg = (const uint16_t*)logits;
  const uint16_t* xb = (const uint16_t*)x;
#define NKT_RP_LAUNCH(V, C)                                                                                    \
  hipLaunchKernelGGL((route_prep_f16_kernel<V, C>), grid, block, 0, stream, lg, T, E, k, flags, ids, w,       \
                     route_blocks, xb, rows, K, sums, x16, xinv)
#define NKT_RP_CASE(V)                                          \
  case V:                                                       \
    switch ((K + 511) / 512) {                                  \
      case 1: NKT_RP_LAUNCH(V, 1); break;                       \
      case 2: NKT_RP_LAUNCH(V, 2); break;                       \
      case 3:                                                   \
      case 4: NKT_RP_LAUNCH(V, 4); break;                       \
      default: NKT_RP_LAUNCH(V, 8); break;                      \
    }                                                           \
    break;
  switch ((E + 63) / 64) {
    NKT_RP_CASE(1)
    NKT_RP_CASE(2)
    NKT_RP_CASE(3)
    NKT_RP_CASE(4)
    default:
      return hipErrorInvalidValue;
  }
#undef NKT_RP_CASE
#undef NKT_RP_LAUNCH
  return hipGetLastError();
}

hipError_t launch_prep_f16(const void* x, int rows, int K, float* sums, uint16_t* x16, float* xinv,
                           hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  if (K % 128 != 0 || K > 4096) return hipErrorInvalidValue;
  const dim3 grid((rows + 3) / 4), block(256);
  const uint16_t* xb = (const uint16_t*)x;
  switch ((K + 511) / 512) {
    case 1: hipLaunchKernelGGL(prep_f16_kernel<1>, grid, block, 0, stream, xb, rows, K, sums, x16, xinv); break;
    case 2: hipLaunchKernelGGL(prep_f16_kernel<2>, grid, block, 0, stream, xb, rows, K, sums, x16, xinv); break;
    case 3:
    case 4: hipLaunchKernelGGL(prep_f16_kernel<4>, grid, block, 0, stream, xb, rows, K, sums, x16, xinv); break;
    default: hipLaunchKernelGGL(prep_f16_kernel<8>, grid, block, 0, stream, xb, rows, K, sums, x16, xinv); break;
  }
  return hipGetLastError();
}

hipError_t launch_group_sums(const void* x, int rows, int K, float* out, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(group_sums_kernel, dim3((rows + 3) / 4), dim3(256), 0, stream, (const uint16_t*)x, rows, K,
                     out);
  return hipGetLastError();
}

// Waves per workgroup: int8 keeps 4 waves of 4 row tiles (its dequantised
// fragments feed 4 column tiles each and its loop fits two workgroups per CU
// without spills); bf16 and int4 take 8 waves of 2 row tiles, which halves
// the weight registers a wave double-buffers (bf16 blocks hold 32 columns,
// int4 adds per-group scale temporaries) and removes their spills.
constexpr int gemm2_waves(int wf) { return wf == WF_I8 ? 4 : 8; }

hipError_t launch_gemm2(const GemmArgs& a, int wf, int phase, int max_tiles, hipStream_t stream,
                        const KernelTimer* tm) {
  if (max_tiles <= 0) return hipSuccess;
  // K parts: the int8 pipeline's down only, fp32 rows, at most 16 K groups per part
  const int kp = a.k_parts > 1 ? a.k_parts : 1;
  if (kp > 1 && (phase != PHASE_DOWN || !gemm2_i8_pipeline(a, wf) || a.y16 || a.K % (128 * kp) != 0 ||
                 a.K / kp > 16 * 128))
    return hipErrorInvalidValue;
  const int n_slabs = phase == PHASE_GATE_UP ? a.I / 128 : a.N / 256 * kp;
  const int64_t items = (int64_t)n_slabs * max_tiles;
  const int sg = slab_group(n_slabs, a.w_expert_bytes);
  dim3 grid((unsigned)((items + kXcds - 1) / kXcds * kXcds)), block(64 * gemm2_waves(wf));
#define NKT_G2(W)                                                                                          \
  case W:                                                                                                  \
    if (phase == PHASE_GATE_UP)                                                                            \
      launch_timed(gemm2_kernel<W, PHASE_GATE_UP, gemm2_waves(W)>, grid, block, 0, stream, tm, a, n_slabs, sg); \
    else                                                                                                   \
      launch_timed(gemm2_kernel<W, PHASE_DOWN, gemm2_waves(W)>, grid, block, 0, stream, tm, a, n_slabs, sg);    \
    break;
  if (gemm2_i8_pipeline(a, wf)) {
    if (phase == PHASE_GATE_UP && a.xinv)
      launch_timed(gemm2_i8_kernel<PHASE_GATE_UP, true>, grid, block, 0, stream, tm, a, n_slabs, sg);
    else if (phase == PHASE_GATE_UP)
      launch_timed(gemm2_i8_kernel<PHASE_GATE_UP, false>, grid, block, 0, stream, tm, a, n_slabs, sg);
    else
      launch_timed(gemm2_i8_kernel<PHASE_DOWN, false>, grid, block, 0, stream, tm, a, n_slabs, sg);
    return hipGetLastError();
  }
  if (gemm2_i4_pipeline(a, wf)) {
    if (phase == PHASE_GATE_UP && a.narrow_tiles)
      launch_timed(gemm2_i4_kernel<PHASE_GATE_UP, true>, grid, block, 0, stream, tm, a, n_slabs, sg);
    else if (phase == PHASE_GATE_UP)
      launch_timed(gemm2_i4_kernel<PHASE_GATE_UP, false>, grid, block, 0, stream, tm, a, n_slabs, sg);
    else if (a.narrow_tiles)
      launch_timed(gemm2_i4_kernel<PHASE_DOWN, true>, grid, block, 0, stream, tm, a, n_slabs, sg);
    else
      launch_timed(gemm2_i4_kernel<PHASE_DOWN, false>, grid, block, 0, stream, tm, a, n_slabs, sg);
    return hipGetLastError();
  }
  switch (wf) {
    NKT_G2(WF_BF16)
    NKT_G2(WF_I4)
    default:
      return hipErrorInvalidValue;
  }
#undef NKT_G2
  return hipGetLastError();
}

}  // namespace nkt
