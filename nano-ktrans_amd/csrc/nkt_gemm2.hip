// K3, prefill form: grouped SwiGLU expert GEMM for tiles of up to 128
// positions of one expert (prefill-sized groups), on the bf16 matrix cores.
//
// Replaces, for large batches, the per-routed-expert loop of
// nano_ktrans/layers/hybrid_moe.py:3501-3533 (SparseExpertMLP /
// PackedSparseExpertMLP.forward, nano_ktrans/layers/expert_mlp.py:20-41) and
// the quantized loop of nano_ktrans/kernels/cpu_moe.py:419-450.
//
// Workgroup = 4 or 8 waves, tile = 64 positions x 256 weight rows, two
// workgroups per CU.  gate_up: the 256 rows are 128 gate rows and the 128
// matching up rows (a wave holds gate and up rows for the same h columns, so
// SwiGLU is wave-local); down: 256 output rows split over the waves.  K
// advances one 128-wide group per step:
//   * the token tile (64 positions x 128 K, bf16, gathered through the
//     permutation for gate_up) is staged in LDS, double-buffered: the next
//     group's rows load into registers while this group computes;
//   * each wave streams its own weight blocks from HBM into registers (one
//     16-byte load per lane per 1 KiB block), one group ahead;
//   * per group a wave runs 4 (or 2) row tiles x 4 column tiles x 4 K steps of
//     v_mfma_f32_16x16x32_bf16, dequantising each weight fragment once.
// Codes enter the matrix core as exact bf16 integers with an offset (int4:
// 136 + q, int8: 128 + q); the offset times the group's activation sum
// (precomputed per source row and group, fp32) is removed per group for
// int4, whose group scale then multiplies the group's fp32 partial; for int8
// the offset times the row's total sum is removed once and the per-row scale
// multiplies the total.  gate_up also writes the per-position group
// sums of the bf16 h it stores, which the down projection consumes.
#include "nkt_common.h"
#include "nkt_internal.h"

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

template <int WF, int PHASE, int kWaves>
__global__ void __launch_bounds__(64 * kWaves, 2) gemm2_kernel(GemmArgs a, int n_slabs) {
  constexpr int kRT = 16 / kWaves;  // 16-row weight tiles per wave
  constexpr int NBLK = 128 / block_k(WF);
  // two separate LDS objects (not one array) so the compiler can tell a
  // direct-to-LDS load into one buffer from reads of the other
  __shared__ __attribute__((aligned(1024))) uint8_t bt0[kBM * 256];
  __shared__ __attribute__((aligned(1024))) uint8_t bt1[kBM * 256];
  __shared__ float xsl0[256];  // int4: group sums of the tile rows (each wave loads all; [0, kBM) used)
  __shared__ float xsl1[256];
  __shared__ int srcl[kBM];
  __shared__ float hpart[kWaves][kBM];
  __shared__ float xtot_l[kBM];

  // XCD-aware work order: workgroup b runs on XCD b % 8, so XCD x takes the
  // x-th contiguous eighth of the (tile-major, slab-minor) item list.  The
  // slabs of one token tile and the tiles of one expert then run side by
  // side on one XCD and share its L2 (token rows and weight slabs are read
  // from HBM about once instead of once per XCD).
  // (the 1-D grid is a multiple of 8 and at least 8 * per_xcd, so every
  // item below n_items has exactly one workgroup)
  const int n_tiles = a.n_tiles ? a.n_tiles[0] : (a.num_rows + kBM - 1) / kBM;
  const int n_items = n_tiles * n_slabs;
  const int b = blockIdx.x;
  const int per_xcd = (n_items + kXcds - 1) / kXcds;
  const int j = b / kXcds;
  if (j >= per_xcd) return;
  const int item = (b % kXcds) * per_xcd + j;
  if (item >= n_items) return;
  const int tile = item / n_slabs;
  const int slab = item - tile * n_slabs;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int G = a.K / 128;
  const int NKB = a.K / block_k(WF);

  int expert, row0, rows;
  if (a.n_tiles) {
    const int4 rec = *(const int4*)(a.tiles + 4 * tile);
    expert = rec.x;
    row0 = rec.y;
    rows = rec.z;
  } else {
    expert = 0;
    row0 = tile * kBM;
    rows = min(kBM, a.num_rows - row0);
  }
  if (tid < kBM) {
    const int p = row0 + (tid < rows ? tid : 0);
    srcl[tid] = a.perm ? a.perm[p] / a.topk : p;
  }
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

  // ---- epilogue ----------------------------------------------------------
  const int rq = 4 * (lane >> 4);
  if (WF == WF_I8) {
    // the code offset: -128 x the row's K sum (group sums added in order)
    if (tid < kBM) {
      const float* xr = a.xsum + (int64_t)srcl[tid] * G;
      float t = 0.f;
      for (int g = 0; g < G; ++g) t += xr[g];
      xtot_l[tid] = t;
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < kCT; ++c) {
      const float cv = -128.0f * xtot_l[c * 16 + (lane & 15)];
#pragma unroll
      for (int r = 0; r < kRT; ++r) acc[r][c] += f32x4{cv, cv, cv, cv};
    }
  }
  if (PHASE == PHASE_GATE_UP) {
    const int hcol0 = slab * 128 + wave * (128 / kWaves);
    constexpr int HR = kRT / 2;
    f32x4 sg[HR], su[HR];
    if (WF == WF_I8) {
#pragma unroll
      for (int r = 0; r < HR; ++r) {
        sg[r] = bf16x4_to_f32(*(const u32x2*)(sexp + wrow[r] + rq));
        su[r] = bf16x4_to_f32(*(const u32x2*)(sexp + wrow[r + HR] + rq));
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
        if (pl < rows) *(u32x2*)((uint16_t*)a.out + (int64_t)(row0 + pl) * a.I + hcol0 + r * 16 + rq) = pk;
      }
      // the 4 lanes holding one position's columns: fixed-order butterfly
      part += __shfl_xor(part, 16);
      part += __shfl_xor(part, 32);
      if (lane < 16) hpart[wave][pl] = part;
    }
    if (a.hsum) {
      __syncthreads();
      if (tid < kBM && tid < rows) {
        float s = hpart[0][tid];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) s += hpart[w][tid];
        a.hsum[(int64_t)(row0 + tid) * (a.I / 128) + slab] = s;
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < kRT; ++r) {
      f32x4 sr = f32x4{1.f, 1.f, 1.f, 1.f};
      if (WF == WF_I8) sr = bf16x4_to_f32(*(const u32x2*)(sexp + wrow[r] + rq));
#pragma unroll
      for (int c = 0; c < kCT; ++c) {
        const int pl = c * 16 + (lane & 15);
        f32x4 v = acc[r][c];
        if (WF == WF_I8) v *= sr;
        if (pl < rows) *(f32x4*)((float*)a.out + (int64_t)(row0 + pl) * a.N + wrow[r] + rq) = v;
      }
    }
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

bool gemm2_supported(int wf, int phase, int N, int K, int I) {
  if (wf != WF_BF16 && wf != WF_I8 && wf != WF_I4) return false;
  if (K % 128 != 0) return false;
  return phase == PHASE_GATE_UP ? (I % 128 == 0) : (N % 256 == 0);
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
  const int n_slabs = phase == PHASE_GATE_UP ? a.I / 128 : a.N / 256;
  const int64_t items = (int64_t)n_slabs * max_tiles;
  dim3 grid((unsigned)((items + kXcds - 1) / kXcds * kXcds)), block(64 * gemm2_waves(wf));
#define NKT_G2(W)                                                                                          \
  case W:                                                                                                  \
    if (phase == PHASE_GATE_UP)                                                                            \
      launch_timed(gemm2_kernel<W, PHASE_GATE_UP, gemm2_waves(W)>, grid, block, 0, stream, tm, a, n_slabs); \
    else                                                                                                   \
      launch_timed(gemm2_kernel<W, PHASE_DOWN, gemm2_waves(W)>, grid, block, 0, stream, tm, a, n_slabs);    \
    break;
  switch (wf) {
    NKT_G2(WF_BF16)
    NKT_G2(WF_I8)
    NKT_G2(WF_I4)
    default:
      return hipErrorInvalidValue;
  }
#undef NKT_G2
  return hipGetLastError();
}

}  // namespace nkt
