// K3: grouped SwiGLU expert GEMM over weight-only quantized experts.
//
// Replaces the per-routed-expert loop of nano_ktrans/layers/hybrid_moe.py:
// 3501-3533 (SparseExpertMLP / PackedSparseExpertMLP.forward,
// nano_ktrans/layers/expert_mlp.py:20-41) and the fp32 quantized loop of
// nano_ktrans/kernels/cpu_moe.py:419-450 (cpu_w4a32_matvec,
// nano_ktrans/kernels/quantized_ops.py:86-124).
//
// One workgroup computes a tile of (BM positions of one expert) x (a slab of
// weight rows).  The A operand of the matrix core is the weight tile, read
// straight from HBM in the 1 KiB block layout (one 16-byte load per lane per
// block, fully coalesced) and dequantised in registers; the B operand is the
// token tile, gathered once per K stage into LDS.  Quantised codes enter the
// matrix core as exact bf16 integers with an offset (int4: 128 + stored
// nibble = 136 + q, int8: stored byte = 128 + q); the offset times the column
// sum of the token tile is removed per 128-wide K group, and the bf16 scale is
// applied to the fp32 partial sum of each group (int4) or once per row (int8),
// so no weight is ever rounded to bf16 after scaling.
//   gate_up phase: the wave holds matching gate and up row tiles and writes
//                  h = silu(gate) * up  (act dtype) by position;
//   down phase:    writes y (fp32) by position.
#include "nkt_common.h"
#include "nkt_internal.h"

namespace nkt {

template <int WF>
struct Fmt {
  static constexpr int NBLK = 128 / block_k(WF);  // 1 KiB blocks per 128-wide K group
  static constexpr int ES = (WF == WF_F32) ? 4 : 2;  // activation element size
};

__device__ __forceinline__ u32x4 dequant_i4_step(uint32_t w) {
  u32x4 a;
  a[0] = (w & 0x000F000Fu) | 0x43004300u;
  a[1] = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
  a[2] = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
  a[3] = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
  return a;
}

__device__ __forceinline__ uint32_t bf16pair_from_bytes(uint32_t w, int lo_byte) {
  const float f0 = (float)((w >> (8 * lo_byte)) & 0xffu);
  const float f1 = (float)((w >> (8 * lo_byte + 8)) & 0xffu);
  return __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
}

__device__ __forceinline__ u32x4 dequant_i8_step(uint32_t w0, uint32_t w1) {
  u32x4 a;
  a[0] = bf16pair_from_bytes(w0, 0);
  a[1] = bf16pair_from_bytes(w0, 2);
  a[2] = bf16pair_from_bytes(w1, 0);
  a[3] = bf16pair_from_bytes(w1, 2);
  return a;
}

__device__ __forceinline__ float silu_f(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

template <int WF, int BM, int NW, int RT, int PHASE, int KC, int PF>
__global__ void __launch_bounds__(NW * 64) gemm_kernel(GemmArgs a) {
  constexpr int NBLK = Fmt<WF>::NBLK;
  constexpr int ES = Fmt<WF>::ES;
  constexpr int CT = BM / 16;
  constexpr int OUT_RT = (PHASE == PHASE_GATE_UP) ? RT / 2 : RT;
  constexpr int LDS_STRIDE = KC * ES + 16;
  constexpr int GPS = KC / 128;  // K groups per LDS stage
  constexpr bool IS_INT = (WF == WF_I4 || WF == WF_I8);

  __shared__ __attribute__((aligned(16))) uint8_t lds_b[BM * LDS_STRIDE];
  __shared__ float lds_xs[IS_INT ? BM * GPS : 1];
  __shared__ int lds_src[BM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  int expert, row0, rows;
  if (a.n_tiles != nullptr) {
    if ((int)blockIdx.x >= a.n_tiles[0]) return;
    expert = a.tiles[4 * blockIdx.x + 0];
    row0 = a.tiles[4 * blockIdx.x + 1];
    rows = a.tiles[4 * blockIdx.x + 2];
  } else {
    expert = 0;
    row0 = blockIdx.x * BM;
    if (row0 >= a.num_rows) return;
    rows = min(BM, a.num_rows - row0);
  }

  const int out_dim = (PHASE == PHASE_GATE_UP) ? a.I : a.N;
  const int orow0 = (blockIdx.y * NW + wave) * OUT_RT * 16;
  const bool wave_active = orow0 + OUT_RT * 16 <= out_dim;
  const int K = a.K;
  const int G = K / 128;
  const int NKB = K / block_k(WF);

  if (tid < BM) {
    int src = -1;
    if (tid < rows) src = a.perm ? a.perm[row0 + tid] / a.topk : row0 + tid;
    lds_src[tid] = src;
  }

  // weight / scale pointers of this wave's row tiles
  const uint8_t* wptr[RT];
  const uint16_t* sptr[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    int wrow;
    if (PHASE == PHASE_GATE_UP)
      wrow = (r < RT / 2) ? orow0 + 16 * r : a.I + orow0 + 16 * (r - RT / 2);
    else
      wrow = orow0 + 16 * r;
    if (!wave_active) wrow = 0;
    const int rb = wrow >> 4;
    wptr[r] = a.w + (int64_t)expert * a.w_expert_bytes + (int64_t)rb * NKB * 1024 + lane * 16;
    if (WF == WF_I4)
      sptr[r] = a.scales + (int64_t)expert * a.s_expert_elems + (int64_t)rb * G * 16 + 4 * (lane >> 4);
    else if (WF == WF_I8)
      sptr[r] = a.scales + (int64_t)expert * a.s_expert_elems + wrow + 4 * (lane >> 4);
    else
      sptr[r] = nullptr;
  }

  f32x4 acc[RT][CT];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int c = 0; c < CT; ++c) acc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 wring[PF][RT][NBLK];
  u32x2 sring[PF][RT];

#pragma unroll
  for (int p = 0; p < PF; ++p) {
    if (wave_active && p < G) {
#pragma unroll
      for (int r = 0; r < RT; ++r) {
#pragma unroll
        for (int i = 0; i < NBLK; ++i)
          wring[p][r][i] = *(const u32x4*)(wptr[r] + (int64_t)(p * NBLK + i) * 1024);
        if (WF == WF_I4) sring[p][r] = *(const u32x2*)(sptr[r] + p * 16);
      }
    }
  }

  for (int g0 = 0; g0 < G; g0 += PF) {
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      const int g = g0 + p;
      if (g < G) {
        const int gs = g % GPS;  // group inside the stage
        if (gs == 0) {
          // ---- stage the token tile for K range [g*128, g*128 + kc) ----
          const int kc0 = g * 128;
          const int kc = min(KC, K - kc0);
          const int n16 = kc * ES / 16;
          __syncthreads();
          for (int idx = tid; idx < BM * n16; idx += NW * 64) {
            const int c = idx / n16;
            const int q = idx - c * n16;
            const int src = lds_src[c];
            u32x4 v = u32x4{0u, 0u, 0u, 0u};
            if (src >= 0)
              v = *(const u32x4*)((const uint8_t*)a.in + ((int64_t)src * K + kc0) * ES + q * 16);
            *(u32x4*)(lds_b + c * LDS_STRIDE + q * 16) = v;
          }
          __syncthreads();
          if (IS_INT) {
            const int ng = kc / 128;
            for (int idx = tid; idx < BM * ng; idx += NW * 64) {
              const int c = idx % BM;
              const int gg = idx / BM;
              const uint8_t* rowp = lds_b + c * LDS_STRIDE + gg * 256;
              float s = 0.f;
#pragma unroll
              for (int q = 0; q < 16; ++q) {
                const u32x4 v = *(const u32x4*)(rowp + q * 16);
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                  s += __uint_as_float(v[h] << 16);
                  s += __uint_as_float(v[h] & 0xffff0000u);
                }
              }
              lds_xs[c * GPS + gg] = s;
            }
            __syncthreads();
          }
        }

        if (wave_active) {
          if (WF == WF_F32) {
#pragma unroll
            for (int i = 0; i < NBLK; ++i) {
#pragma unroll
              for (int s = 0; s < 4; ++s) {
                float bv[CT];
#pragma unroll
                for (int c = 0; c < CT; ++c)
                  bv[c] = *(const float*)(lds_b + (c * 16 + (lane & 15)) * LDS_STRIDE +
                                          (gs * 128 + i * 16 + 4 * s + (lane >> 4)) * 4);
#pragma unroll
                for (int r = 0; r < RT; ++r) {
                  const float av = __uint_as_float(wring[p][r][i][s]);
#pragma unroll
                  for (int c = 0; c < CT; ++c) acc[r][c] = mfma_f32(av, bv[c], acc[r][c]);
                }
              }
            }
          } else {
            float xsv[CT];
            if (IS_INT) {
#pragma unroll
              for (int c = 0; c < CT; ++c) xsv[c] = lds_xs[(c * 16 + (lane & 15)) * GPS + gs];
            }
            f32x4 tmp[WF == WF_I4 ? RT : 1][WF == WF_I4 ? CT : 1];
            if (WF == WF_I4) {
#pragma unroll
              for (int r = 0; r < RT; ++r)
#pragma unroll
                for (int c = 0; c < CT; ++c) {
                  const float cv = -136.0f * xsv[c];
                  tmp[r][c] = f32x4{cv, cv, cv, cv};
                }
            } else if (WF == WF_I8) {
#pragma unroll
              for (int r = 0; r < RT; ++r)
#pragma unroll
                for (int c = 0; c < CT; ++c) {
                  const float cv = -128.0f * xsv[c];
                  acc[r][c] += f32x4{cv, cv, cv, cv};
                }
            }
#pragma unroll
            for (int s = 0; s < 4; ++s) {
              u32x4 bf[CT];
#pragma unroll
              for (int c = 0; c < CT; ++c)
                bf[c] = *(const u32x4*)(lds_b + (c * 16 + (lane & 15)) * LDS_STRIDE +
                                        (gs * 128 + 32 * s + 8 * (lane >> 4)) * 2);
#pragma unroll
              for (int r = 0; r < RT; ++r) {
                u32x4 av;
                if (WF == WF_I4)
                  av = dequant_i4_step(wring[p][r][0][s]);
                else if (WF == WF_I8)
                  av = dequant_i8_step(wring[p][r][s >> 1][2 * (s & 1)],
                                       wring[p][r][s >> 1][2 * (s & 1) + 1]);
                else
                  av = wring[p][r][s];
#pragma unroll
                for (int c = 0; c < CT; ++c) {
                  if (WF == WF_I4)
                    tmp[r][c] = mfma_bf16(av, bf[c], tmp[r][c]);
                  else
                    acc[r][c] = mfma_bf16(av, bf[c], acc[r][c]);
                }
              }
            }
            if (WF == WF_I4) {
#pragma unroll
              for (int r = 0; r < RT; ++r) {
                const u32x2 sv = sring[p][r];
                const f32x4 s4 = f32x4{__uint_as_float(sv[0] << 16), __uint_as_float(sv[0] & 0xffff0000u),
                                       __uint_as_float(sv[1] << 16), __uint_as_float(sv[1] & 0xffff0000u)};
#pragma unroll
                for (int c = 0; c < CT; ++c) acc[r][c] += s4 * tmp[r][c];
              }
            }
          }
          // refill this ring slot with group g + PF
          if (g + PF < G) {
#pragma unroll
            for (int r = 0; r < RT; ++r) {
#pragma unroll
              for (int i = 0; i < NBLK; ++i)
                wring[p][r][i] = *(const u32x4*)(wptr[r] + (int64_t)((g + PF) * NBLK + i) * 1024);
              if (WF == WF_I4) sring[p][r] = *(const u32x2*)(sptr[r] + (g + PF) * 16);
            }
          }
        }
      }
    }
  }

  if (!wave_active) return;

  // ---- epilogue ----
  const int col = lane & 15;
  const int rq = 4 * (lane >> 4);
  if (WF == WF_I8) {
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      const u32x2 sv = *(const u32x2*)(sptr[r]);
      const f32x4 s4 = f32x4{__uint_as_float(sv[0] << 16), __uint_as_float(sv[0] & 0xffff0000u),
                             __uint_as_float(sv[1] << 16), __uint_as_float(sv[1] & 0xffff0000u)};
#pragma unroll
      for (int c = 0; c < CT; ++c) acc[r][c] *= s4;
    }
  }

  if (PHASE == PHASE_GATE_UP) {
#pragma unroll
    for (int r = 0; r < RT / 2; ++r) {
#pragma unroll
      for (int c = 0; c < CT; ++c) {
        const int t = c * 16 + col;
        if (t < rows) {
          const f32x4 gt = acc[r][c];
          const f32x4 up = acc[r + RT / 2][c];
          float h[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) h[v] = silu_f(gt[v]) * up[v];
          const int64_t o = (int64_t)(row0 + t) * a.I + orow0 + 16 * r + rq;
          if (a.act_bf16) {
            u32x2 pk;
            pk[0] = pack_bf16x2(h[0], h[1]);
            pk[1] = pack_bf16x2(h[2], h[3]);
            *(u32x2*)((uint16_t*)a.out + o) = pk;
          } else {
            *(f32x4*)((float*)a.out + o) = f32x4{h[0], h[1], h[2], h[3]};
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < RT; ++r) {
#pragma unroll
      for (int c = 0; c < CT; ++c) {
        const int t = c * 16 + col;
        if (t < rows) {
          const int64_t yrow = a.out_rows ? a.out_rows[row0 + t] : row0 + t;
          const int64_t o = yrow * a.N + orow0 + 16 * r + rq;
          *(f32x4*)((float*)a.out + o) = acc[r][c];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// configuration table
// ---------------------------------------------------------------------------
// Tokens per expert (T k / E) up to which the decode form runs, from the
// measured crossover of the two forms' layer times, with the prefill form's
// short tiles on copies that skip empty column tiles: int8 weights 4.5 (the
// decode form wins at 4.3 tokens per expert, the prefill form at 5 under
// even and skewed routing alike), 3.5 in a layer with a shared expert, which
// the prefill form runs beside the routed experts on the side stream
// (Qwen1.5-MoE T = 64 / 67: 131 / 134.2 -> 126.7 / 128.8 us), int4 8 (at 8 the forms are level under
// even routing and the decode form wins under Zipf routing; at 10 - 16 the
// prefill form wins: Qwen3 T = 192 107.8 -> 99.1 us, Mixtral T = 48 222 ->
// 197, T = 64 285 -> 225) -- 6 for experts of I >= 8192, whose decode down
// takes the long-K ring (Mixtral, T = 28 / 32: 189.6 / 194.8 -> 183.9 /
// 180.5 us; level at 6, decode ahead at 5), others 12.
double decode_form_max_avg(int wf, int I, bool shared) {
  return wf == WF_I8 ? (shared ? 3.5 : 4.5) : wf == WF_I4 ? (I >= 8192 ? 6.0 : 8.0) : 12.0;
}

int gemm_tile_m(int num_tokens, int topk, int num_experts, int wf, bool prefill_form, int I, bool shared) {
  const double avg = (double)num_tokens * topk / (double)num_experts;
  if (avg <= decode_form_max_avg(wf, I, shared)) return 16;
  if (wf != WF_F32 && prefill_form) return kPrefillTileM;
  if (avg <= 40.0) return 32;
  return 64;
}

// Waves per block and row tiles per wave for each token-tile height: 16
// positions take 8 waves of 2 row tiles, except fp32 weights (the tiny
// layers: few tiles, long fp32 MFMA chains), which take 4 waves of one
// output row tile so the grid has four times the workgroups (Mixtral-style
// H = 256, I = 512, T = 16: 10 down workgroups instead of 40); larger tiles 4
// waves of 4.
constexpr int gemm_waves(int wf, int bm) { return bm == 16 && wf != WF_F32 ? 8 : 4; }
constexpr int gemm_row_tiles(int wf, int bm, int phase) {
  return bm != 16 ? 4 : (wf == WF_F32 && phase == PHASE_DOWN) ? 1 : 2;
}

int gemm_rows_per_block(int wf, int phase, int bm) {
  const int rt = gemm_row_tiles(wf, bm, phase);
  return gemm_waves(wf, bm) * (phase == PHASE_GATE_UP ? rt / 2 : rt) * 16;
}

template <int WF, int BM, int PHASE>
static hipError_t launch_gemm_t(const GemmArgs& a, int grid_tiles, hipStream_t stream,
                                const KernelTimer* tm) {
  constexpr int NW = gemm_waves(WF, BM);
  constexpr int RT = gemm_row_tiles(WF, BM, PHASE);
  // LDS stage: BM x KC activations (~33 KiB); fp32 activations take half the K
  constexpr int KC0 = (BM == 16) ? 1024 : (BM == 32 ? 512 : 256);
  constexpr int KC = (WF == WF_F32) ? KC0 / 2 : KC0;
  // groups of weight loads kept in flight per wave
  constexpr int PF = (WF == WF_I4) ? (BM == 16 ? 4 : 2) : (WF == WF_I8 ? 2 : 1);
  const int out_dim = (PHASE == PHASE_GATE_UP) ? a.I : a.N;
  const int rows_per_block = NW * ((PHASE == PHASE_GATE_UP) ? RT / 2 : RT) * 16;
  dim3 grid(grid_tiles, (out_dim + rows_per_block - 1) / rows_per_block);
  launch_timed(gemm_kernel<WF, BM, NW, RT, PHASE, KC, PF>, grid, dim3(NW * 64), 0, stream, tm, a);
  return hipGetLastError();
}

template <int WF>
static hipError_t launch_gemm_wf(const GemmArgs& a, int phase, int bm, int grid_tiles,
                                 hipStream_t stream, const KernelTimer* tm) {
  if (phase == PHASE_GATE_UP) {
    if (bm == 16) return launch_gemm_t<WF, 16, PHASE_GATE_UP>(a, grid_tiles, stream, tm);
    if (bm == 32) return launch_gemm_t<WF, 32, PHASE_GATE_UP>(a, grid_tiles, stream, tm);
    if (bm == 64) return launch_gemm_t<WF, 64, PHASE_GATE_UP>(a, grid_tiles, stream, tm);
  } else {
    if (bm == 16) return launch_gemm_t<WF, 16, PHASE_DOWN>(a, grid_tiles, stream, tm);
    if (bm == 32) return launch_gemm_t<WF, 32, PHASE_DOWN>(a, grid_tiles, stream, tm);
    if (bm == 64) return launch_gemm_t<WF, 64, PHASE_DOWN>(a, grid_tiles, stream, tm);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gemm(const GemmArgs& a, int wf, int phase, int bm, int grid_tiles,
                       hipStream_t stream, const KernelTimer* tm) {
  if (grid_tiles <= 0) return hipSuccess;
  switch (wf) {
    case WF_F32:
      return launch_gemm_wf<WF_F32>(a, phase, bm, grid_tiles, stream, tm);
    case WF_BF16:
      return launch_gemm_wf<WF_BF16>(a, phase, bm, grid_tiles, stream, tm);
    case WF_I8:
      return launch_gemm_wf<WF_I8>(a, phase, bm, grid_tiles, stream, tm);
    case WF_I4:
      return launch_gemm_wf<WF_I4>(a, phase, bm, grid_tiles, stream, tm);
    default:
      return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------------
// Repack one projection [N, K] from the source layout into 1 KiB blocks.
// One thread writes one lane's 16 bytes of one block.
// ---------------------------------------------------------------------------
template <int WF>
__global__ void __launch_bounds__(256) pack_kernel(const void* __restrict__ src,
                                                   const uint16_t* __restrict__ src_scales, int N,
                                                   int K, int n_valid, uint8_t* __restrict__ dst,
                                                   uint16_t* __restrict__ dst_scales) {
  const int KB = block_k(WF);
  const int NKB = K / KB;
  const int64_t nthreads = (int64_t)(N / 16) * NKB * 64;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid < nthreads) {
    const int lane = (int)(gid & 63);
    const int64_t blk = gid >> 6;
    const int kb = (int)(blk % NKB);
    const int rb = (int)(blk / NKB);
    const int row = rb * 16 + (lane & 15);
    const int kq = lane >> 4;
    u32x4 out;
    if (WF == WF_I4) {
      const uint32_t* s = (const uint32_t*)src + (int64_t)row * (K / 8);
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const uint32_t w = s[kb * 16 + 4 * st + kq];  // columns kb*128 + 32st + 8kq + 0..7
        uint32_t o = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int colofs = (j < 4) ? 2 * j : 2 * (j - 4) + 1;
          o |= ((w >> (4 * colofs)) & 0xfu) << (4 * j);
        }
        out[st] = o;
      }
    } else if (WF == WF_I8) {
      const uint8_t* s = (const uint8_t*)src + (int64_t)row * K;
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const uint8_t* p = s + kb * 64 + 32 * st + 8 * kq;
        out[2 * st] = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
        out[2 * st + 1] = (uint32_t)p[4] | ((uint32_t)p[5] << 8) | ((uint32_t)p[6] << 16) | ((uint32_t)p[7] << 24);
      }
    } else if (WF == WF_BF16) {
      const uint16_t* s = (const uint16_t*)src + (int64_t)(row < n_valid ? row : 0) * K + kb * 32 + 8 * kq;
#pragma unroll
      for (int h = 0; h < 4; ++h)
        out[h] = row < n_valid ? (uint32_t)s[2 * h] | ((uint32_t)s[2 * h + 1] << 16) : 0u;
    } else {
      const float* s = (const float*)src + (int64_t)row * K + kb * 16 + kq;
#pragma unroll
      for (int st = 0; st < 4; ++st) out[st] = __float_as_uint(s[4 * st]);
    }
    *(u32x4*)(dst + blk * 1024 + lane * 16) = out;
  }
  // scales
  if (WF == WF_I4) {
    const int G = K / 128;
    const int64_t ns = (int64_t)N * G;
    if (gid < ns) {
      const int n = (int)(gid / G);
      const int g = (int)(gid % G);
      dst_scales[((int64_t)(n >> 4) * G + g) * 16 + (n & 15)] = src_scales[(int64_t)n * G + g];
    }
  } else if (WF == WF_I8) {
    if (gid < N) dst_scales[gid] = src_scales[gid];
  }
}

hipError_t launch_pack(int wf, const void* src, const void* src_scales, int N, int K, uint8_t* dst,
                       uint16_t* dst_scales, hipStream_t stream, int n_valid) {
  if (n_valid < 0) n_valid = N;
  if (n_valid != N && wf != WF_BF16) return hipErrorInvalidValue;  // row padding: bf16 only
  const int64_t nthreads = (int64_t)(N / 16) * (K / block_k(wf)) * 64;
  const int64_t nscale = (wf == WF_I4) ? (int64_t)N * (K / 128) : N;
  const int64_t total = nthreads > nscale ? nthreads : nscale;
  dim3 grid((unsigned)((total + 255) / 256)), block(256);
  switch (wf) {
    case WF_F32:
      hipLaunchKernelGGL(pack_kernel<WF_F32>, grid, block, 0, stream, src,
                         (const uint16_t*)src_scales, N, K, n_valid, dst, dst_scales);
      break;
    case WF_BF16:
      hipLaunchKernelGGL(pack_kernel<WF_BF16>, grid, block, 0, stream, src,
                         (const uint16_t*)src_scales, N, K, n_valid, dst, dst_scales);
      break;
    case WF_I8:
      hipLaunchKernelGGL(pack_kernel<WF_I8>, grid, block, 0, stream, src,
                         (const uint16_t*)src_scales, N, K, n_valid, dst, dst_scales);
      break;
    case WF_I4:
      hipLaunchKernelGGL(pack_kernel<WF_I4>, grid, block, 0, stream, src,
                         (const uint16_t*)src_scales, N, K, n_valid, dst, dst_scales);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace nkt
