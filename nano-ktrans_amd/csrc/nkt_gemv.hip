// K3, decode form: grouped SwiGLU expert GEMM for tiles of at most 16
// positions (decode-sized groups).
//
// Replaces, for small batches, the per-routed-expert loop of
// nano_ktrans/layers/hybrid_moe.py:3501-3533 (SparseExpertMLP /
// PackedSparseExpertMLP.forward, nano_ktrans/layers/expert_mlp.py:20-41) and
// the quantized loop of nano_ktrans/kernels/cpu_moe.py:419-450.
//
// One wave owns one (tile, row set, K part): a tile is up to 16 positions of
// one expert, a row set is RT 16-row output tiles (gate_up: RT gate tiles and
// the RT matching up tiles, so SwiGLU is local), the K part is every S-th
// 128-wide K group.  The wave reads its weight blocks straight from HBM into
// registers, one 16-byte load per lane per 1 KiB block.  Normally K is split
// over S waves of one workgroup so that each wave owns NG groups (about 8 KiB
// of weights) and issues all of their loads at once (many short waves stream
// HBM better than few long ones); for long K the wave streams its groups
// through a D-deep register ring whose refills are issued right after the
// slot is consumed, always (past the last group they re-read it, an L2 hit),
// so the loop has no branch, store or barrier.  The matrix core takes the
// weights as the A operand and the tile's activations as B.  Tiles of at most
// four positions use the quad form: one 16-byte load per lane per group,
// landing in LDS through a direct-to-LDS load (no registers held while in
// flight), each step's B operand built by a DPP row shift; larger tiles load
// the B-operand layout (four loads per group) into registers one group at a
// time.  int4 scales also arrive through a direct-to-LDS load.  Gathered rows
// come from the per-tile source rows K2 writes (indexed by tile, so their
// load overlaps the tile record's).  The S partial sums meet in LDS and are
// added in K-part order.
//
// Dequantisation is the same as the prefill kernel's: codes enter the matrix
// core as exact bf16 integers with an offset (int4: 136 + q, int8: 128 + q),
// the offset times the group's activation sum is removed per group, the bf16
// scale multiplies each group's fp32 partial (int4: one explicit fused
// multiply-add into the running sum, so every kernel that shares this
// accumulation rounds alike) or the row total (int8).
#include "nkt_common.h"
#include "nkt_group.h"
#include "nkt_internal.h"
#include "nkt_route_token.h"

namespace nkt {

// 16-row output tiles per wave
constexpr int kGemvRtGateUp = 1;
constexpr int kGemvRtDown = 2;
constexpr int kGemvFewWaves = 256;  // down launches with fewer (row set, tile) items take one row tile per wave

namespace {

// One K group of NT weight tiles (+ int4 scales).
template <int WF, int NT>
struct WSlot {
  static constexpr int NBLK = 128 / block_k(WF);
  u32x4 w[NT][NBLK];
  u32x2 s[NT];
};

// A ring slot: weights plus the group's activations in the B-operand layout.
template <int WF, int NT>
struct RSlot {
  WSlot<WF, NT> w;
  u32x4 x[4];
};

// Weight loads address a uniform per-expert base plus a 32-bit offset
// (global_load ... saddr form, or a raw buffer load: one offset register per
// load).
// STREAM: non-temporal weight loads (nt policy), for tiles of fewer than 16
// positions -- an expert's only tile unless it has more than 16 -- whose
// weights no other tile of the launch reads: they then displace less of what
// the caches hold for the launch's other workgroups (activations, scales).
// Full 16-position tiles (an expert with 16 or more positions, the shared
// expert's chunks at 16 or more tokens) load with the default policy, so the
// expert's other tiles find the weights in the caches.  Measured on the
// decode layers: 4 - 7 % faster from 4 to 128 tokens with this split, while
// streaming every tile is up to 17 % slower where the shared expert's chunks
// span several tiles; the one-token int8 kernels keep the default policy
// (1 % faster).  The streaming form is a raw buffer load whose policy operand
// (an immediate) sets nt: the compiler never merges it with the default-policy
// load when both forms sit in one kernel, as it may merge loads that differ
// only in a non-temporal hint.
constexpr int kBufPolicyNT = 2;             // buffer load policy bits: nt
constexpr int kBufResourceWord3 = 0x20000;  // raw buffer resource, CDNA (gfx9) data format
template <int WF, int NT, bool STREAM, bool SCALES = true>
__device__ __forceinline__ void load_w(WSlot<WF, NT>& r, const uint8_t* wexp, const uint16_t* sexp,
                                       const uint32_t (&rbo)[NT], const uint32_t (&sbo)[NT], int g,
                                       uint32_t lane) {
  constexpr int NBLK = WSlot<WF, NT>::NBLK;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int i = 0; i < NBLK; ++i) {
      const uint32_t off = rbo[t] + (uint32_t)(g * NBLK + i) * 1024u + lane * 16u;
      if constexpr (STREAM) {
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc((void*)wexp, (short)0, -1, kBufResourceWord3);
        r.w[t][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, kBufPolicyNT));
      } else {
        r.w[t][i] = *(const u32x4*)(wexp + off);
      }
    }
    if (WF == WF_I4 && SCALES) r.s[t] = *(const u32x2*)(sexp + (sbo[t] + (uint32_t)g * 16u + 4u * (lane >> 4)));
  }
}

// B operand of group g, one load per MFMA step: lane l holds
// x[row of column l%16][128g + 32s + 8(l/16) .. +7] in x[s].
__device__ __forceinline__ void load_x_full(u32x4 (&x)[4], const uint8_t* xrow, int g) {
#pragma unroll
  for (int s = 0; s < 4; ++s) x[s] = *(const u32x4*)(xrow + (g * 128 + 32 * s) * 2);
}

// Sum of the two bf16 values of w added to acc (v_dot2 with (1, 1)).
__device__ __forceinline__ float add_bf16_pair(uint32_t w, float acc) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), __builtin_bit_cast(bf16x2, 0x3f803f80u), acc,
                                         false);
}

// Sum of the group's 128 activations of the lane's column (lanes l, l^16,
// l^32, l^48 hold its four 32-wide quarters).
__device__ __forceinline__ float group_sum_full(const u32x4 (&x)[4]) {
  float a = 0.f, b = 0.f;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    a = add_bf16_pair(x[s][0], a);
    b = add_bf16_pair(x[s][1], b);
    a = add_bf16_pair(x[s][2], a);
    b = add_bf16_pair(x[s][3], b);
  }
  float xs = add_xor16(a + b);
  return add_xor32(xs);
}

// Tiles of at most four positions (almost every decode tile) load their
// activations compactly, one 16-byte load per lane per group: lane (q, j) =
// (l / 16, l % 16) holds x[row j % 4][128g + 32 (j / 4) + 8q .. +7].  The B
// operand of step s needs, in lane (q, c), x[row c][128g + 32s + 8q ..], held
// by lane (q, 4s + c) of the same row: a DPP row_shl by 4s.  Only columns
// c < 4 carry data; the others hold copies of other rows and their outputs are
// never stored (rows past the tile's count are padding).
template <int CTRL>
__device__ __forceinline__ u32x4 row_shl4(u32x4 v) {
  return u32x4{(uint32_t)__builtin_amdgcn_mov_dpp((int)v[0], CTRL, 0xf, 0xf, true),
               (uint32_t)__builtin_amdgcn_mov_dpp((int)v[1], CTRL, 0xf, 0xf, true),
               (uint32_t)__builtin_amdgcn_mov_dpp((int)v[2], CTRL, 0xf, 0xf, true),
               (uint32_t)__builtin_amdgcn_mov_dpp((int)v[3], CTRL, 0xf, 0xf, true)};
}

__device__ __forceinline__ u32x4 quad_operand(u32x4 xq, int s) {
  switch (s) {
    case 1:
      return row_shl4<0x104>(xq);
    case 2:
      return row_shl4<0x108>(xq);
    case 3:
      return row_shl4<0x10C>(xq);
    default:
      return xq;
  }
}

// Group sum of a quad-form load: lanes c < 4 of every row end with the sum of
// the group's 128 activations of column c.
__device__ __forceinline__ float quad_group_sum(u32x4 xq) {
  float v = add_bf16_pair(xq[0], 0.f);
  v = add_bf16_pair(xq[1], v);
  v = add_bf16_pair(xq[2], v);
  v = add_bf16_pair(xq[3], v);
  v = v + __uint_as_float(dpp_u32<0x108>(__float_as_uint(v)));  // + lane c + 8
  v = v + __uint_as_float(dpp_u32<0x104>(__float_as_uint(v)));  // + lanes c + 4, c + 12
  v = add_xor16(v);
  return add_xor32(v);
}

// A operand of tile t, step s.
template <int WF, int NT>
__device__ __forceinline__ u32x4 a_operand(const WSlot<WF, NT>& r, int t, int s, const DqConst& k) {
  if (WF == WF_I4) return dq_i4_k(r.w[t][0][s], k);
  if (WF == WF_I8) return dq_i8(r.w[t][s >> 1][2 * (s & 1)], r.w[t][s >> 1][2 * (s & 1) + 1]);
  return r.w[t][s];
}

// Marks the slot's registers as redefined here: dequantisation that both
// activation forms share stays inside each form's branch instead of being
// hoisted above it with every group's operands live at once (int8 and bf16;
// the int4 path gets the same from its branch-local constants).
template <int WF, int NT>
__device__ __forceinline__ void pin_slot(WSlot<WF, NT>& r) {
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int i = 0; i < WSlot<WF, NT>::NBLK; ++i) __asm__ volatile("" : "+v"(r.w[t][i]));
  if (WF == WF_I4)
#pragma unroll
    for (int t = 0; t < NT; ++t) __asm__ volatile("" : "+v"(r.s[t]));
}

// One group: BOP(s) gives the B operand of step s (built once, it feeds the
// NT tiles); xs: the group sum of the lane's column (int formats).  use ==
// false computes and adds nothing (a select, so no load is ever
// control-dependent).
template <int WF, int NT, class BOp>
__device__ __forceinline__ void mma_group_b(const WSlot<WF, NT>& r, BOp bop, float xs, f32x4 (&acc)[NT], bool use,
                                            const DqConst& k) {
  // int4: acc + scale x partial as one explicit fused multiply-add (the same
  // instruction in every kernel that accumulates a tile here, so the same
  // bits); otherwise acc + partial
#pragma clang fp contract(off)
  const float c = WF == WF_I4 ? -136.0f * xs : WF == WF_I8 ? -128.0f * xs : 0.0f;
  f32x4 tmp[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) tmp[t] = f32x4{c, c, c, c};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const u32x4 b = bop(s);
#pragma unroll
    for (int t = 0; t < NT; ++t) tmp[t] = mfma_bf16(a_operand<WF, NT>(r, t, s, k), b, tmp[t]);
    // one step's operands at a time (the scheduler would dequantise every
    // step ahead, a register per value)
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (WF == WF_I4) {
      const f32x4 sc = bf16x4_to_f32(r.s[t]);
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[t][v] = use ? __builtin_fmaf(sc[v], tmp[t][v], acc[t][v]) : acc[t][v];
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[t][v] = use ? acc[t][v] + tmp[t][v] : acc[t][v];
    }
  }
}

// Adds one group's contribution to acc; use == false computes it and adds
// nothing (a select, so no load is ever control-dependent).  xs: the group
// sum of the lane's column (int formats).
template <int WF, int NT>
__device__ __forceinline__ void mma_group(const WSlot<WF, NT>& r, const u32x4 (&xb)[4], float xs,
                                          f32x4 (&acc)[NT], bool use) {
#pragma clang fp contract(off)
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    f32x4 tmp;
    if (WF == WF_I4) {
      const float c = -136.0f * xs;
      tmp = f32x4{c, c, c, c};
#pragma unroll
      for (int s = 0; s < 4; ++s) tmp = mfma_bf16(dq_i4(r.w[t][0][s]), xb[s], tmp);
      const f32x4 sc = bf16x4_to_f32(r.s[t]);
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[t][v] = use ? __builtin_fmaf(sc[v], tmp[v], acc[t][v]) : acc[t][v];
      continue;
    } else if (WF == WF_I8) {
      const float c = -128.0f * xs;
      tmp = f32x4{c, c, c, c};
#pragma unroll
      for (int s = 0; s < 4; ++s)
        tmp = mfma_bf16(dq_i8(r.w[t][s >> 1][2 * (s & 1)], r.w[t][s >> 1][2 * (s & 1) + 1]), xb[s], tmp);
    } else {
      tmp = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) tmp = mfma_bf16(r.w[t][s], xb[s], tmp);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[t][v] = use ? acc[t][v] + tmp[v] : acc[t][v];
  }
}

// Output rows orow0 .. orow0 + 16 RT of the tile's positions: SwiGLU into h
// (gate_up) or y / bf16 logits (down); int8 row scales applied here.
// yrow: the output row of this lane's position (down).
// up: gate_up's first up row (int8 scales); out: h (rows hstride apart) or y.
template <int WF, int PHASE, int RT>
__device__ __forceinline__ void gemv_epilogue(const GemmArgs& a, const f32x4 (&acc)[PHASE == PHASE_GATE_UP ? 2 * RT : RT],
                                              int rows, int row0, int orow0, const uint16_t* sexp, int up, void* out,
                                              int hstride, uint32_t lane, int yrow) {
  const int t_out = lane & 15;
  if (t_out >= rows) return;
  const int64_t pos = row0 + t_out;
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const int orow = orow0 + 16 * r + 4 * (lane >> 4);
    f32x4 s0 = acc[r];
    if (PHASE == PHASE_GATE_UP) {
      f32x4 s1 = acc[RT + r];
      if (WF == WF_I8) {
        s0 *= bf16x4_to_f32(*(const u32x2*)(sexp + orow));
        s1 *= bf16x4_to_f32(*(const u32x2*)(sexp + up + orow));
      }
      float h[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) h[v] = silu_f32(s0[v]) * s1[v];
      u32x2 pk;
      pk[0] = pack_bf16x2(h[0], h[1]);
      pk[1] = pack_bf16x2(h[2], h[3]);
      *(u32x2*)((uint16_t*)out + pos * hstride + orow) = pk;
    } else {
      if (WF == WF_I8) s0 *= bf16x4_to_f32(*(const u32x2*)(sexp + orow));
      if (a.out_cols > 0) {
        // bf16 [rows, out_cols] (router logits): columns past out_cols are padding
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (orow + v < a.out_cols)
            ((uint16_t*)out)[pos * a.out_cols + orow + v] = (uint16_t)f32_to_bf16_bits(s0[v]);
      } else {
        *(f32x4*)((float*)out + (int64_t)yrow * a.N + orow) = s0;
      }
    }
  }
}

// Where one tile's operands live: its weight blocks and scales (expert base),
// gate_up's first up row, the K extent of a stored weight row (the stride of
// its 16-row blocks), the activation rows (xstride elements apart) and
// gate_up's output row stride (h).
struct TileSrc {
  const uint8_t* w;
  const uint16_t* s;
  const uint8_t* x;
  int up;
  int kstride;
  int xstride;
  int hstride;
};

__device__ __forceinline__ TileSrc routed_src(const GemmArgs& a, int expert) {
  return TileSrc{a.w + (int64_t)expert * a.w_expert_bytes, a.scales + (int64_t)expert * a.s_expert_elems,
                 (const uint8_t*)a.in, a.I, a.K, a.K, a.I};
}

// Chunk c of the shared expert (GemmArgs::sh_chunks): gate_up rows [cI, cI + I)
// of the gate and the up projection (sh_I rows apart), output columns
// [cI, cI + I) of the shared h rows (sh_I apart); down the K range
// [cI, cI + I) of every row, its input the same columns of the shared h.
template <int WF, int PHASE>
__device__ __forceinline__ TileSrc shared_chunk_src(const GemmArgs& a, int c) {
  if (PHASE == PHASE_GATE_UP) {
    const int r0 = c * a.I;
    return TileSrc{a.sh_w + (int64_t)(r0 >> 4) * (a.K / block_k(WF)) * 1024,
                   WF == WF_BF16 ? a.sh_scales : a.sh_scales + (int64_t)r0 * (WF == WF_I4 ? a.K / 128 : 1),
                   (const uint8_t*)a.in, a.sh_I, a.K, a.K, a.sh_I};
  }
  return TileSrc{a.sh_w + (int64_t)c * (a.K / block_k(WF)) * 1024,
                 WF == WF_I4 ? a.sh_scales + (int64_t)c * (a.K / 128) * 16 : a.sh_scales,
                 (const uint8_t*)a.sh_h + (int64_t)c * a.K * 2, 0, a.sh_I, a.sh_I, 0};
}

}  // namespace

// One (tile, row set, K part) of the decode form: this wave's fp32 partial
// sums of the row set's NT 16-row output tiles for the tile's positions,
// columns = positions (16 at most, rows of them real).  ts: where the tile's
// operands live; src / srcq: the input row of the lane's column in the full /
// quad form; region: this wave's LDS staging area (NG KiB + the int4 scales).
template <int WF, int PHASE, int RT, int S, int NG, int D, bool FULL, bool STREAM>
__device__ __forceinline__ void gemv_accumulate(const GemmArgs& a, const TileSrc& ts, int rows, int src, int srcq,
                                                int kpart, int rowset, uint8_t* region, uint32_t lane,
                                                f32x4 (&acc)[PHASE == PHASE_GATE_UP ? 2 * RT : RT]) {
  constexpr int NT = (PHASE == PHASE_GATE_UP) ? 2 * RT : RT;
  constexpr int kStageX = NG * 1024;
  const int col = lane & 15;
  const int G = a.K / 128;
  const int NKB = ts.kstride / block_k(WF);  // blocks per stored 16-row block
  const int GS = ts.kstride / 128;           // scale groups per stored row
  const uint8_t* xbase = ts.x + 16 * (lane >> 4);

  const uint8_t* wexp = ts.w;
  const uint16_t* sexp = ts.s;
  const int orow0 = rowset * RT * 16;  // first output row of the row set
  uint32_t rbo[NT], sbo[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int wrow = (PHASE == PHASE_GATE_UP) ? (t < RT ? orow0 + 16 * t : ts.up + orow0 + 16 * (t - RT))
                                              : orow0 + 16 * t;
    const uint32_t rb = (uint32_t)(wrow >> 4);
    rbo[t] = rb * (uint32_t)NKB * 1024u;
    sbo[t] = rb * (uint32_t)GS * 16u;
  }

  // this wave's groups: kpart + S*i, i < n
  // (FULL: G == S * NG, every wave has exactly NG groups)
  const int n = FULL ? NG : kpart < G ? (G - kpart + S - 1) / S : 0;
  const int n_last = FULL ? NG - 1 : n > 0 ? n - 1 : 0;
  const int g_base = FULL ? kpart : kpart < G ? kpart : 0;
  constexpr bool IS_INT = WF == WF_I4 || WF == WF_I8;

#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (NG > 0) {
    // weights first (registers), then the scales (LDS): the activation
    // addresses may still wait for src
    WSlot<WF, NT> sl[NG > 0 ? NG : 1];
#pragma unroll
    for (int i = 0; i < NG; ++i)
      load_w<WF, NT, STREAM, false>(sl[i], wexp, sexp, rbo, sbo, g_base + S * min(i, n_last), lane);
    // the int4 scales: lane (t, i, part) = (l / 8NG, l / 8 % NG, l % 8) loads
    // 4 bytes (rows 2 part, 2 part + 1) of tile t's scales for group i
    const uint16_t* s_src = sexp;
    if (WF == WF_I4) {
      const int t = lane / (8 * NG), i = (lane / 8) % NG;
      uint32_t sb = sbo[0];
#pragma unroll
      for (int tt = 1; tt < NT; ++tt) sb = (t == tt) ? sbo[tt] : sb;
      s_src = sexp + sb + (uint32_t)(g_base + S * min(i, n_last)) * 16u + 2u * (lane % 8);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (rows <= 4) {
      // quad form: one load per group into LDS, the B operands built per step
      const uint8_t* xq_row = ts.x + (int64_t)srcq * ts.xstride * 2 + 64 * (col >> 2) + 16 * (lane >> 4);
#pragma unroll
      for (int i = 0; i < NG; ++i) load16_to_lds(xq_row + (g_base + S * min(i, n_last)) * 256, region + i * 1024);
      if (WF == WF_I4 && lane < (uint32_t)(NT * NG * 8)) load4_to_lds(s_src, region + kStageX);
      wait_vmem();
      // defined inside each form's branch (an opaque value): the int4
      // dequantisation cannot be hoisted above the branch
      const DqConst kdq = dq_const();
#pragma unroll
      for (int i = 0; i < NG; ++i) {
        const u32x4 xq = *(const u32x4*)(region + i * 1024 + lane * 16);
        if (WF == WF_I4)
#pragma unroll
          for (int t = 0; t < NT; ++t) sl[i].s[t] = *(const u32x2*)(region + kStageX + (t * NG + i) * 32 + 8 * (lane >> 4));
        if (WF != WF_I4) pin_slot<WF, NT>(sl[i]);  // (int4: the constants above)
        mma_group_b<WF, NT>(sl[i], [&](int st) { return quad_operand(xq, st); }, IS_INT ? quad_group_sum(xq) : 0.f,
                            acc, FULL || i < n, kdq);
      }
    } else {
      // larger tiles: full B operands in registers, one group's at a time
      const uint8_t* xrow = xbase + (int64_t)src * ts.xstride * 2;
      if (WF == WF_I4 && lane < (uint32_t)(NT * NG * 8)) load4_to_lds(s_src, region + kStageX);
      const DqConst kdq = dq_const();
#pragma unroll
      for (int i = 0; i < NG; ++i) {
        u32x4 xb[4];
        load_x_full(xb, xrow, g_base + S * min(i, n_last));
        wait_vmem();
        if (WF == WF_I4)
#pragma unroll
          for (int t = 0; t < NT; ++t) sl[i].s[t] = *(const u32x2*)(region + kStageX + (t * NG + i) * 32 + 8 * (lane >> 4));
        if (WF != WF_I4) pin_slot<WF, NT>(sl[i]);
        mma_group_b<WF, NT>(sl[i], [&](int st) { return xb[st]; }, IS_INT ? group_sum_full(xb) : 0.f, acc,
                            FULL || i < n, kdq);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  } else if (rows <= 4) {
    // the ring with quad-form activations (one register load per group)
    const uint8_t* xq_row = ts.x + (int64_t)srcq * ts.xstride * 2 + 64 * (col >> 2) + 16 * (lane >> 4);
    WSlot<WF, NT> rw[D];
    u32x4 rx[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int g = g_base + S * min(d, n_last);
      load_w<WF, NT, STREAM>(rw[d], wexp, sexp, rbo, sbo, g, lane);
      rx[d] = *(const u32x4*)(xq_row + g * 256);
    }
    __builtin_amdgcn_sched_barrier(0);
    const DqConst kdq = dq_const();
    for (int i0 = 0; i0 < n; i0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        if (WF != WF_I4) pin_slot<WF, NT>(rw[d]);
        const u32x4 xq = rx[d];
        mma_group_b<WF, NT>(rw[d], [&](int st) { return quad_operand(xq, st); }, IS_INT ? quad_group_sum(xq) : 0.f,
                            acc, i0 + d < n, kdq);
        __builtin_amdgcn_sched_barrier(0);
        const int g = g_base + S * min(i0 + d + D, n_last);
        load_w<WF, NT, STREAM>(rw[d], wexp, sexp, rbo, sbo, g, lane);
        rx[d] = *(const u32x4*)(xq_row + g * 256);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  } else {
    const uint8_t* xrow = xbase + (int64_t)src * ts.xstride * 2;
    RSlot<WF, NT> ring[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int g = g_base + S * min(d, n_last);
      load_w<WF, NT, STREAM>(ring[d].w, wexp, sexp, rbo, sbo, g, lane);
      load_x_full(ring[d].x, xrow, g);
    }
    // sched_barrier: the scheduler would otherwise sink each refill down to
    // its use in the next iteration (shorter live ranges, no latency hiding)
    __builtin_amdgcn_sched_barrier(0);
    const DqConst kdq = dq_const();
    for (int i0 = 0; i0 < n; i0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        if (WF != WF_I4) pin_slot<WF, NT>(ring[d].w);
        mma_group_b<WF, NT>(ring[d].w, [&](int st) { return ring[d].x[st]; },
                            IS_INT ? group_sum_full(ring[d].x) : 0.f, acc, i0 + d < n, kdq);
        __builtin_amdgcn_sched_barrier(0);
        const int g = g_base + S * min(i0 + d + D, n_last);
        load_w<WF, NT, STREAM>(ring[d].w, wexp, sexp, rbo, sbo, g, lane);
        load_x_full(ring[d].x, xrow, g);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

}

// Waves per workgroup: S K-parts of P row sets.
__host__ __device__ constexpr int gemv_rowsets_per_wg(int S) { return S == 1 ? 4 : S == 2 ? 2 : 1; }

// Grid: x = blocks of P row sets, y = tile slots (a slot past the routed tile
// count exits at once).  NG > 0: each wave issues the loads of all its (at
// most NG) groups at once and then consumes them; NG == 0: each wave streams
// its groups through the D-deep ring.
// ROUTE (gate_up, one token): the tile record comes from routing the
// token inside the workgroup (GemmArgs::route_logits) instead of K2's list.
// SH: tiles from GemmArgs::sh_tile0 on may be the shared expert's chunks
// (a separate instance, so the routed-only launches carry none of it; the
// ROUTE instance always may).
template <int WF, int PHASE, int RT, int S, int NG, int D, bool FULL, bool ROUTE = false, bool SH = false>
__global__ void __launch_bounds__(S * gemv_rowsets_per_wg(S) * 64) gemv_kernel(GemmArgs a, int n_rowsets) {
  constexpr int P = gemv_rowsets_per_wg(S);
  constexpr int NT = (PHASE == PHASE_GATE_UP) ? 2 * RT : RT;
  // Per-wave LDS region: the direct-to-LDS staging of the quad-form
  // activations (NG KiB) and the int4 scales (32 B per tile and group), then
  // reused for the wave's K-part partial sums (NT KiB).
  constexpr int kStageX = NG * 1024;
  constexpr int kStageS = (WF == WF_I4) ? NT * NG * 32 : 0;
  constexpr int kRed = S > 1 ? NT * 1024 : 0;
  constexpr int kRegion = (kStageX + kStageS > kRed ? kStageX + kStageS : kRed) > 16
                              ? (kStageX + kStageS > kRed ? kStageX + kStageS : kRed)
                              : 16;
  __shared__ __attribute__((aligned(16))) uint8_t lds[S * P][kRegion];
  __shared__ uint32_t arrived[P];  // K parts of each row set that have stored their sums

  const int tile = blockIdx.y;
  const uint32_t lane = threadIdx.x & 63;
  const int col = lane & 15;
  // a tile of the shared expert's chunks (GemmArgs::sh_chunks): no tile record
  const int sh_j = tile - a.sh_tile0;
  const bool sh_batch = SH && a.sh_chunks > 0 && sh_j >= 0;
  // the input row of the lane's column comes straight from the tile index, so
  // this load is issued first and waiting for it never waits for weights
  int src = 0, srcq = 0;
  if (!ROUTE && a.tile_src && !sh_batch) {
    src = a.tile_src[tile * kTileSrcCols + col];
    srcq = a.tile_src[tile * kTileSrcCols + (col & 3)];
  }

  const int wave = threadIdx.x >> 6;
  const int kpart = wave % S;
  const int rs_raw = blockIdx.x * P + wave / S;
  const bool rs_ok = rs_raw < n_rowsets;
  const int rowset = rs_ok ? rs_raw : 0;

  // routed tiles: K2 writes every record up to the grid's max_tiles, those
  // past the last tile with no rows (no wait for the tile count)
  int expert = 0, row0 = 0, rows = 0;
  int shc = -1;  // the shared-expert chunk of a shared tile, else -1
  if (sh_batch) {
    const int nT = (a.sh_tokens + 15) >> 4;
    shc = sh_j / nT;
    row0 = (sh_j - shc * nT) * 16;
    rows = shc < a.sh_chunks ? min(16, a.sh_tokens - row0) : 0;
    // K4 for chunk 0's tokens: wave 0 of the tile's workgroups, one token each
    if (PHASE == PHASE_GATE_UP && shc == 0 && wave == 0) {
      for (int t = blockIdx.x; t < rows; t += gridDim.x) {
        const float g = shared_gate_value(a.in, a.sh_gate_w, a.act_bf16, row0 + t, a.K, (int)lane);
        if (lane == 0) a.sh_gate[row0 + t] = g;
      }
    }
  }
  if (ROUTE) {
    // K1 on the token's logits by wave 0 (the same code and bits as the
    // routing kernels; workgroup (0, 0) the whole of it, the others its
    // selection alone); tile = position = rank of the expert id among the k.
    // Tiles k .. k + sh_chunks - 1 (sh_tile0 = k) are the shared expert's
    // chunks: no routing, and wave 0 of workgroup (0, k) computes its gate.
    __shared__ float rsv[kMaxTopK];
    __shared__ int rsi[kMaxTopK];
    __shared__ int rids[kMaxTopK];
    __shared__ int rpos[kMaxTopK];
    __shared__ int r_expert;
    __shared__ uint32_t rmask[8];
    const int k = a.topk;
    const bool first = blockIdx.x == 0 && tile == 0;
    if (tile >= k && tile < k + a.sh_chunks) shc = tile - k;
    if (wave == 0 && shc == 0 && blockIdx.x == 0) {
      const float g = shared_gate_value(a.in, a.sh_gate_w, a.act_bf16, 0, a.K, (int)lane);
      if (lane == 0) a.sh_gate[0] = g;
    }
    if (wave == 0 && shc < 0 && !first) {
      // only the tile's expert: K1's selection (route_mask, the same bits),
      // then the tile-th selected id in ascending order
      route_mask<2, true>(a.route_logits, 0, a.route_E, k, a.route_flags, rmask);
      if (lane == 0) {
        int r = tile, e = 0;
        for (int wd = 0; wd < 4; ++wd) {
          const int c = __popc(rmask[wd]);
          if (r >= 0 && r < c) e = 32 * wd + nth_set_bit(rmask[wd], r);
          r -= c;
        }
        r_expert = e;
      }
    }
    if (wave == 0 && shc < 0 && first) {
      int id;
      float w;
      route_token<2, true>(a.route_logits, 0, a.route_E, k, a.route_flags, rsv, rsi, &id, &w);
      int pos = 0;
      for (int i = 0; i < k; ++i) pos += (__builtin_amdgcn_readlane(id, i) < id) ? 1 : 0;
      if ((int)lane < k) {
        rids[lane] = id;
        rpos[lane] = pos;
        if (pos == tile) r_expert = id;
        a.ro_ids[lane] = id;
        a.ro_w[lane] = w;
        a.ro_perm[pos] = lane;
        a.ro_inv[lane] = pos;
        a.ro_wpos[pos] = w;
      }
    }
    __syncthreads();
    if (first) {
      // K2 for one token: expert e holds position (#ids below e) if picked
      const int nth = S * P * 64;
      for (int e = threadIdx.x; e < a.route_E; e += nth) {
        int c = 0, o = 0;
        for (int i = 0; i < k; ++i) {
          c += rids[i] == e ? 1 : 0;
          o += rids[i] < e ? 1 : 0;
        }
        a.ro_counts[e] = c;
        a.ro_offsets[e] = o;
      }
      if (threadIdx.x == 0) {
        a.ro_offsets[a.route_E] = k;
        a.ro_n_tiles[0] = k;
      }
      for (int ti = threadIdx.x; ti < a.ro_max_tiles; ti += nth) {
        int e = 0;
        for (int i = 0; i < k; ++i) e = rpos[i] == ti ? rids[i] : e;
        *(int4*)(a.ro_tiles + 4 * ti) = ti < k ? int4{e, ti, 1, 0} : int4{0, 0, 0, 0};
      }
      for (int i = threadIdx.x; i < a.ro_max_tiles * kTileSrcCols; i += nth) a.ro_tile_src[i] = 0;
    }
    expert = shc < 0 ? r_expert : 0;
    row0 = shc < 0 ? tile : 0;
    rows = tile < k || shc >= 0 ? 1 : 0;
    src = 0;
    srcq = 0;
  } else if (sh_batch) {
    // tokens row0 .. row0 + rows - 1 of x (gate_up) or of the shared h (down)
  } else if (a.n_tiles) {
    const int4 rec = *(const int4*)(a.tiles + 4 * tile);
    expert = rec.x;
    row0 = rec.y;
    rows = rec.z;
  } else {
    expert = 0;
    row0 = tile * 16;
    rows = min(16, a.num_rows - row0);
  }
  if (rows <= 0) return;
  // split-K reduction by the last of a row set's waves to arrive (the others
  // end at once): measured faster for six or more K parts of the down
  // projection and of int4 gate_up (Mixtral), slower for fewer parts and
  // for int8 gate_up, which keep the workgroup barrier
  constexpr bool kLastReduces = S >= 6 && (PHASE == PHASE_DOWN || WF == WF_I4);
  if (kLastReduces) {
    if (threadIdx.x < P) arrived[threadIdx.x] = 0u;
    __syncthreads();
  }
  // down: the output row of this lane's position, loaded before the K loop
  int yrow = row0 + (lane & 15);
  const bool sh = (ROUTE || SH) && shc >= 0;
  if (PHASE == PHASE_DOWN && a.out_rows && !sh && (int)(lane & 15) < rows) yrow = a.out_rows[yrow];
  if (!ROUTE && (!a.tile_src || sh)) {  // rows read in place
    src = row0 + (col < rows ? col : 0);
    srcq = row0 + ((col & 3) < rows ? (col & 3) : 0);
  }
  const TileSrc ts = sh ? shared_chunk_src<WF, PHASE>(a, shc) : routed_src(a, expert);
  const int orow0 = rowset * RT * 16;  // first output row of the row set
  f32x4 acc[NT];
  // streaming weight loads for tiles below 16 positions (ROUTE: one position
  // per tile; int8 keeps the default policy there)
  if ((ROUTE && WF != WF_I8) || (!ROUTE && rows < 16))
    gemv_accumulate<WF, PHASE, RT, S, NG, D, FULL, true>(a, ts, rows, src, srcq, kpart, rowset,
                                                         lds[__builtin_amdgcn_readfirstlane(wave)], lane, acc);
  else
    gemv_accumulate<WF, PHASE, RT, S, NG, D, FULL, false>(a, ts, rows, src, srcq, kpart, rowset,
                                                          lds[__builtin_amdgcn_readfirstlane(wave)], lane, acc);

  if (S > 1 && !kLastReduces) {
    // each wave's partial sums go to its own region (its staged data is
    // consumed), the K part 0 wave adds the S parts in order
#pragma unroll
    for (int t = 0; t < NT; ++t) *(f32x4*)(lds[wave] + t * 1024 + lane * 16) = acc[t];
    __syncthreads();
    if (kpart != 0) return;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f32x4 s = *(const f32x4*)(lds[wave] + t * 1024 + lane * 16);
#pragma unroll
      for (int k = 1; k < S; ++k) s += *(const f32x4*)(lds[wave + k] + t * 1024 + lane * 16);
      acc[t] = s;
    }
  }
  if (kLastReduces) {
    // each wave's partial sums go to its own region (its staged data is
    // consumed); the last of the row set's S waves to arrive (an LDS counter:
    // LDS operations of a wave complete in order, so every earlier arrival's
    // sums are visible to it) adds the S parts in K-part order, the others
    // end at once and free their registers
#pragma unroll
    for (int t = 0; t < NT; ++t) *(f32x4*)(lds[wave] + t * 1024 + lane * 16) = acc[t];
    const int rs_local = wave / S;
    uint32_t prior = 0;
    if (lane == 0) prior = __hip_atomic_fetch_add(&arrived[rs_local], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
    prior = __builtin_amdgcn_readfirstlane(prior);
    if (prior != (uint32_t)(S - 1)) return;
    const int base = rs_local * S;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f32x4 s = *(const f32x4*)(lds[base] + t * 1024 + lane * 16);
#pragma unroll
      for (int k = 1; k < S; ++k) s += *(const f32x4*)(lds[base + k] + t * 1024 + lane * 16);
      acc[t] = s;
    }
  }
  if (!rs_ok) return;
  void* out = a.out;
  if (sh)
    out = PHASE == PHASE_GATE_UP ? (void*)((uint16_t*)a.sh_h + (int64_t)shc * a.I)
                                 : (void*)(a.sh_y + (int64_t)shc * a.sh_tokens * a.N);
  // (ROUTE: one token, position 0, so the h row stride does not matter)
  gemv_epilogue<WF, PHASE, RT>(a, acc, rows, row0, orow0, ts.s, ts.up, out, ROUTE ? a.I : ts.hstride, lane, yrow);
}

// ---------------------------------------------------------------------------
// Decode gate_up that routes its tokens itself (2 .. kSrMaxTokens tokens,
// given bf16 logits), so no routing launch precedes it.  Grid: x = blocks of
// P row sets, y = 1 + lanes.
//   * Workgroup (0, 0) runs K1 + K2 for every token (route_group_body, the
//     routing kernels' code) and writes their outputs for the down GEMV and
//     the combine, which run after this launch; workgroups (x > 0, 0) end.
//   * Every other workgroup finds the token sets itself: wave w selects
//     tokens w, w + waves, ... (route_mask: K1's selection bits), wave 0
//     transposes the token masks into per-expert masks M_e and scans
//     count_e in expert order, so expert e's first position is K2's
//     offset_e and token t's position is offset_e + its rank in M_e (K2's
//     order); the HBM-resident experts with tokens are listed in id order.
//     Lane y - 1 of the row set block takes listed experts y - 1,
//     y - 1 + lanes, ...: each is one tile of at most 16 positions (its rows
//     gathered from x by M_e), computed as gemv_kernel computes a routed
//     tile, the K parts added in order, h stored at the positions.
// The lane loop meets at two workgroup barriers per expert (the K-part sums
// in LDS, then the LDS regions free for the next expert's staging).
// ---------------------------------------------------------------------------
template <int S, int P, int kRegion>
struct SrLds {
  uint8_t region[S * P][kRegion];
  uint32_t selmask[kSrMaxTokens][8];
  int32_t act_e[kMaxExperts];
  int32_t act_off[kMaxExperts];
  uint32_t act_m[kMaxExperts];
  int32_t n_act;
};

template <int WF, int RT, int S, int NG, int P, int VPL>
__global__ void __launch_bounds__(S * P * 64) gemv_sr_kernel(GemmArgs a, int n_rowsets) {
  constexpr int NT = 2 * RT;
  constexpr int kWaves = S * P;
  constexpr int D = (WF == WF_BF16) ? 2 : 3;
  constexpr int kStageX = NG * 1024;
  constexpr int kStageS = (WF == WF_I4) ? NT * NG * 32 : 0;
  constexpr int kRed = S > 1 ? NT * 1024 : 0;
  constexpr int kRegion = (kStageX + kStageS > kRed ? kStageX + kStageS : kRed) > 16
                              ? (kStageX + kStageS > kRed ? kStageX + kStageS : kRed)
                              : 16;
  union SrShared {
    SrLds<S, P, kRegion> ex;
    RouteGroupLds<kSrMaxTokens, kSrMaxTokens * kMaxTopK, kWaves> rt;
  };
  __shared__ __attribute__((aligned(16))) SrShared lds;

  const int T = a.route_T;
  const int E = a.route_E;
  const int k = a.topk;
  const int wave = threadIdx.x >> 6;
  const uint32_t lane = threadIdx.x & 63;
  if (blockIdx.y == 0) {
    if (blockIdx.x != 0) return;
    route_group_body<VPL, true, kWaves>(a.route_logits, T, E, k, a.route_flags, kTileSrcCols, a.ro_max_tiles,
                                        a.ro_ids, a.ro_w, a.ro_counts, a.ro_offsets, a.ro_perm, a.ro_inv, a.ro_tiles,
                                        a.ro_n_tiles, a.ro_tile_src, a.ro_resident, a.ro_wpos, lds.rt);
    return;
  }
  SrLds<S, P, kRegion>& L = lds.ex;
  // residency of the scan lane's experts, read before the selection
  unsigned res = 0;
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int e = VPL * (int)lane + i;
      res |= (unsigned)(!a.ro_resident || (e < E && a.ro_resident[e])) << i;
    }
  }
  for (int t = wave; t < T; t += kWaves) route_mask<VPL, true>(a.route_logits, t, E, k, a.route_flags, L.selmask[t]);
  __syncthreads();
  if (wave == 0) {
    uint32_t m[VPL];
    int cnt[VPL], act[VPL];
    int lane_val = 0;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int e = VPL * (int)lane + i;
      m[i] = 0u;
      for (int t = 0; t < T; ++t) m[i] |= ((L.selmask[t][(e >> 5) & 7] >> (e & 31)) & 1u) << t;
      if (e >= E) m[i] = 0u;
      cnt[i] = __popc(m[i]);
      act[i] = (cnt[i] > 0 && ((res >> i) & 1u)) ? 1 : 0;
      lane_val += cnt[i] | (act[i] << 16);
    }
    const int incl = wave_inclusive_scan(lane_val);
    int run = incl - lane_val;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int r = run >> 16;
      if (act[i]) {
        L.act_e[r] = VPL * (int)lane + i;
        L.act_off[r] = run & 0xffff;
        L.act_m[r] = m[i];
      }
      run += cnt[i] | (act[i] << 16);
    }
    if (lane == 63) L.n_act = incl >> 16;
  }
  __syncthreads();

  const int n_act = L.n_act;
  const int lanes = gridDim.y - 1;
  const int col = lane & 15;
  const int kpart = wave % S;
  const int rs_raw = blockIdx.x * P + wave / S;
  const bool rs_ok = rs_raw < n_rowsets;
  const int rowset = rs_ok ? rs_raw : 0;
  const int orow0 = rowset * RT * 16;
  uint8_t* region = L.region[__builtin_amdgcn_readfirstlane(wave)];
  for (int j = blockIdx.y - 1; j < n_act; j += lanes) {
    const int expert = L.act_e[j];
    const int row0 = L.act_off[j];
    const uint32_t msk = L.act_m[j];
    const int rows = __popc(msk);
    const int src = nth_set_bit(msk, col < rows ? col : 0);
    const int srcq = nth_set_bit(msk, (int)(col & 3) < rows ? (col & 3) : 0);
    const TileSrc ts = routed_src(a, expert);
    f32x4 acc[NT];
    gemv_accumulate<WF, PHASE_GATE_UP, RT, S, NG, D, true, true>(a, ts, rows, src, srcq, kpart, rowset, region, lane, acc);
    if (S > 1) {
#pragma unroll
      for (int t = 0; t < NT; ++t) *(f32x4*)(region + t * 1024 + lane * 16) = acc[t];
      __syncthreads();
      if (kpart == 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          f32x4 sum = *(const f32x4*)(L.region[wave] + t * 1024 + lane * 16);
#pragma unroll
          for (int kk = 1; kk < S; ++kk) sum += *(const f32x4*)(L.region[wave + kk] + t * 1024 + lane * 16);
          acc[t] = sum;
        }
        if (rs_ok) gemv_epilogue<WF, PHASE_GATE_UP, RT>(a, acc, rows, row0, orow0, ts.s, ts.up, a.out, ts.hstride, lane, 0);
      }
      __syncthreads();
    } else if (rs_ok) {
      gemv_epilogue<WF, PHASE_GATE_UP, RT>(a, acc, rows, row0, orow0, ts.s, ts.up, a.out, ts.hstride, lane, 0);
    }
  }
}

// ---------------------------------------------------------------------------
// Down projection + combine for a few tokens (T <= kDcMaxTokens).  Workgroup
// (row set, t) owns 16 output rows of token t: its waves take the (pair,
// K part) items of the token's k pairs -- pair j's position inv[t k + j] (its
// h row) and expert ids[t k + j], computed as a one-position tile through
// gemv_accumulate exactly as the down GEMV computes that position's column
// (with at most 4 tokens every decode tile holds at most 4 positions, so the
// down GEMV takes the same quad form) -- and leave the column-0 partial sums
// in LDS at the rank of the position among the token's (ascending position =
// ascending expert id); then y = the K parts added in order (x the int8 row
// scale) and out = sum over the ranks in order of w y, + gate x shared expert
// row, + residual, one rounding -- the arithmetic of the down GEMV followed
// by combine_kernel, so the same bits, with no y round trip through HBM and
// no combine launch.
// With a.sh_chunks = C > 0 the shared expert's down projection rides along
// as C more items n_pos .. n_pos + C - 1 (its h row t), chunk c the K range
// [cI, cI + I) of the shared down rows (its input the same columns of the
// shared h the gate_up launch wrote); its row is the C chunk rows added in
// chunk order (each x the int8 row scale), times the gate that launch wrote.
// ---------------------------------------------------------------------------
constexpr int kDcWaves = 16;
constexpr int kDcMaxItems = 64;  // positions x K parts

template <int WF, int S, int NG, int D, bool FULL>
__global__ void __launch_bounds__(64 * kDcWaves) gemv_down_combine_kernel(GemmArgs a, CombineTail c, int n_pos) {
  constexpr int RT = 1;
  constexpr int NT = RT;
  constexpr int kStageX = NG * 1024;
  constexpr int kStageS = (WF == WF_I4) ? NT * NG * 32 : 0;
  constexpr int kRegion = kStageX + kStageS > 16 ? kStageX + kStageS : 16;
  __shared__ __attribute__((aligned(16))) uint8_t lds[kDcWaves][kRegion];
  __shared__ f32x4 part[kDcMaxItems][4];  // [rank x S + K part][lane / 16]: rows 4 (l / 16) .. + 3, column 0
  __shared__ float wrank[kMaxTopK];                         // routing weight of each rank
  __shared__ float spos[kMaxTopK + kMaxSharedChunks][16];  // int8: row scales of each rank's expert
  const uint32_t lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rowset = blockIdx.x;
  const int t = blockIdx.y;  // the token
  const int n_sh = a.sh_chunks;
  const int n_items = (n_pos + n_sh) * S;
  const int32_t* tinv = c.inv + (int64_t)t * n_pos;
  for (int q = wave; q < n_items; q += kDcWaves) {
    const int slot = q / S, kpart = q % S;
    const bool sh = slot >= n_pos;
    // the pair's position (its h row) and expert, its routing weight with
    // K part 0 (the combine's operand), and, in lanes < k, the positions of
    // the token's pairs for the rank (ascending position = ascending id)
    const int p = sh ? 0 : tinv[slot];
    const int expert = sh ? 0 : c.ids[(int64_t)t * n_pos + slot];
    const int pm = (!sh && (int)lane < n_pos) ? tinv[lane] : 0;
    float wv = 0.f;
    if (!sh && kpart == 0 && lane == 0) wv = c.w[(int64_t)t * n_pos + slot];
    float sc = 0.f;
    if (WF == WF_I8 && kpart == 0 && lane < 16u)
      sc = bf16_bits_to_f32(sh ? a.sh_scales[rowset * 16 + lane]
                               : a.scales[(int64_t)expert * a.s_expert_elems + rowset * 16 + lane]);
    const TileSrc ts = sh ? shared_chunk_src<WF, PHASE_DOWN>(a, slot - n_pos) : routed_src(a, expert);
    const int src = sh ? t : p;
    f32x4 acc[NT];
    gemv_accumulate<WF, PHASE_DOWN, RT, S, NG, D, FULL, WF != WF_I8>(a, ts, 1, src, src, kpart, rowset, lds[wave], lane, acc);
    const int rank = sh ? slot : (int)__popcll(__ballot((int)lane < n_pos && pm < p));
    if ((lane & 15) == 0) part[rank * S + kpart][lane >> 4] = acc[0];
    if (kpart == 0) {
      if (!sh && lane == 0) wrank[rank] = wv;
      if (WF == WF_I8 && lane < 16u) spos[rank][lane] = sc;
    }
  }
  __syncthreads();
  if (threadIdx.x >= 16) return;
  {
  // every product rounded before it is added, as combine_kernel adds its
  // terms (never fused into an FMA): the same bits as the separate launches
#pragma clang fp contract(off)
  // thread r: output row orow0 + r (tile row r = 4 (r / 4) + r % 4 of lane group r / 4)
  const int r = threadIdx.x;
  const int orow = rowset * 16 + r;
  const int64_t o = (int64_t)t * a.N + orow;
  float acc = 0.f;
  for (int p = 0; p < n_pos; ++p) {
    float y = part[p * S][r >> 2][r & 3];
    for (int kp = 1; kp < S; ++kp) y += part[p * S + kp][r >> 2][r & 3];
    if (WF == WF_I8) y *= spos[p][r];
    const float term = wrank[p] * y;
    acc = p == 0 ? term : acc + term;
  }
  if (n_sh > 0) {
    float ys = 0.f;
    for (int j = 0; j < n_sh; ++j) {
      const int p = n_pos + j;
      float y = part[p * S][r >> 2][r & 3];
      for (int kp = 1; kp < S; ++kp) y += part[p * S + kp][r >> 2][r & 3];
      if (WF == WF_I8) y *= spos[p][r];
      ys = j == 0 ? y : ys + y;
    }
    acc += c.shared_gate[t] * ys;
  } else if (c.y_shared) {
    acc += c.shared_gate[t] * c.y_shared[o];
  }
  if (c.residual) acc += bf16_bits_to_f32(((const uint16_t*)c.residual)[o]);
  ((uint16_t*)c.out)[o] = (uint16_t)f32_to_bf16_bits(acc);
  }
}

// ---------------------------------------------------------------------------
// launch
// ---------------------------------------------------------------------------
namespace {

template <int WF, int PHASE, int RT, int S, int NG>
hipError_t launch_gemv_s(const GemmArgs& a, int max_tiles, int n_rowsets, hipStream_t stream,
                         const KernelTimer* tm) {
  constexpr int P = gemv_rowsets_per_wg(S);
  constexpr int D = (WF == WF_BF16) ? 2 : 3;
  dim3 grid((n_rowsets + P - 1) / P, max_tiles);
  const bool full = NG > 0 && a.K / 128 == S * NG;
  if constexpr (PHASE == PHASE_GATE_UP) {
    if (a.route_logits) {
      if (full)
        launch_timed(gemv_kernel<WF, PHASE, RT, S, NG, D, true, true>, grid, dim3(S * P * 64), 0, stream, tm, a,
                     n_rowsets);
      else
        launch_timed(gemv_kernel<WF, PHASE, RT, S, NG, D, false, true>, grid, dim3(S * P * 64), 0, stream, tm, a,
                     n_rowsets);
      return hipGetLastError();
    }
  }
  if (a.sh_chunks > 0) {
    if (full)
      launch_timed(gemv_kernel<WF, PHASE, RT, S, NG, D, true, false, true>, grid, dim3(S * P * 64), 0, stream, tm,
                   a, n_rowsets);
    else
      launch_timed(gemv_kernel<WF, PHASE, RT, S, NG, D, false, false, true>, grid, dim3(S * P * 64), 0, stream, tm,
                   a, n_rowsets);
    return hipGetLastError();
  }
  if (full)
    launch_timed(gemv_kernel<WF, PHASE, RT, S, NG, D, true>, grid, dim3(S * P * 64), 0, stream, tm, a, n_rowsets);
  else
    launch_timed(gemv_kernel<WF, PHASE, RT, S, NG, D, false>, grid, dim3(S * P * 64), 0, stream, tm, a, n_rowsets);
  return hipGetLastError();
}

// Every wave takes NG K groups and issues all of their loads at once (many
// short waves stream HBM better than few long ones): a target of 4 groups
// of int4 (8 KiB of weights for two row tiles) or int8 (16 KiB; measured
// against 2 groups: Qwen1.5-MoE T = 4 / 16 48.7 / 95 -> 45.5 / 89 us, Qwen3
// int8 T = 16 45.5 -> 44.1 us) and 2 of bf16.  The S = ceil(G / target) K
// parts (at most 8) then split the G groups as evenly as they go,
// NG = ceil(G / S) each; K too long for eight parts of four groups streams
// through the ring instead.
__host__ __device__ constexpr int gemv_target_groups(int wf) { return wf == WF_BF16 ? 2 : 4; }

template <int WF, int PHASE, int RT, int NG>
hipError_t launch_gemv_ng(const GemmArgs& a, int S, int max_tiles, int n_rowsets, hipStream_t stream,
                          const KernelTimer* tm) {
  switch (S) {
    case 1:
      return launch_gemv_s<WF, PHASE, RT, 1, NG>(a, max_tiles, n_rowsets, stream, tm);
    case 2:
      return launch_gemv_s<WF, PHASE, RT, 2, NG>(a, max_tiles, n_rowsets, stream, tm);
    case 3:
      return launch_gemv_s<WF, PHASE, RT, 3, NG>(a, max_tiles, n_rowsets, stream, tm);
    case 4:
      return launch_gemv_s<WF, PHASE, RT, 4, NG>(a, max_tiles, n_rowsets, stream, tm);
    case 5:
    case 6:
      return launch_gemv_s<WF, PHASE, RT, 6, NG>(a, max_tiles, n_rowsets, stream, tm);
    default:
      return launch_gemv_s<WF, PHASE, RT, 8, NG>(a, max_tiles, n_rowsets, stream, tm);
  }
}

template <int WF, int PHASE, int RT>
hipError_t launch_gemv_rt(const GemmArgs& a, int max_tiles, hipStream_t stream, const KernelTimer* tm) {
  const int out_dim = (PHASE == PHASE_GATE_UP) ? a.I : a.N;
  const int n_rowsets = out_dim / (RT * 16);
  const int G = a.K / 128;
  constexpr int target = gemv_target_groups(WF);
  int S = (G + target - 1) / target;
  if (S > 8) S = 8;
  if (S == 5 || S == 7) ++S;  // instantiated part counts: 1, 2, 3, 4, 6, 8
  const int NG = (G + S - 1) / S;
  switch (NG) {
    case 1:
      return launch_gemv_ng<WF, PHASE, RT, 1>(a, S, max_tiles, n_rowsets, stream, tm);
    case 2:
      return launch_gemv_ng<WF, PHASE, RT, 2>(a, S, max_tiles, n_rowsets, stream, tm);
    case 3:
      return launch_gemv_ng<WF, PHASE, RT, 3>(a, S, max_tiles, n_rowsets, stream, tm);
    case 4:
      return launch_gemv_ng<WF, PHASE, RT, 4>(a, S, max_tiles, n_rowsets, stream, tm);
    default:
      return launch_gemv_s<WF, PHASE, RT, 8, 0>(a, max_tiles, n_rowsets, stream, tm);
  }
}

template <int WF, int S, int NG>
hipError_t launch_down_combine_s(const GemmArgs& a, const CombineTail& c, int n_pos, hipStream_t stream) {
  constexpr int D = (WF == WF_BF16) ? 2 : 3;
  dim3 grid(a.N / 16, c.tokens), block(64 * kDcWaves);
  if (NG > 0 && a.K / 128 == S * NG)
    hipLaunchKernelGGL((gemv_down_combine_kernel<WF, S, NG, D, true>), grid, block, 0, stream, a, c, n_pos);
  else
    hipLaunchKernelGGL((gemv_down_combine_kernel<WF, S, NG, D, false>), grid, block, 0, stream, a, c, n_pos);
  return hipGetLastError();
}

template <int WF, int NG>
hipError_t launch_down_combine_ng(const GemmArgs& a, const CombineTail& c, int n_pos, int S, hipStream_t stream) {
  switch (S) {
    case 1:
      return launch_down_combine_s<WF, 1, NG>(a, c, n_pos, stream);
    case 2:
      return launch_down_combine_s<WF, 2, NG>(a, c, n_pos, stream);
    case 3:
      return launch_down_combine_s<WF, 3, NG>(a, c, n_pos, stream);
    case 4:
      return launch_down_combine_s<WF, 4, NG>(a, c, n_pos, stream);
    case 5:
    case 6:
      return launch_down_combine_s<WF, 6, NG>(a, c, n_pos, stream);
    default:
      return launch_down_combine_s<WF, 8, NG>(a, c, n_pos, stream);
  }
}

// the K split of the down GEMV (launch_gemv_rt), so the partial sums match it
template <int WF>
hipError_t launch_down_combine_wf(const GemmArgs& a, const CombineTail& c, int n_pos, hipStream_t stream) {
  const int G = a.K / 128;
  constexpr int target = gemv_target_groups(WF);
  int S = (G + target - 1) / target;
  if (S > 8) S = 8;
  if (S == 5 || S == 7) ++S;
  const int NG = (G + S - 1) / S;
  if ((n_pos + a.sh_chunks) * S > kDcMaxItems) return hipErrorInvalidValue;
  switch (NG) {
    case 1:
      return launch_down_combine_ng<WF, 1>(a, c, n_pos, S, stream);
    case 2:
      return launch_down_combine_ng<WF, 2>(a, c, n_pos, S, stream);
    case 3:
      return launch_down_combine_ng<WF, 3>(a, c, n_pos, S, stream);
    case 4:
      return launch_down_combine_ng<WF, 4>(a, c, n_pos, S, stream);
    default:
      return launch_down_combine_s<WF, 8, 0>(a, c, n_pos, stream);
  }
}

template <int WF>
hipError_t launch_gemv_wf(const GemmArgs& a, int phase, int max_tiles, hipStream_t stream,
                          const KernelTimer* tm) {
  if (phase == PHASE_GATE_UP) return launch_gemv_rt<WF, PHASE_GATE_UP, kGemvRtGateUp>(a, max_tiles, stream, tm);
  // few tiles (the shared expert: one): one row tile per wave doubles the
  // waves streaming the weights
  if ((int64_t)(a.N / (kGemvRtDown * 16)) * max_tiles < kGemvFewWaves && a.N % 16 == 0)
    return launch_gemv_rt<WF, PHASE_DOWN, 1>(a, max_tiles, stream, tm);
  return launch_gemv_rt<WF, PHASE_DOWN, kGemvRtDown>(a, max_tiles, stream, tm);
}

// the decode gate_up's K split (launch_gemv_rt), so h has the same bits
void gemv_split(int wf, int K, int& S, int& NG) {
  const int G = K / 128;
  const int target = gemv_target_groups(wf);
  S = (G + target - 1) / target;
  if (S > 8) S = 8;
  if (S == 5 || S == 7) ++S;
  NG = (G + S - 1) / S;
}

// Lanes of the self-routing gate_up: each active expert a lane of its own
// up to kSrLanes, more experts shared out over them.  Measured (Qwen3 int4,
// given logits, per layer): T = 2 / 3 / 4 21.0 / 27.0 / 29.1 us with the
// routing launch against 18.0 / 24.2 / 27.5 us at 16 lanes (24, 32, 48 and
// 64 lanes, and 4 lanes at T = 2, slower); T = 8 / 16 40 / 53 against 40.4 / 58.5 at 16
// lanes and more with more lanes (every workgroup selects every token, so
// the selection work grows with both), and slower again with two or four
// row sets per workgroup (fewer, fatter workgroups): hence at most
// kSrMaxTokens tokens.
constexpr int kSrLanes = 16;

template <int WF>
hipError_t launch_gemv_sr_wf(const GemmArgs& a, int lanes, hipStream_t stream, const KernelTimer* tm) {
  constexpr int S = 4, NG = 4, P = 1;  // the split gemv_sr_supported admits, one row set per workgroup
  const int n_rowsets = a.I / (kGemvRtGateUp * 16);
  dim3 grid((n_rowsets + P - 1) / P, 1 + lanes);
  launch_timed(gemv_sr_kernel<WF, kGemvRtGateUp, S, NG, P, 2>, grid, dim3(S * P * 64), 0, stream, tm, a, n_rowsets);
  return hipGetLastError();
}

}  // namespace

bool gemv_supported(int wf, int phase, int N, int K, int I) {
  if (wf != WF_BF16 && wf != WF_I8 && wf != WF_I4) return false;
  if (K % 128 != 0) return false;
  const int out_dim = phase == PHASE_GATE_UP ? I : N;
  const int rows_per_set = (phase == PHASE_GATE_UP ? kGemvRtGateUp : kGemvRtDown) * 16;
  return out_dim % rows_per_set == 0;
}

int64_t gemv_workgroups(int wf, int phase, int N, int K, int I, int max_tiles) {
  const int RT = phase == PHASE_GATE_UP ? kGemvRtGateUp : kGemvRtDown;
  const int out_dim = phase == PHASE_GATE_UP ? I : N;
  const int G = K / 128;
  const int target = gemv_target_groups(wf);
  int S = (G + target - 1) / target;
  if (S > 8) S = 8;
  if (S == 5 || S == 7) ++S;
  const int P = gemv_rowsets_per_wg(S);
  const int n_rowsets = out_dim / (RT * 16);
  return (int64_t)((n_rowsets + P - 1) / P) * max_tiles;
}

bool down_combine_supported(int wf, int N, int K, int I, int n_pos) {
  if (!gemv_supported(wf, PHASE_DOWN, N, K, I) || N % 16 != 0 || n_pos < 1 || n_pos > kMaxTopK + kMaxSharedChunks)
    return false;
  const int G = K / 128;
  const int target = gemv_target_groups(wf);
  int S = (G + target - 1) / target;
  if (S > 8) S = 8;
  if (S == 5 || S == 7) ++S;
  return n_pos * S <= kDcMaxItems;
}

hipError_t launch_down_combine(const GemmArgs& a, const CombineTail& c, int wf, int n_pos, hipStream_t stream) {
  if (!c.w || !c.ids || !c.inv || !c.out || n_pos < 1 || n_pos > kMaxTopK || c.tokens < 1 ||
      c.tokens > kDcMaxTokens || (a.sh_chunks > 0 && a.sh_tokens != c.tokens))
    return hipErrorInvalidValue;
  if (a.sh_chunks < 0 || a.sh_chunks > kMaxSharedChunks ||
      (a.sh_chunks > 0 && (!a.sh_w || !a.sh_h || !c.shared_gate || (wf != WF_BF16 && !a.sh_scales) ||
                           (int64_t)a.sh_chunks * a.K != a.sh_I)))
    return hipErrorInvalidValue;
  if (!down_combine_supported(wf, a.N, a.K, a.I, n_pos + a.sh_chunks)) return hipErrorInvalidValue;
  switch (wf) {
    case WF_BF16:
      return launch_down_combine_wf<WF_BF16>(a, c, n_pos, stream);
    case WF_I8:
      return launch_down_combine_wf<WF_I8>(a, c, n_pos, stream);
    case WF_I4:
      return launch_down_combine_wf<WF_I4>(a, c, n_pos, stream);
    default:
      return hipErrorInvalidValue;
  }
}

bool gemv_sr_supported(int wf, int N, int K, int I, int T, int E, int k) {
  // int8 (Qwen3 shape, T = 2 / 3 / 4): 30.3 / 35.5 / 40.4 us with the
  // routing launch against 30.3 / 35.6 / 43.6 self-routed -- the longer
  // int8 GEMV gains nothing from the launch it saves
  if (wf != WF_I4) return false;
  if (!gemv_supported(wf, PHASE_GATE_UP, N, K, I)) return false;
  int S = 0, NG = 0;
  gemv_split(wf, K, S, NG);
  if (S != 4 || NG != 4 || K != 128 * S * NG) return false;
  return T >= 2 && T <= kSrMaxTokens && E > 64 && E <= 128 && k >= 1 && k <= kMaxTopK;
}

hipError_t launch_gemv_sr(const GemmArgs& a, int wf, int lanes, hipStream_t stream, const KernelTimer* tm) {
  if (!gemv_sr_supported(wf, a.N, a.K, a.I, a.route_T, a.route_E, a.topk) || !a.route_logits || !a.act_bf16 ||
      !a.out || !a.ro_ids || !a.ro_w || !a.ro_counts || !a.ro_offsets || !a.ro_perm || !a.ro_inv || !a.ro_tiles ||
      !a.ro_n_tiles || a.ro_max_tiles < 1 || a.sh_chunks != 0)
    return hipErrorInvalidValue;
  if (lanes <= 0) {
    const int most = a.route_T * a.topk < a.route_E ? a.route_T * a.topk : a.route_E;
    lanes = most < kSrLanes ? most : kSrLanes;
  }
  if (lanes > kMaxExperts) lanes = kMaxExperts;
  return launch_gemv_sr_wf<WF_I4>(a, lanes, stream, tm);
}

hipError_t launch_gemv(const GemmArgs& a, int wf, int phase, int max_tiles, hipStream_t stream,
                       const KernelTimer* tm) {
  if (max_tiles <= 0) return hipSuccess;
  if (a.perm && !a.tile_src) return hipErrorInvalidValue;  // gathered rows come from tile_src
  // shared-expert chunks: a tile slot for each (chunk, 16-token tile), after
  // the routed tiles (the single-token routing gate_up: right after its k)
  if (a.sh_chunks != 0) {
    const int64_t sh_tiles = (int64_t)a.sh_chunks * ((a.sh_tokens + 15) / 16);
    if (a.sh_chunks < 0 || a.sh_chunks > kMaxSharedChunks || a.sh_tokens < 1 || a.sh_tile0 < 0 ||
        a.sh_tile0 + sh_tiles > max_tiles || !a.act_bf16 || !a.sh_w || !a.sh_h ||
        (wf != WF_BF16 && !a.sh_scales) || (int64_t)a.sh_chunks * a.I != a.sh_I ||
        (a.route_logits && (a.sh_tokens != 1 || a.sh_tile0 != a.topk)))
      return hipErrorInvalidValue;
    if (phase == PHASE_GATE_UP ? (!a.sh_gate_w || !a.sh_gate) : !a.sh_y) return hipErrorInvalidValue;
  }
  switch (wf) {
    case WF_BF16:
      return launch_gemv_wf<WF_BF16>(a, phase, max_tiles, stream, tm);
    case WF_I8:
      return launch_gemv_wf<WF_I8>(a, phase, max_tiles, stream, tm);
    case WF_I4:
      return launch_gemv_wf<WF_I4>(a, phase, max_tiles, stream, tm);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace nkt
