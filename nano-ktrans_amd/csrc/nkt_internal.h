// Launch wrappers shared between the kernel files and the C ABI.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nkt {

// Device weight layout: a projection W [N, K] of one expert is cut into
// 1 KiB blocks of 16 rows x KB columns (KB = 16 fp32, 32 bf16, 64 int8,
// 128 int4).  Lane l of a wavefront reads the 16 bytes at offset 16*l of a
// block: row (l % 16) and the K values that lane feeds to the matrix core.
// Blocks are ordered (expert, row block, K block), so a wavefront streaming
// one 16-row tile over K reads consecutive kilobytes.
//   int4 block:  lane word s (s = 0..3) = columns 32s + 8*(l/16) + 0..7,
//                nibble j < 4 -> column offset 2j, nibble j >= 4 -> 2(j-4)+1,
//                stored value q + 8.
//   int8 block:  lane bytes [8s, 8s+8) (s = 0, 1) = columns 32s + 8*(l/16) + 0..7,
//                stored value q + 128.
//   bf16 block:  lane halves 0..7 = columns 8*(l/16) + 0..7.
//   fp32 block:  lane float s (s = 0..3) = column 4s + l/16.
// Scales (int formats, bf16): int4 [expert][row block][K/128][16 rows],
// int8 [expert][N].
__host__ __device__ constexpr int block_k(int wf) {
  return wf == 0 ? 16 : wf == 1 ? 32 : wf == 2 ? 64 : 128;
}

struct GemmArgs {
  const uint8_t* w;        // packed blocks, all experts
  const uint16_t* scales;  // bf16 scales (int formats) or nullptr
  int64_t w_expert_bytes;  // bytes per expert
  int64_t s_expert_elems;  // scale elements per expert
  int N;                   // weight rows (2I for gate_up, H for down)
  int K;                   // inner dimension
  int I;                   // gate_up: rows [0, I) gate, [I, 2I) up; output width I
  const void* in;          // activations, row-major [rows, K], act dtype
  const int32_t* perm;     // gather: position -> pair, row = pair / topk; nullptr: row = position
  int topk;
  void* out;               // gate_up: h [pos, I] act dtype; down: y [pos, N] fp32
  const int32_t* tiles;    // [max_tiles][4] = expert, first position, rows, 0
  const int32_t* n_tiles;  // device scalar; nullptr: dense tiles over num_rows (expert 0)
  int num_rows;
  int act_bf16;
  const float* xsum;       // prefill, int formats: group sums of the input rows [rows, K/128]
  float* hsum;             // prefill gate_up: group sums of the stored h [positions, I/128]
  const int32_t* tile_src; // decode gate_up: [max_tiles][kTileSrcCols] input row of each tile column
  int out_cols;            // decode down, > 0: store bf16 [rows, out_cols] (columns < out_cols)
  int64_t in_bytes;        // extent of in: its rows x K x activation size
  // prefill int8 gate_up on the fp16 matrix cores: destination of the
  // power-of-two-scaled fp16 copy of in, and per input row 1 / scale
  uint16_t* in16;
  float* xinv;
  // down of the routed experts: output row of each position (its pair
  // t k + slot), so y comes out in pair order; nullptr: the position
  const int32_t* out_rows;
  // prefill down, compact y (y16 != nullptr, out unused): y16 [rows, N] fp16
  // by position, each 256-row slab of a position times a power of two whose
  // inverse goes to yscale [rows, N / 256]
  uint16_t* y16;
  float* yscale;
  // prefill int8 down, k_parts > 1: the K range in k_parts equal parts, each
  // (tile, slab) item once per part; part p's fp32 partial rows go to
  // out + p num_rows N, and the combine adds the parts in order
  int k_parts;
  // prefill int4, nonzero: a tile of at most 16 / 32 / 48 positions (an
  // expert's last or only one) runs a copy of the pipeline over the first
  // one / two / three of its four 16-position column tiles (set where experts
  // average at most 48 positions)
  int narrow_tiles;
  // single-token decode gate_up that routes its token itself
  // (route_logits != nullptr, [1, route_E] bf16): every workgroup runs K1
  // on the one row of logits, workgroup (0, 0) also writes K1's and K2's
  // outputs into the ro_* regions (ids, weights, counts, offsets, perm, inv,
  // ro_max_tiles tile records and their source rows, the tile count)
  const void* route_logits;
  int route_E;
  unsigned route_flags;
  int ro_max_tiles;
  int32_t* ro_ids;
  float* ro_w;
  int32_t* ro_counts;
  int32_t* ro_offsets;
  int32_t* ro_perm;
  int32_t* ro_inv;
  int32_t* ro_tiles;
  int32_t* ro_n_tiles;
  int32_t* ro_tile_src;
  float* ro_wpos;
  // decode gate_up of 2 .. kSrMaxTokens tokens that routes them itself
  // (launch_gemv_sr): route_T tokens of route_logits [route_T, route_E];
  // ro_resident (nullable) the experts' HBM residency, as K2 takes it
  int route_T;
  const uint8_t* ro_resident;
  // decode form with a shared expert of intermediate size sh_I =
  // sh_chunks x I (sh_chunks > 0): the shared expert rides in the routed
  // launches.  Chunk c is an expert of the routed shape cut from the shared
  // one: gate_up rows [cI, cI + I) of its gate and of its up projection
  // (output columns [cI, cI + I) of the shared h), down the K range
  // [cI, cI + I) of its down projection (input the same shared h columns).
  // Tile sh_tile0 + c * nT + j (nT = ceil(sh_tokens / 16)) is chunk c on
  // tokens 16 j .. 16 j + 15, read in place.  sh_w / sh_scales: the shared
  // slot of this phase.  gate_up: the token tiles of chunk 0 also write
  // sigmoid(x . sh_gate_w) to sh_gate (K4); down: chunk c's rows go to
  // sh_y + c sh_tokens H (fp32 [sh_tokens, H]), which the combine adds in
  // chunk order.  The down + combine launch (up to kDcMaxTokens tokens)
  // takes the chunks as more items of each token instead.
  int sh_chunks;
  int sh_I;
  int sh_tile0;
  int sh_tokens;
  const uint8_t* sh_w;
  const uint16_t* sh_scales;
  void* sh_h;  // bf16 [sh_tokens, sh_I]
  const void* sh_gate_w;
  float* sh_gate;
  float* sh_y;
};

// most chunks of a shared expert in the routed decode launches
constexpr int kMaxSharedChunks = 8;

enum GemmPhase : int { PHASE_GATE_UP = 0, PHASE_DOWN = 1 };

// Optional pair of events stamped by the dispatch itself at a kernel's start
// and end (hipExtLaunchKernelGGL): the kernel's own duration, no launch gap.
struct KernelTimer {
  hipEvent_t start, stop;
};

template <typename Kernel, typename... Args>
inline void launch_timed(Kernel kernel, dim3 grid, dim3 block, uint32_t lds, hipStream_t stream,
                         const KernelTimer* tm, Args... args) {
  if (tm)
    hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, tm->start, tm->stop, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
}

// positions per tile of the prefill form of K3
constexpr int kPrefillTileM = 64;
// positions per tile of the decode form; K2 then also writes, per tile, the
// input row of each of its kTileSrcCols columns (0 past the tile's rows)
constexpr int kTileSrcCols = 16;

hipError_t launch_route(const void* logits, int act_bf16, int T, int E, int k, unsigned flags,
                        int32_t* ids, float* w, hipStream_t stream);

// K1 + K2 in one workgroup when route_group_fused(T, k).  resident (nullable,
// [E] device bytes): experts with 0 are grouped but get no GEMM tiles.
// wpos (nullable, [T k]): the routing weight of each position (pair perm[pos]).
bool route_group_fused(int T, int k);
hipError_t launch_route_group(const void* logits, int act_bf16, int T, int E, int k,
                              unsigned flags, int bm, int max_tiles, int32_t* ids, float* w,
                              int32_t* counts, int32_t* offsets, int32_t* perm, int32_t* inv,
                              int32_t* tiles, int32_t* n_tiles, int32_t* tile_src,
                              const uint8_t* resident, float* wpos, hipStream_t stream);

// Router (optional) + K1 + K2 as one launch of several workgroups that hand
// their results on without waiting (route_spread_ok(T, k, E, H, gemv)).
// x == nullptr: routing of the given logits_in [T, E] (act dtype).  Else the
// router GEMV first, logits [T, E] bf16 = x . gate^T written to logits_out
// (gate_packed: the router weight in the bf16 block layout, rows padded to
// 32), with norm_w != nullptr x RMS-normalised first (bf16 weight [H], eps;
// the normalised rows written to normed).  sync: the workspace's status words
// (the counters use words 0 .. 16, zero before and after every call); masks:
// T x 8 words of the sync area (zero before and after).  The remaining
// outputs are launch_route_group's.
bool route_spread_ok(int T, int k, int E, int H, bool gemv);
hipError_t launch_route_spread(const void* logits_in, int act_bf16, const void* x, const void* gate_packed,
                               const void* norm_w, float eps, void* normed, int H, int T, int E, int k,
                               unsigned flags, int bm, int max_tiles, void* logits_out, uint32_t* sync,
                               uint32_t* masks, int32_t* ids, float* w, int32_t* counts, int32_t* offsets,
                               int32_t* perm, int32_t* inv, int32_t* tiles, int32_t* n_tiles, int32_t* tile_src,
                               const uint8_t* resident, float* wpos, hipStream_t stream, bool gemv_only = false);

// K2 over many workgroups (large batches): hist holds group_hist_blocks(T*k) x E int32.
int group_hist_blocks(int P);
hipError_t launch_group_multi(const int32_t* ids, int T, int k, int E, int bm, int max_tiles, int32_t* hist,
                              int32_t* counts, int32_t* offsets, int32_t* perm, int32_t* inv, int32_t* tiles,
                              int32_t* n_tiles, int32_t* tile_src, const uint8_t* resident,
                              hipStream_t stream);

// K2 from given routing: ids_in int64 [T, k] and w_in fp32 [T, k] (the
// caller's top-k), sanitised into ids / w (a slot with an id outside [0, E)
// or repeating an earlier slot's id of its token is dropped: it takes the
// smallest unused id with weight 0, and *status becomes 1), then grouped as
// launch_route_group / launch_group_multi group K1's output (one launch when
// route_group_fused(T, k), else three; hist as for launch_group_multi).
hipError_t launch_given_group(const int64_t* ids_in, const float* w_in, int T, int E, int k, int bm, int max_tiles,
                              int32_t* hist, int32_t* ids, float* w, int32_t* counts, int32_t* offsets, int32_t* perm,
                              int32_t* inv, int32_t* tiles, int32_t* n_tiles, int32_t* tile_src,
                              const uint8_t* resident, float* wpos, uint32_t* status, hipStream_t stream);

// Tokens per expert up to which the decode form runs (by weight format, the
// experts' intermediate size I and whether the layer has a shared expert).
double decode_form_max_avg(int wf, int I, bool shared);

// Tile shapes: returns the token-tile height (BM) used for num_tokens:
// 16 for decode-sized expert groups (gemv form), else kPrefillTileM when
// the prefill form takes the shape (prefill_form), else 32 / 64 (the tiled
// form that also serves fp32 weights).
int gemm_tile_m(int num_tokens, int topk, int num_experts, int wf, bool prefill_form, int I, bool shared);

// Rows of weights (gate_up: output columns of h) covered by one workgroup.
int gemm_rows_per_block(int wf, int phase, int bm);

hipError_t launch_gemm(const GemmArgs& a, int wf, int phase, int bm, int grid_tiles,
                       hipStream_t stream, const KernelTimer* tm = nullptr);

// Decode form of K3 (tiles of at most 16 positions, split-K in a workgroup).
bool gemv_supported(int wf, int phase, int N, int K, int I);
hipError_t launch_gemv(const GemmArgs& a, int wf, int phase, int max_tiles, hipStream_t stream,
                       const KernelTimer* tm = nullptr);

// Workgroups of a decode-form launch (gemv_supported shapes; the down
// launch at its two-tile row sets).
int64_t gemv_workgroups(int wf, int phase, int N, int K, int I, int max_tiles);

// Decode gate_up that routes its own tokens (given bf16 logits, 2 ..
// kSrMaxTokens tokens, so every expert's tokens make one tile): one launch does
// K1 + K2 (one workgroup, writing the ro_* outputs as the routing kernels
// do) and the gate_up GEMV, whose workgroups each find the experts' token
// sets from the logits themselves.  gemv_sr_supported says which shapes it
// takes; lanes: workgroups per row set block sharing the active experts
// (0: the library's choice).
constexpr int kSrMaxTokens = 4;
bool gemv_sr_supported(int wf, int N, int K, int I, int T, int E, int k);
hipError_t launch_gemv_sr(const GemmArgs& a, int wf, int lanes, hipStream_t stream, const KernelTimer* tm = nullptr);

// The combine's inputs beyond y for the down + combine kernel of T tokens:
// routing weights w, expert ids and pair positions inv [T, k] (written by
// K1 / K2), the gated shared expert (y_shared [T, H] fp32 and its gate [T],
// nullable), residual [T, H] (act dtype, nullable), out [T, H] bf16.
struct CombineTail {
  const float* w;       // routing weights [T, k]
  const int32_t* ids;   // expert ids [T, k]
  const int32_t* inv;   // position (h row) of each pair [T, k]
  const float* y_shared;
  const float* shared_gate;
  const void* residual;
  void* out;
  int tokens;  // T
};

// most tokens of the down GEMV + combine launch
constexpr int kDcMaxTokens = 4;

// Down GEMV + combine in one launch for up to kDcMaxTokens tokens (n_pos =
// k pairs per token, h rows by position, bf16).
bool down_combine_supported(int wf, int N, int K, int I, int n_pos);
hipError_t launch_down_combine(const GemmArgs& a, const CombineTail& c, int wf, int n_pos, hipStream_t stream);

// Prefill form of K3 (tiles of 64 positions, bf16 / int8 / int4 weights).
bool gemm2_supported(int wf, int phase, int N, int K, int I);
hipError_t launch_gemm2(const GemmArgs& a, int wf, int phase, int max_tiles, hipStream_t stream,
                        const KernelTimer* tm = nullptr);
// fp32 sums of every 128-wide K group of the rows of a bf16 matrix [rows, K]
hipError_t launch_group_sums(const void* x, int rows, int K, float* out, hipStream_t stream);
// the same sums, plus the fp16 copy of each row scaled by a power of two
// (x16, same layout) and 1 / scale per row (xinv); K <= 4096
hipError_t launch_prep_f16(const void* x, int rows, int K, float* sums, uint16_t* x16, float* xinv,
                           hipStream_t stream);
// K1 for T tokens (bf16 logits, as launch_route) and launch_prep_f16 of
// rows rows of x in one launch.
hipError_t launch_route_prep_f16(const void* logits, int T, int E, int k, unsigned flags, int32_t* ids, float* w,
                                 const void* x, int rows, int K, float* sums, uint16_t* x16, float* xinv,
                                 hipStream_t stream);
// whether launch_gemm2 runs a on the int8 pipeline kernel (which then takes
// gate_up's input as the fp16 copy when a.xinv is set)
bool gemm2_i8_pipeline(const GemmArgs& a, int wf);
// whether launch_gemm2 runs a on the int4 pipeline kernel
bool gemm2_i4_pipeline(const GemmArgs& a, int wf);

// Repack [N, K] into the block layout; rows >= n_valid (bf16 only) are zero
// and not read (n_valid < 0: all N rows).
hipError_t launch_pack(int wf, const void* src, const void* src_scales, int N, int K,
                       uint8_t* dst, uint16_t* dst_scales, hipStream_t stream, int n_valid = -1);

hipError_t launch_shared_gate(const void* x, const void* gate_w, int act_bf16, int T, int H,
                              float* gate_out, hipStream_t stream);

// y: the k expert rows of token t at rows t k .. t k + k - 1 (pair order,
// inv == nullptr) or at rows inv[t k + j] (position order); y16 != nullptr:
// the rows are the prefill down's compact y (fp16 + yscale), y unused.
// sh_rows > 1 (fp32 y only): the shared expert's row of token t is the sum
// of y_shared rows j T + t, j < sh_rows, added in order (its chunks).
hipError_t launch_combine(const float* y, const int32_t* ids, const float* w, const int32_t* inv, const float* y_shared,
                          const float* shared_gate, const uint8_t* resident, const void* extra, const void* residual,
                          int T, int k, int H, void* out, int out_bf16, hipStream_t stream,
                          const uint16_t* y16 = nullptr, const float* yscale = nullptr, int sh_rows = 1);

// bf16 RMSNorm rows of x [T, H] with weight w [H] (decoder-block form)
hipError_t launch_rmsnorm(const void* x, const void* w, float eps, int T, int H, void* out, hipStream_t stream);

}  // namespace nkt
