// C ABI of the MoE expert path (declared in include/nkt_moe.h).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <new>

#include "../../include/nkt_moe.h"
#include "nkt_common.h"
#include "nkt_internal.h"

namespace {

using namespace nkt;

struct Handle {
  int E, k, H, I, Is, wf, act_bf16;
  unsigned flags;
  int max_tokens;
  const void* w[NKT_NUM_SLOTS];
  const uint8_t* resident;  // [E] device bytes, 0 = expert not in HBM; nullptr = all resident
  // the shared expert's side stream (default priority) and its fork / join
  // events, made on the first layer call outside graph capture
  hipStream_t side = nullptr;
  hipEvent_t fork_ev = nullptr, join_ev = nullptr;
  int side_device = -1;
  std::mutex side_mu;  // one fork / join in flight per handle
  ~Handle() {
    if (fork_ev) (void)hipEventDestroy(fork_ev);
    if (join_ev) (void)hipEventDestroy(join_ev);
    if (side) (void)hipStreamDestroy(side);
  }
};

constexpr int kWsTiles = NKT_WS_NUM_REGIONS;       // int32 [max_tiles][4]
constexpr int kWsNTiles = NKT_WS_NUM_REGIONS + 1;  // int32 [1]
constexpr int kWsXsum = NKT_WS_NUM_REGIONS + 2;    // fp32 [T, H/128]   group sums of x (prefill form)
constexpr int kWsHsum = NKT_WS_NUM_REGIONS + 3;    // fp32 [T*k, I/128] group sums of h
constexpr int kWsShHsum = NKT_WS_NUM_REGIONS + 4;  // fp32 [T, I_s/128] group sums of the shared h
constexpr int kWsHist = NKT_WS_NUM_REGIONS + 5;   // int32 [blocks, E] per-block expert histograms
constexpr int kWsTileSrc = NKT_WS_NUM_REGIONS + 6; // int32 [max_tiles, 16] decode tiles' input rows
constexpr int kWsX16 = NKT_WS_NUM_REGIONS + 7;     // fp16 [T, H] scaled copy of x (int8 prefill gate_up)
constexpr int kWsXInv = NKT_WS_NUM_REGIONS + 8;    // fp32 [T] 1 / scale of each row of that copy
constexpr int kWsTagged = NKT_WS_NUM_REGIONS + 9; // u32 [T, 8] the single-launch router's published selection masks
constexpr int kWsWpos = NKT_WS_NUM_REGIONS + 10;  // fp32 [T k] routing weights by position (fused route + group)
constexpr int kWsShChunkY = NKT_WS_NUM_REGIONS + 11;  // fp32 [Is / I, T, H] the shared expert's chunk rows
constexpr int kWsAll = NKT_WS_NUM_REGIONS + 12;

void set_err(char* err, size_t len, const char* fmt, ...) {
  if (!err || len == 0) return;
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(err, len, fmt, ap);
  va_end(ap);
}

int bytes_per_weight_x2(int wf) {  // bytes per weight, times two
  return wf == WF_F32 ? 8 : wf == WF_BF16 ? 4 : wf == WF_I8 ? 2 : 1;
}

// rows / cols of the projection in a slot
bool slot_shape(const Handle* h, int slot, int* N, int* K, int* experts) {
  switch (slot) {
    case NKT_SLOT_GATE_UP:
    case NKT_SLOT_GATE_UP_SCALES:
      *N = 2 * h->I, *K = h->H, *experts = h->E;
      return true;
    case NKT_SLOT_DOWN:
    case NKT_SLOT_DOWN_SCALES:
      *N = h->H, *K = h->I, *experts = h->E;
      return true;
    case NKT_SLOT_SHARED_GATE_UP:
    case NKT_SLOT_SHARED_GATE_UP_SCALES:
      *N = 2 * h->Is, *K = h->H, *experts = 1;
      return h->Is > 0;
    case NKT_SLOT_SHARED_DOWN:
    case NKT_SLOT_SHARED_DOWN_SCALES:
      *N = h->H, *K = h->Is, *experts = 1;
      return h->Is > 0;
    default:
      return false;
  }
}

bool is_scale_slot(int slot) {
  return slot == NKT_SLOT_GATE_UP_SCALES || slot == NKT_SLOT_DOWN_SCALES ||
         slot == NKT_SLOT_SHARED_GATE_UP_SCALES || slot == NKT_SLOT_SHARED_DOWN_SCALES;
}

int64_t code_bytes(const Handle* h, int N, int K) {
  return (int64_t)N * K * bytes_per_weight_x2(h->wf) / 2;
}

int64_t scale_elems(const Handle* h, int N, int K) {
  if (h->wf == WF_I4) return (int64_t)N * (K / 128);
  if (h->wf == WF_I8) return N;
  return 0;
}

// router gate rows, padded for the decode GEMM's 32-row sets
int router_rows(const Handle* h) { return (h->E + 31) / 32 * 32; }

size_t slot_bytes(const Handle* h, int slot) {
  if (slot == NKT_SLOT_SHARED_GATE) return h->Is > 0 ? (size_t)h->H * (h->act_bf16 ? 2 : 4) : 0;
  if (slot == NKT_SLOT_ROUTER) return h->act_bf16 ? (size_t)router_rows(h) * h->H * 2 : 0;
  int N, K, ne;
  if (!slot_shape(h, slot, &N, &K, &ne)) return 0;
  if (is_scale_slot(slot)) return (size_t)ne * scale_elems(h, N, K) * 2;
  return (size_t)ne * code_bytes(h, N, K);
}

struct WsLayout {
  size_t off[kWsAll];
  size_t total;
  int bm;
  int bm_shared;
  int max_tiles;
};

constexpr int kSharedDecodeMaxTokens = 256;

// NKT_WS_Y row order: pair (t k + slot) for the decode form, else position
bool y_pair_order(const WsLayout& L) { return L.bm == kTileSrcCols; }

// the prefill form covers both projections of the routed (or shared) experts
bool prefill_form_ok(const Handle* h, bool shared) {
  const int I = shared ? h->Is : h->I;
  return gemm2_supported(h->wf, PHASE_GATE_UP, 2 * I, h->H, I) &&
         gemm2_supported(h->wf, PHASE_DOWN, h->H, I, I);
}

size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

// Sync area sizes: 32 words (the single-launch router's counters, the status
// word; padded), then the router's mask area (64 KiB, of which it uses
// T x 8 words: the published size of the area is kept).
constexpr size_t kSyncStatusBytes = 256;
constexpr size_t kSyncTaggedBytes = (size_t)kFusedRouteMaxTokens * kMaxExperts * 4;
static_assert(kSyncStatusBytes + kSyncTaggedBytes == NKT_SYNC_AREA_BYTES, "the sync area's published size");

// Chunks of the shared expert that ride in the routed experts' launches
// when both run in the decode form: Is / I of the routed shape (Qwen1.5-MoE:
// 5632 / 1408 = 4), each one more expert of every tile of 16 tokens, the
// shared gate from gate_up and the chunk rows added by the combine; 0 (the
// shared expert keeps launches of its own) without a shared expert, with Is
// not a multiple of I, more than kMaxSharedChunks chunks or fp32
// activations.
int shared_chunk_count(const Handle* h, const WsLayout& L) {
  if (h->Is <= 0 || h->Is % h->I != 0 || !h->act_bf16) return 0;
  if (L.bm != kTileSrcCols || L.bm_shared != kTileSrcCols) return 0;
  const int c = h->Is / h->I;
  return c <= kMaxSharedChunks ? c : 0;
}

// K parts of the shared expert's prefill-form int8 down in the layer call:
// the smallest count that leaves at most 16 K groups per part (Qwen1.5-MoE:
// 44 groups -> 4 parts of 11), so each (token tile, weight slab) item runs
// K / parts deep (5632: 88 stages of 64 -> 22) on parts times the
// workgroups; the combine adds the parts' fp32 rows in order.  Only while
// the undivided down has at most kSharedPartsMaxItems items: beside the
// routed experts on the side stream, a small grid of deep items ends last
// and the parts pay; a larger one already fills what the routed launches
// leave, and parts then only compete with them.  Measured (Qwen1.5-MoE int8,
// graph replays, us per layer, one part -> parts): T = 320 / 512 / 640 / 768
// 165 / 181 / 189 / 208 -> 157 / 172 / 184 / 198, T = 896 (112 items) 224
// either way, T = 1024 236 -> 248; the parts on the caller's stream after
// the routed experts instead: T = 512 / 1024 191 / 261.  1 (one part) when
// the K groups admit no such count, for other weight formats and for the
// decode form.
constexpr int kSharedPartsMaxItems = 96;

int shared_down_parts(const Handle* h, const WsLayout& L, int T) {
  if (h->Is <= 0 || h->wf != WF_I8 || L.bm_shared != kPrefillTileM || h->Is % 128 != 0 || h->H % 256 != 0) return 1;
  if ((int64_t)(h->H / 256) * ((T + kPrefillTileM - 1) / kPrefillTileM) > kSharedPartsMaxItems) return 1;
  const int G = h->Is / 128;
  if (G <= 16) return 1;
  for (int p = 2; p <= kMaxSharedChunks; ++p)
    if (G % p == 0 && G / p <= 16) return p;
  return 1;
}

// int8 weights with bf16 activations: the prefill gate_up runs on the fp16
// matrix cores from a power-of-two-scaled fp16 copy of x (H <= 4096)
bool int8_f16_input(const Handle* h) { return h->wf == WF_I8 && h->act_bf16 && h->H <= 4096; }

WsLayout ws_layout(const Handle* h, int T) {
  WsLayout L;
  const size_t P = (size_t)T * h->k;
  const size_t es = h->act_bf16 ? 2 : 4;
  L.bm = gemm_tile_m(T > 0 ? T : 1, h->k, h->E, h->wf, prefill_form_ok(h, false), h->I, h->Is > 0);
  // the shared expert takes every token as one group.  While the routed
  // experts run in the decode form it does too (riding in their launches as
  // chunk tiles where it can); once they run in the prefill form, its own
  // prefill-form launches fork beside theirs on the side stream, which
  // measured faster at every such T (Qwen1.5-MoE int8 T = 96 / 128 / 192 /
  // 256 146 / 150 / 169 / 190 -> 129 / 133 / 137 / 138 us per layer), while
  // inside the decode range the chunk tiles win (T = 48 / 64 121 / 132
  // against 140 / 147).  Without the int8 / int4 prefill pipelines the
  // decode form's split-K grid keeps it up to kSharedDecodeMaxTokens.
  const bool shared_prefill = (h->wf == WF_I8 || h->wf == WF_I4) && prefill_form_ok(h, true) && L.bm != kTileSrcCols;
  L.bm_shared = (T <= kSharedDecodeMaxTokens && h->Is > 0 && !shared_prefill &&
                 gemv_supported(h->wf, PHASE_GATE_UP, 2 * h->Is, h->H, h->Is) &&
                 gemv_supported(h->wf, PHASE_DOWN, h->H, h->Is, h->Is))
                    ? 16
                    : gemm_tile_m(T > 0 ? T : 1, 1, 1, h->wf, prefill_form_ok(h, true), h->Is, false);
  L.max_tiles = (int)(P / L.bm) + (int)(P < (size_t)h->E ? P : (size_t)h->E);
  size_t sz[kWsAll];
  sz[NKT_WS_TOPK_IDS] = P * 4;
  sz[NKT_WS_TOPK_WEIGHTS] = P * 4;
  sz[NKT_WS_COUNTS] = (size_t)h->E * 4;
  sz[NKT_WS_OFFSETS] = (size_t)(h->E + 1) * 4;
  sz[NKT_WS_PERM] = P * 4;
  sz[NKT_WS_INV] = P * 4;
  sz[NKT_WS_H] = P * h->I * es;
  sz[NKT_WS_Y] = P * h->H * 4;
  sz[NKT_WS_SHARED_GATE] = h->Is > 0 ? (size_t)T * 4 : 0;
  sz[NKT_WS_SHARED_H] = h->Is > 0 ? (size_t)T * h->Is * es : 0;
  sz[NKT_WS_SHARED_Y] = h->Is > 0 ? (size_t)T * h->H * 4 : 0;
  sz[NKT_WS_ROUTER_LOGITS] = h->act_bf16 ? (size_t)T * h->E * 2 : 0;
  sz[NKT_WS_NORMED] = h->act_bf16 ? (size_t)T * h->H * 2 : 0;
  sz[kWsTiles] = (size_t)L.max_tiles * 16;
  sz[kWsNTiles] = 4;
  sz[kWsXsum] = (size_t)T * (h->H / 128) * 4;
  sz[kWsHsum] = P * (h->I / 128) * 4;
  sz[kWsShHsum] = h->Is > 0 ? (size_t)T * (h->Is / 128) * 4 : 0;
  sz[kWsHist] = (size_t)group_hist_blocks((int)P) * h->E * 4;
  sz[kWsTileSrc] = L.bm == kTileSrcCols ? (size_t)L.max_tiles * kTileSrcCols * 4 : 0;
  const bool x16 = int8_f16_input(h);
  sz[kWsX16] = x16 ? (size_t)T * h->H * 2 : 0;
  sz[kWsXInv] = x16 ? (size_t)T * 4 : 0;
  sz[kWsWpos] = P * 4;
  const int parts = shared_down_parts(h, L, T);
  const int sh_rows = parts > 1 ? parts : shared_chunk_count(h, L);  // the two never apply together
  sz[kWsShChunkY] = (size_t)sh_rows * T * h->H * 4;
  // The sync area first, the same size and place for every handle and
  // token count (counters and status, the router's published masks): it must be
  // zero before a workspace's first use, every call of every handle leaves
  // it zero, and so no region's old contents -- of this handle or of another
  // sharing the workspace -- ever land there.
  sz[NKT_WS_SYNC] = kSyncStatusBytes;
  sz[kWsTagged] = kSyncTaggedBytes;
  size_t o = 0;
  for (int i : {(int)NKT_WS_SYNC, kWsTagged}) {
    L.off[i] = o;
    o += align_up(sz[i]);
  }
  for (int i = 0; i < kWsAll; ++i) {
    if (i == NKT_WS_SYNC || i == kWsTagged) continue;
    L.off[i] = o;
    o += align_up(sz[i]);
  }
  L.total = o;
  return L;
}

bool check_hip(hipError_t e, const char* what, char* err, size_t len) {
  if (e == hipSuccess) return true;
  set_err(err, len, "%s: %s", what, hipGetErrorString(e));
  return false;
}

bool check_call(Handle* h, int T, void* ws, size_t ws_bytes, char* err, size_t len) {
  if (!h) {
    set_err(err, len, "null handle");
    return false;
  }
  if (T < 0 || T > h->max_tokens) {
    set_err(err, len, "num_tokens=%d outside [0, max_tokens=%d]", T, h->max_tokens);
    return false;
  }
  const WsLayout L = ws_layout(h, T);
  if (T > 0 && (!ws || ws_bytes < L.total)) {
    set_err(err, len, "workspace too small: need %zu bytes, got %zu", L.total, ws_bytes);
    return false;
  }
  return true;
}

bool check_weights(const Handle* h, bool shared, char* err, size_t len) {
  const int need[] = {NKT_SLOT_GATE_UP, NKT_SLOT_DOWN};
  for (int s : need)
    if (!h->w[s]) {
      set_err(err, len, "weight slot %d not bound", s);
      return false;
    }
  if (h->wf == WF_I4 || h->wf == WF_I8) {
    if (!h->w[NKT_SLOT_GATE_UP_SCALES] || !h->w[NKT_SLOT_DOWN_SCALES]) {
      set_err(err, len, "scale slots not bound");
      return false;
    }
  }
  if (shared) {
    if (!h->w[NKT_SLOT_SHARED_GATE_UP] || !h->w[NKT_SLOT_SHARED_DOWN] || !h->w[NKT_SLOT_SHARED_GATE]) {
      set_err(err, len, "shared expert slots not bound");
      return false;
    }
    if ((h->wf == WF_I4 || h->wf == WF_I8) &&
        (!h->w[NKT_SLOT_SHARED_GATE_UP_SCALES] || !h->w[NKT_SLOT_SHARED_DOWN_SCALES])) {
      set_err(err, len, "shared expert scale slots not bound");
      return false;
    }
  }
  return true;
}

template <typename T>
T* ws_ptr(void* ws, const WsLayout& L, int region) {
  return (T*)((uint8_t*)ws + L.off[region]);
}

GemmArgs expert_args(const Handle* h, int phase, bool shared, const void* in, void* ws,
                     const WsLayout& L, int T) {
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  const int I = shared ? h->Is : h->I;
  const int N = phase == PHASE_GATE_UP ? 2 * I : h->H;
  const int K = phase == PHASE_GATE_UP ? h->H : I;
  const int slot = shared ? (phase == PHASE_GATE_UP ? NKT_SLOT_SHARED_GATE_UP : NKT_SLOT_SHARED_DOWN)
                          : (phase == PHASE_GATE_UP ? NKT_SLOT_GATE_UP : NKT_SLOT_DOWN);
  a.w = (const uint8_t*)h->w[slot];
  a.scales = (const uint16_t*)h->w[slot + 1];
  a.w_expert_bytes = code_bytes(h, N, K);
  a.s_expert_elems = scale_elems(h, N, K);
  a.N = N;
  a.K = K;
  a.I = I;
  a.in = in;
  a.topk = h->k;
  a.act_bf16 = h->act_bf16;
  float* hs = ws_ptr<float>(ws, L, shared ? kWsShHsum : kWsHsum);
  a.xsum = phase == PHASE_GATE_UP ? ws_ptr<float>(ws, L, kWsXsum) : hs;
  a.hsum = phase == PHASE_GATE_UP ? hs : nullptr;
  if (shared) {
    a.perm = nullptr;
    a.out = phase == PHASE_GATE_UP ? ws_ptr<void>(ws, L, NKT_WS_SHARED_H) : ws_ptr<void>(ws, L, NKT_WS_SHARED_Y);
    a.tiles = nullptr;
    a.n_tiles = nullptr;
    a.num_rows = T;
  } else {
    a.perm = phase == PHASE_GATE_UP ? ws_ptr<int32_t>(ws, L, NKT_WS_PERM) : nullptr;
    a.out = phase == PHASE_GATE_UP ? ws_ptr<void>(ws, L, NKT_WS_H) : ws_ptr<void>(ws, L, NKT_WS_Y);
    a.tiles = ws_ptr<int32_t>(ws, L, kWsTiles);
    a.n_tiles = ws_ptr<int32_t>(ws, L, kWsNTiles);
    a.num_rows = T * h->k;
    if (phase == PHASE_GATE_UP && L.bm == kTileSrcCols) a.tile_src = ws_ptr<int32_t>(ws, L, kWsTileSrc);
    a.narrow_tiles = (int64_t)T * h->k <= 48 * (int64_t)h->E;
  }
  const int64_t in_rows = (!shared && phase == PHASE_GATE_UP) ? T : a.num_rows;
  a.in_bytes = in_rows * K * (h->act_bf16 ? 2 : 4);
  // the decode form writes y in pair order (the combine then issues all its
  // loads at once); the prefill form keeps position order (contiguous rows)
  if (!shared && phase == PHASE_DOWN && y_pair_order(L)) a.out_rows = ws_ptr<int32_t>(ws, L, NKT_WS_PERM);
  if (phase == PHASE_GATE_UP && int8_f16_input(h)) {
    a.in16 = ws_ptr<uint16_t>(ws, L, kWsX16);
    a.xinv = ws_ptr<float>(ws, L, kWsXInv);
  }
  return a;
}

constexpr int kSpreadMinTokens = 16;

// prep (nullable): the int8 gate_up's fp16 input to make in the routing
// launch when routing takes the large-batch path (*prep_done says whether it
// did); prep_first: take that path for any T (a shared expert then forks
// beside the routed experts as soon as the copy exists)
int do_route(Handle* h, const void* logits, int T, void* ws, const WsLayout& L, hipStream_t st,
             char* err, size_t len, const GemmArgs* prep = nullptr, bool* prep_done = nullptr,
             bool prep_first = false) {
  if (prep_done) *prep_done = false;
  if (!logits) {
    set_err(err, len, "null router_logits");
    return NKT_ERR;
  }
  int32_t* ids = ws_ptr<int32_t>(ws, L, NKT_WS_TOPK_IDS);
  float* wts = ws_ptr<float>(ws, L, NKT_WS_TOPK_WEIGHTS);
  int32_t* counts = ws_ptr<int32_t>(ws, L, NKT_WS_COUNTS);
  int32_t* offsets = ws_ptr<int32_t>(ws, L, NKT_WS_OFFSETS);
  int32_t* perm = ws_ptr<int32_t>(ws, L, NKT_WS_PERM);
  int32_t* inv = ws_ptr<int32_t>(ws, L, NKT_WS_INV);
  int32_t* tiles = ws_ptr<int32_t>(ws, L, kWsTiles);
  int32_t* n_tiles = ws_ptr<int32_t>(ws, L, kWsNTiles);
  int32_t* tile_src = L.bm == kTileSrcCols ? ws_ptr<int32_t>(ws, L, kWsTileSrc) : nullptr;
  // more than 16 tokens: K1 on one wave per token over several workgroups,
  // the last to finish groups (Qwen3 int4 T = 64: 90 -> 83 us per layer);
  // up to 16 the one-workgroup route + group is as fast (measured T = 8 / 16)
  const bool small_paths = !(prep && prep_first && h->act_bf16);
  if (small_paths && T > kSpreadMinTokens && route_spread_ok(T, h->k, h->E, h->H, false)) {
    if (!check_hip(launch_route_spread(logits, h->act_bf16, nullptr, nullptr, nullptr, 0.f, nullptr, h->H, T, h->E,
                                       h->k, h->flags, L.bm, L.max_tiles, nullptr, ws_ptr<uint32_t>(ws, L, NKT_WS_SYNC),
                                       ws_ptr<uint32_t>(ws, L, kWsTagged), ids, wts, counts, offsets, perm, inv, tiles,
                                       n_tiles, tile_src, h->resident, ws_ptr<float>(ws, L, kWsWpos), st),
                   "route + group kernel", err, len))
      return NKT_ERR;
    return NKT_OK;
  }
  if (small_paths && route_group_fused(T, h->k)) {
    if (!check_hip(launch_route_group(logits, h->act_bf16, T, h->E, h->k, h->flags, L.bm, L.max_tiles,
                                      ids, wts, counts, offsets, perm, inv, tiles, n_tiles, tile_src,
                                      h->resident, ws_ptr<float>(ws, L, kWsWpos), st),
                   "route+group kernel", err, len))
      return NKT_ERR;
    return NKT_OK;
  }
  if (prep && h->act_bf16) {
    if (!check_hip(launch_route_prep_f16(logits, T, h->E, h->k, h->flags, ids, wts, prep->in, T, prep->K,
                                         const_cast<float*>(prep->xsum), prep->in16, prep->xinv, st),
                   "route + input kernel", err, len))
      return NKT_ERR;
    if (prep_done) *prep_done = true;
  } else if (!check_hip(launch_route(logits, h->act_bf16, T, h->E, h->k, h->flags, ids, wts, st),
                        "route kernel", err, len)) {
    return NKT_ERR;
  }
  if (!check_hip(launch_group_multi(ids, T, h->k, h->E, L.bm, L.max_tiles, ws_ptr<int32_t>(ws, L, kWsHist), counts,
                                    offsets, perm, inv, tiles, n_tiles, tile_src, h->resident, st),
                 "group kernels", err, len))
    return NKT_ERR;
  return NKT_OK;
}

// K2 from the caller's routing: topk_ids int64 [T, k], topk_weights fp32
// [T, k] (sanitised into NKT_WS_TOPK_IDS / NKT_WS_TOPK_WEIGHTS; a dropped
// slot sets status word NKT_STATUS_BAD_ROUTING)
int do_route_given(Handle* h, const int64_t* ids, const float* w, int T, void* ws, const WsLayout& L, hipStream_t st,
                   char* err, size_t len) {
  if (!ids || !w) {
    set_err(err, len, "null topk_ids or topk_weights");
    return NKT_ERR;
  }
  if (!check_hip(launch_given_group(ids, w, T, h->E, h->k, L.bm, L.max_tiles, ws_ptr<int32_t>(ws, L, kWsHist),
                                    ws_ptr<int32_t>(ws, L, NKT_WS_TOPK_IDS), ws_ptr<float>(ws, L, NKT_WS_TOPK_WEIGHTS),
                                    ws_ptr<int32_t>(ws, L, NKT_WS_COUNTS), ws_ptr<int32_t>(ws, L, NKT_WS_OFFSETS),
                                    ws_ptr<int32_t>(ws, L, NKT_WS_PERM), ws_ptr<int32_t>(ws, L, NKT_WS_INV),
                                    ws_ptr<int32_t>(ws, L, kWsTiles), ws_ptr<int32_t>(ws, L, kWsNTiles),
                                    L.bm == kTileSrcCols ? ws_ptr<int32_t>(ws, L, kWsTileSrc) : nullptr, h->resident,
                                    ws_ptr<float>(ws, L, kWsWpos),
                                    ws_ptr<uint32_t>(ws, L, NKT_WS_SYNC) + NKT_STATUS_BAD_ROUTING, st),
                 "given routing + group kernel", err, len))
    return NKT_ERR;
  return NKT_OK;
}

// Router GEMV (decode-form GEMM over dense 16-token tiles, bf16 gate rows)
// into the bf16 logits region, then K1 + K2 on those logits.
bool check_route_hidden(const Handle* h, const void* x, char* err, size_t len) {
  if (!x) {
    set_err(err, len, "null hidden_states");
    return false;
  }
  if (!h->act_bf16) {
    set_err(err, len, "the fused router needs bf16 activations");
    return false;
  }
  if (!h->w[NKT_SLOT_ROUTER]) {
    set_err(err, len, "router weight not bound (NKT_SLOT_ROUTER)");
    return false;
  }
  if (!gemv_supported(WF_BF16, PHASE_DOWN, router_rows(h), h->H, 0)) {
    set_err(err, len, "hidden size %d unsupported by the router GEMM", h->H);
    return false;
  }
  return true;
}

// norm_w (nullable): x is RMS-normalised first (bf16 weight [H], eps) into
// NKT_WS_NORMED, which then feeds the router GEMV -- inside the routing
// launch when it takes the batch, else by a launch of its own.
int do_route_hidden(Handle* h, const void* x, int T, void* ws, const WsLayout& L, hipStream_t st, char* err,
                    size_t len, const void* norm_w = nullptr, float eps = 0.f) {
  if (!check_route_hidden(h, x, err, len)) return NKT_ERR;
  void* normed = ws_ptr<void>(ws, L, NKT_WS_NORMED);
  if (route_spread_ok(T, h->k, h->E, h->H, true)) {
    if (!check_hip(launch_route_spread(nullptr, 1, x, h->w[NKT_SLOT_ROUTER], norm_w, eps, norm_w ? normed : nullptr,
                                       h->H, T, h->E, h->k, h->flags, L.bm, L.max_tiles,
                                       ws_ptr<void>(ws, L, NKT_WS_ROUTER_LOGITS), ws_ptr<uint32_t>(ws, L, NKT_WS_SYNC),
                                       ws_ptr<uint32_t>(ws, L, kWsTagged), ws_ptr<int32_t>(ws, L, NKT_WS_TOPK_IDS),
                                       ws_ptr<float>(ws, L, NKT_WS_TOPK_WEIGHTS), ws_ptr<int32_t>(ws, L, NKT_WS_COUNTS),
                                       ws_ptr<int32_t>(ws, L, NKT_WS_OFFSETS), ws_ptr<int32_t>(ws, L, NKT_WS_PERM),
                                       ws_ptr<int32_t>(ws, L, NKT_WS_INV), ws_ptr<int32_t>(ws, L, kWsTiles),
                                       ws_ptr<int32_t>(ws, L, kWsNTiles),
                                       L.bm == kTileSrcCols ? ws_ptr<int32_t>(ws, L, kWsTileSrc) : nullptr, h->resident,
                                       ws_ptr<float>(ws, L, kWsWpos), st),
                   norm_w ? "rmsnorm + router + route + group kernel" : "router + route + group kernel", err, len))
      return NKT_ERR;
    return NKT_OK;
  }
  if (norm_w) {
    if (!check_hip(launch_rmsnorm(x, norm_w, eps, T, h->H, normed, st), "rmsnorm kernel", err, len)) return NKT_ERR;
    x = normed;
  }
  const int Ep = router_rows(h);
  GemmArgs r;
  memset(&r, 0, sizeof(r));
  r.w = (const uint8_t*)h->w[NKT_SLOT_ROUTER];
  r.N = Ep;
  r.K = h->H;
  r.in = x;
  r.topk = 1;
  r.out = ws_ptr<void>(ws, L, NKT_WS_ROUTER_LOGITS);
  r.num_rows = T;
  r.act_bf16 = 1;
  r.out_cols = h->E;
  if (!check_hip(launch_gemv(r, WF_BF16, PHASE_DOWN, (T + 15) / 16, st), "router gemm", err, len)) return NKT_ERR;
  return do_route(h, ws_ptr<void>(ws, L, NKT_WS_ROUTER_LOGITS), T, ws, L, st, err, len);
}

// Batches of up to kLogitsFirstMaxTokens from hidden states: the router GEMV
// (with the decoder block's RMSNorm) as a launch of its own -- phase A of
// the single-launch router -- then the layer as from given logits (routing
// inside the gate_up launch for one token, the self-routing gate_up for 2 ..
// 4, the one-workgroup route + group launch up to 16).  Measured (Qwen3
// int4, graph replays, us per layer, single launch -> this): hidden states
// T = 1 / 2 / 4 / 8 / 16 22.7 / 26.6 / 36.7 / 46.7 / 58.6 -> 18.8 / 22.8 /
// 33.2 / 45.2 / 57.8, decoder block 26.7 / 31.4 / 40.9 / 51.1 / 63.5 ->
// 23.0 / 26.8 / 37.4 / 49.6 / 62.1; at T = 24 .. 64 within +-1 us either
// way (the decoder block up to 3 us slower), so the single launch stays there.
constexpr int kLogitsFirstMaxTokens = 16;

bool logits_first(const Handle* h, int T) {
  return T <= kLogitsFirstMaxTokens && route_spread_ok(T, h->k, h->E, h->H, true);
}

int do_router_logits(Handle* h, const void* x, int T, void* ws, const WsLayout& L, hipStream_t st, char* err,
                     size_t len, const void* norm_w = nullptr, float eps = 0.f) {
  if (!check_route_hidden(h, x, err, len)) return NKT_ERR;
  if (!check_hip(launch_route_spread(nullptr, 1, x, h->w[NKT_SLOT_ROUTER], norm_w, eps,
                                     norm_w ? ws_ptr<void>(ws, L, NKT_WS_NORMED) : nullptr, h->H, T, h->E, h->k,
                                     h->flags, L.bm, L.max_tiles, ws_ptr<void>(ws, L, NKT_WS_ROUTER_LOGITS), nullptr,
                                     nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                     nullptr, nullptr, nullptr, st, true),
                 norm_w ? "rmsnorm + router kernel" : "router kernel", err, len))
    return NKT_ERR;
  return NKT_OK;
}

// K3 launch for one projection: the decode form for tiles of at most 16
// positions, the prefill form for its tiles, the tiled form otherwise.
// The prefill form's gate_up first sums the activations per 128-wide group
// (int formats; the down projection reads the sums gate_up writes).
// prep_done: the int8 gate_up's fp16 input copy and group sums are already
// made (by the routing launch).
hipError_t launch_expert_gemm(const Handle* h, const GemmArgs& a, int phase, int bm, int tiles,
                              hipStream_t st, const KernelTimer* tm = nullptr, bool prep_done = false) {
  if (bm == 16 && gemv_supported(h->wf, phase, a.N, a.K, a.I)) return launch_gemv(a, h->wf, phase, tiles, st, tm);
  if (bm == kPrefillTileM && gemm2_supported(h->wf, phase, a.N, a.K, a.I)) {
    GemmArgs b = a;
    if (phase == PHASE_GATE_UP && (h->wf == WF_I4 || h->wf == WF_I8)) {
      const int rows_in = a.perm ? a.num_rows / a.topk : a.num_rows;
      hipError_t e;
      if (a.in16 && a.xinv && gemm2_i8_pipeline(a, h->wf)) {
        e = prep_done ? hipSuccess : launch_prep_f16(a.in, rows_in, a.K, const_cast<float*>(a.xsum), a.in16, a.xinv, st);
        b.in = a.in16;
      } else {
        e = launch_group_sums(a.in, rows_in, a.K, const_cast<float*>(a.xsum), st);
        b.xinv = nullptr;
      }
      if (e != hipSuccess) return e;
    }
    return launch_gemm2(b, h->wf, phase, tiles, st, tm);
  }
  return launch_gemm(a, h->wf, phase, bm, tiles, st, tm);
}

// The layer call's prefill form keeps y compact: fp16 by position with a
// power-of-two scale per 256-column slab, in the NKT_WS_Y region (the fp16
// rows first, then the fp32 inverse scales [T k, H / 256]) -- half the bytes
// down writes and the combine reads again; the combine still sums in fp32.
// The stage entry points keep NKT_WS_Y in fp32.
bool compact_y(const Handle* h, const WsLayout& L) {
  return L.bm == kPrefillTileM && prefill_form_ok(h, false) && h->H % 256 == 0;
}
uint16_t* y16_ptr(void* ws, const WsLayout& L) { return ws_ptr<uint16_t>(ws, L, NKT_WS_Y); }
float* yscale_ptr(const Handle* h, void* ws, const WsLayout& L, int T) {
  return (float*)(ws_ptr<uint8_t>(ws, L, NKT_WS_Y) + (size_t)T * h->k * h->H * 2);
}

// The shared expert's chunks in a routed launch of this phase
// (GemmArgs::sh_chunks): tiles from tile0 on; gate_up also writes the gate.
void set_shared_chunks(const Handle* h, GemmArgs& a, int phase, void* ws, const WsLayout& L, int T, int tile0,
                       int chunks) {
  const bool gu = phase == PHASE_GATE_UP;
  a.sh_chunks = chunks;
  a.sh_I = h->Is;
  a.sh_tile0 = tile0;
  a.sh_tokens = T;
  a.sh_w = (const uint8_t*)h->w[gu ? NKT_SLOT_SHARED_GATE_UP : NKT_SLOT_SHARED_DOWN];
  a.sh_scales = (const uint16_t*)h->w[(gu ? NKT_SLOT_SHARED_GATE_UP : NKT_SLOT_SHARED_DOWN) + 1];
  a.sh_h = ws_ptr<void>(ws, L, NKT_WS_SHARED_H);
  if (gu) {
    a.sh_gate_w = h->w[NKT_SLOT_SHARED_GATE];
    a.sh_gate = ws_ptr<float>(ws, L, NKT_WS_SHARED_GATE);
  } else {
    a.sh_y = ws_ptr<float>(ws, L, kWsShChunkY);
  }
}

// chunks > 0: the shared expert's chunks ride along (after the routed tiles)
int do_expert_phase(Handle* h, int phase, const void* x, int T, void* ws, const WsLayout& L,
                    hipStream_t st, char* err, size_t len, const KernelTimer* tm = nullptr, bool compact = false,
                    int chunks = 0, bool prep_done = false) {
  if (phase == PHASE_GATE_UP && !x) {
    set_err(err, len, "null hidden_states");
    return NKT_ERR;
  }
  if (!check_weights(h, chunks > 0, err, len)) return NKT_ERR;
  const int tiles = L.max_tiles + chunks * ((T + 15) / 16);
  if (phase == PHASE_GATE_UP) {
    GemmArgs a = expert_args(h, PHASE_GATE_UP, false, x, ws, L, T);
    if (chunks > 0) set_shared_chunks(h, a, PHASE_GATE_UP, ws, L, T, L.max_tiles, chunks);
    if (!check_hip(launch_expert_gemm(h, a, PHASE_GATE_UP, L.bm, tiles, st, tm, prep_done), "gate_up gemm", err, len))
      return NKT_ERR;
  } else {
    GemmArgs b = expert_args(h, PHASE_DOWN, false, ws_ptr<void>(ws, L, NKT_WS_H), ws, L, T);
    if (compact && compact_y(h, L)) {
      b.y16 = y16_ptr(ws, L);
      b.yscale = yscale_ptr(h, ws, L, T);
    }
    if (chunks > 0) set_shared_chunks(h, b, PHASE_DOWN, ws, L, T, L.max_tiles, chunks);
    if (!check_hip(launch_expert_gemm(h, b, PHASE_DOWN, L.bm, tiles, st, tm), "down gemm", err, len))
      return NKT_ERR;
  }
  return NKT_OK;
}

int do_experts(Handle* h, const void* x, int T, void* ws, const WsLayout& L, hipStream_t st,
               char* err, size_t len, bool compact = false, int chunks = 0, bool prep_done = false) {
  if (do_expert_phase(h, PHASE_GATE_UP, x, T, ws, L, st, err, len, nullptr, false, chunks, prep_done) != NKT_OK)
    return NKT_ERR;
  return do_expert_phase(h, PHASE_DOWN, x, T, ws, L, st, err, len, nullptr, compact, chunks);
}

// parts > 1 (the layer call, shared_down_parts): the down runs in K parts
// whose fp32 rows go to the chunk-row region for the combine to add
int do_shared(Handle* h, const void* x, int T, void* ws, const WsLayout& L, hipStream_t st,
              char* err, size_t len, bool prep_done = false, int parts = 1) {
  if (h->Is <= 0) {
    set_err(err, len, "handle has no shared expert");
    return NKT_ERR;
  }
  if (!x) {
    set_err(err, len, "null hidden_states");
    return NKT_ERR;
  }
  if (!check_weights(h, true, err, len)) return NKT_ERR;
  if (!check_hip(launch_shared_gate(x, h->w[NKT_SLOT_SHARED_GATE], h->act_bf16, T, h->H,
                                    ws_ptr<float>(ws, L, NKT_WS_SHARED_GATE), st),
                 "shared gate kernel", err, len))
    return NKT_ERR;
  const int bm = L.bm_shared;
  const int tiles = (T + bm - 1) / bm;
  GemmArgs a = expert_args(h, PHASE_GATE_UP, true, x, ws, L, T);
  if (!check_hip(launch_expert_gemm(h, a, PHASE_GATE_UP, bm, tiles, st, nullptr, prep_done), "shared gate_up gemm",
                 err, len))
    return NKT_ERR;
  GemmArgs b = expert_args(h, PHASE_DOWN, true, ws_ptr<void>(ws, L, NKT_WS_SHARED_H), ws, L, T);
  if (parts > 1) {
    b.k_parts = parts;
    b.out = ws_ptr<void>(ws, L, kWsShChunkY);
  }
  if (!check_hip(launch_expert_gemm(h, b, PHASE_DOWN, bm, tiles, st), "shared down gemm", err, len))
    return NKT_ERR;
  return NKT_OK;
}

// chunks > 0: the shared expert's row is the sum of its chunk rows
int do_combine(Handle* h, int T, void* out, void* ws, const WsLayout& L, hipStream_t st, char* err,
               size_t len, const void* extra = nullptr, const void* residual = nullptr, bool compact = false,
               int chunks = 0) {
  if (!out) {
    set_err(err, len, "null output");
    return NKT_ERR;
  }
  const bool sh = h->Is > 0;
  const bool y16 = compact && compact_y(h, L);
  const float* ysh = !sh ? nullptr : chunks > 0 ? ws_ptr<float>(ws, L, kWsShChunkY) : ws_ptr<float>(ws, L, NKT_WS_SHARED_Y);
  if (!check_hip(launch_combine(ws_ptr<float>(ws, L, NKT_WS_Y), ws_ptr<int32_t>(ws, L, NKT_WS_TOPK_IDS),
                                ws_ptr<float>(ws, L, NKT_WS_TOPK_WEIGHTS),
                                y_pair_order(L) ? nullptr : ws_ptr<int32_t>(ws, L, NKT_WS_INV), ysh,
                                sh ? ws_ptr<float>(ws, L, NKT_WS_SHARED_GATE) : nullptr, h->resident,
                                extra, residual, T, h->k, h->H, out, h->act_bf16, st,
                                y16 ? y16_ptr(ws, L) : nullptr, y16 ? yscale_ptr(h, ws, L, T) : nullptr,
                                chunks > 0 ? chunks : 1),
                 "combine kernel", err, len))
    return NKT_ERR;
  return NKT_OK;
}

constexpr int kSharedSideMinTokens = 8;
// the few-token layer (down + combine in one launch) never forks the shared expert
static_assert(kSharedSideMinTokens > kDcMaxTokens, "side stream and the down + combine launch");


// Whether the shared expert can run on the side stream beside the routed
// experts: its decode form (T up to kSharedDecodeMaxTokens) touches no
// workspace region the routed experts use; the stream and events are made on
// the first call outside graph capture, on the current device.
bool side_stream_ready(Handle* h, hipStream_t st) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  if (!h->side) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return false;
    if (hipStreamCreateWithFlags(&h->side, hipStreamNonBlocking) != hipSuccess) {
      h->side = nullptr;
      return false;
    }
    if (hipEventCreateWithFlags(&h->fork_ev, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&h->join_ev, hipEventDisableTiming) != hipSuccess) {
      if (h->fork_ev) (void)hipEventDestroy(h->fork_ev);
      (void)hipStreamDestroy(h->side);
      h->side = nullptr;
      h->fork_ev = h->join_ev = nullptr;
      return false;
    }
    h->side_device = dev;
  }
  return dev == h->side_device;
}

bool shared_side_ready(Handle* h, int T, const WsLayout& L, hipStream_t st) {
  // a single token's layer is too short for the fork and join to pay
  // (measured: Qwen1.5-MoE T=1 slower by 1 us, T=16 faster by 6 us)
  if (h->Is <= 0 || L.bm_shared != kTileSrcCols || T < kSharedSideMinTokens) return false;
  return side_stream_ready(h, st);
}

// K1 + K2 and the decode gate_up in one launch (launch_gemv_sr): 2 ..
// kSrMaxTokens tokens from given bf16 logits, no shared-expert chunks,
// shapes the kernel takes (int4 weights).  Measured (Qwen3 int4 layer,
// graph replays): T = 2 / 3 / 4 21.0 / 27.0 / 29.1 -> 18.0 / 24.2 / 27.5 us.
bool sr_ok(const Handle* h, int T, const WsLayout& L, const void* logits, int chunks) {
  return logits && h->act_bf16 && chunks == 0 && L.bm == kTileSrcCols &&
         gemv_sr_supported(h->wf, 2 * h->I, h->H, h->I, T, h->E, h->k);
}

int do_sr_gate_up(Handle* h, const void* x, const void* logits, int T, void* ws, const WsLayout& L,
                  hipStream_t st, char* err, size_t len) {
  if (!x) {
    set_err(err, len, "null hidden_states");
    return NKT_ERR;
  }
  GemmArgs a = expert_args(h, PHASE_GATE_UP, false, x, ws, L, T);
  a.route_logits = logits;
  a.route_E = h->E;
  a.route_flags = h->flags;
  a.route_T = T;
  a.ro_resident = h->resident;
  a.ro_max_tiles = L.max_tiles;
  a.ro_ids = ws_ptr<int32_t>(ws, L, NKT_WS_TOPK_IDS);
  a.ro_w = ws_ptr<float>(ws, L, NKT_WS_TOPK_WEIGHTS);
  a.ro_counts = ws_ptr<int32_t>(ws, L, NKT_WS_COUNTS);
  a.ro_offsets = ws_ptr<int32_t>(ws, L, NKT_WS_OFFSETS);
  a.ro_perm = ws_ptr<int32_t>(ws, L, NKT_WS_PERM);
  a.ro_inv = ws_ptr<int32_t>(ws, L, NKT_WS_INV);
  a.ro_tiles = ws_ptr<int32_t>(ws, L, kWsTiles);
  a.ro_n_tiles = ws_ptr<int32_t>(ws, L, kWsNTiles);
  a.ro_tile_src = ws_ptr<int32_t>(ws, L, kWsTileSrc);
  a.ro_wpos = ws_ptr<float>(ws, L, kWsWpos);
  if (!check_hip(launch_gemv_sr(a, h->wf, 0, st), "routing gate_up gemm", err, len)) return NKT_ERR;
  return NKT_OK;
}

// Routing (route(st)), the routed experts, the shared expert and the combine
// of one layer call.  The shared expert forks onto the side stream after
// everything the caller queued on st (its input is ready) and joins back
// before the combine: it overlaps the routing and the routed experts, and a
// graph captured on st holds it as a parallel branch.
// The caller has checked the routing input (logits, or x and the router);
// every other argument and weight slot is checked here before the fork, so
// that a rejected call leaves no fork behind.  After the fork the join is
// recorded and waited for on every path, errors included: the caller's
// stream never runs ahead of the side stream's reads of x and the workspace,
// and a graph being captured on st stays joined.
// allow_side false: the shared expert stays on st (no side stream is made).
// logits (nullable): the router logits when the caller gave them; a single
// token then is routed inside its gate_up launch instead of by route().
// x_from_route: the routing launch writes x (the decoder block's folded
// RMSNorm), so the shared expert forks only after it.
template <typename Route>
int run_layer(Handle* h, const void* x, int T, void* out, void* ws, const WsLayout& L, hipStream_t st, char* err,
              size_t len, Route route, const void* residual = nullptr, bool allow_side = true,
              const void* logits = nullptr, bool x_from_route = false) {
  if (!x || !out) {
    set_err(err, len, "null hidden_states or output");
    return NKT_ERR;
  }
  if (!check_weights(h, h->Is > 0, err, len)) return NKT_ERR;
  // one token, or a few tokens whose pairs rarely share an expert (T k at
  // most E / 4) with int4 weights (decode form, every expert HBM-resident):
  // the down GEMV and the combine run as one launch, whose workgroups each
  // read the weight rows of one token's pairs.  Measured: Qwen3 int4 T = 2 /
  // 3 / 4 24 / 28 / 29.5 -> 21 / 27 / 29 us; where tokens share experts
  // (Mixtral-8x7B T = 4: 104 -> 117 us) or the rows are int8 (Qwen3 int8
  // T = 4: 29.3 -> 30.1 us) the separate launches win.
  const bool few = L.bm == kTileSrcCols && !h->resident && h->act_bf16 &&
                   (T == 1 || (T <= kDcMaxTokens && h->wf == WF_I4 && 4 * T * h->k <= h->E)) &&
                   down_combine_supported(h->wf, h->H, h->I, h->I, h->k);
  // the shared expert as chunks of the routed launches (no launches of its
  // own); the down + combine launch takes them as more items
  int chunks = shared_chunk_count(h, L);
  if (few && chunks > 0 && !down_combine_supported(h->wf, h->H, h->I, h->I, h->k + chunks)) chunks = 0;
  std::unique_lock<std::mutex> lk(h->side_mu, std::defer_lock);
  const bool side = allow_side && !x_from_route && chunks == 0 && shared_side_ready(h, T, L, st);
  if (side) {
    lk.lock();
    if (!check_hip(hipEventRecord(h->fork_ev, st), "fork event", err, len) ||
        !check_hip(hipStreamWaitEvent(h->side, h->fork_ev, 0), "fork wait", err, len))
      return NKT_ERR;
    const int rs = do_shared(h, x, T, ws, L, h->side, err, len);
    const hipError_t je = hipEventRecord(h->join_ev, h->side);
    if (je != hipSuccess) {
      if (rs == NKT_OK) check_hip(je, "join event", err, len);
      (void)hipStreamSynchronize(h->side);  // no event to wait on: drain the branch instead
      return NKT_ERR;
    }
    if (rs != NKT_OK) {
      (void)hipStreamWaitEvent(st, h->join_ev, 0);
      return NKT_ERR;
    }
  }
  if (few) {
    int rc = NKT_OK;
    // routing inside gate_up pays when its workgroups run in about one round
    // (Qwen3: 384, Qwen1.5-MoE: 352 + 352 for the shared expert's chunks);
    // with more (Mixtral-8x7B: 1792) every round would wait for the routing
    // again, and the routing launch is cheaper.  The shared expert's chunk
    // tiles follow the token's k tiles.
    constexpr int64_t kInlineRouteMaxWorkgroups = 1024;
    const int route_tiles = L.max_tiles > h->k + chunks ? L.max_tiles : h->k + chunks;
    const bool inline_route =
        T == 1 && logits && h->E <= 128 &&
        gemv_workgroups(h->wf, PHASE_GATE_UP, 2 * h->I, h->H, h->I, route_tiles) <= kInlineRouteMaxWorkgroups;
    if (inline_route) {
      // K1 + K2 inside the gate_up launch (every workgroup routes the token)
      GemmArgs a = expert_args(h, PHASE_GATE_UP, false, x, ws, L, T);
      a.route_logits = logits;
      a.route_E = h->E;
      a.route_flags = h->flags;
      a.ro_max_tiles = L.max_tiles;
      a.ro_ids = ws_ptr<int32_t>(ws, L, NKT_WS_TOPK_IDS);
      a.ro_w = ws_ptr<float>(ws, L, NKT_WS_TOPK_WEIGHTS);
      a.ro_counts = ws_ptr<int32_t>(ws, L, NKT_WS_COUNTS);
      a.ro_offsets = ws_ptr<int32_t>(ws, L, NKT_WS_OFFSETS);
      a.ro_perm = ws_ptr<int32_t>(ws, L, NKT_WS_PERM);
      a.ro_inv = ws_ptr<int32_t>(ws, L, NKT_WS_INV);
      a.ro_tiles = ws_ptr<int32_t>(ws, L, kWsTiles);
      a.ro_n_tiles = ws_ptr<int32_t>(ws, L, kWsNTiles);
      a.ro_tile_src = ws_ptr<int32_t>(ws, L, kWsTileSrc);
      a.ro_wpos = ws_ptr<float>(ws, L, kWsWpos);
      if (chunks > 0) set_shared_chunks(h, a, PHASE_GATE_UP, ws, L, T, h->k, chunks);
      if (!check_hip(launch_expert_gemm(h, a, PHASE_GATE_UP, L.bm, route_tiles, st), "routing gate_up gemm", err,
                     len))
        return NKT_ERR;
    } else if (sr_ok(h, T, L, logits, chunks)) {
      rc = do_sr_gate_up(h, x, logits, T, ws, L, st, err, len);
    } else {
      rc = route();
      if (rc == NKT_OK) rc = do_expert_phase(h, PHASE_GATE_UP, x, T, ws, L, st, err, len, nullptr, false, chunks);
    }
    if (rc == NKT_OK && h->Is > 0 && chunks == 0) rc = do_shared(h, x, T, ws, L, st, err, len);
    if (rc != NKT_OK) return rc;
    if (!out) {
      set_err(err, len, "null output");
      return NKT_ERR;
    }
    GemmArgs b = expert_args(h, PHASE_DOWN, false, ws_ptr<void>(ws, L, NKT_WS_H), ws, L, T);
    const bool sh = h->Is > 0;
    if (chunks > 0) set_shared_chunks(h, b, PHASE_DOWN, ws, L, T, 0, chunks);
    const CombineTail c{ws_ptr<float>(ws, L, NKT_WS_TOPK_WEIGHTS),
                        ws_ptr<int32_t>(ws, L, NKT_WS_TOPK_IDS),
                        ws_ptr<int32_t>(ws, L, NKT_WS_INV),
                        sh && chunks == 0 ? ws_ptr<float>(ws, L, NKT_WS_SHARED_Y) : nullptr,
                        sh ? ws_ptr<float>(ws, L, NKT_WS_SHARED_GATE) : nullptr,
                        residual,
                        out,
                        T};
    if (!check_hip(launch_down_combine(b, c, h->wf, h->k, st), "down + combine kernel", err, len)) return NKT_ERR;
    return NKT_OK;
  }
  // given logits and the int8 prefill gate_up on the fp16 matrix cores: its
  // input copy is made in the routing launch
  const GemmArgs g = expert_args(h, PHASE_GATE_UP, false, x, ws, L, T);
  const bool prep_in_route = logits && L.bm == kPrefillTileM && g.in16 && g.xinv &&
                             gemm2_supported(h->wf, PHASE_GATE_UP, g.N, g.K, g.I) && gemm2_i8_pipeline(g, h->wf);
  bool prep_done = false;
  // a few tokens from given logits: routing inside the gate_up launch
  const bool sr = sr_ok(h, T, L, logits, chunks);
  int rc = sr ? do_sr_gate_up(h, x, logits, T, ws, L, st, err, len)
              : prep_in_route ? do_route(h, logits, T, ws, L, st, err, len, &g, &prep_done,
                                         h->Is > 0 && chunks == 0 && allow_side && !side)
                              : route();
  // a shared expert in the prefill form forks here, once the routing launch
  // has made the fp16 input copy both expert GEMMs read: its launches (a
  // dense down of few workgroups among them) run beside the routed experts'
  // on the side stream and fill what those leave idle
  bool late = false;
  // the shared expert's prefill down in K parts (shared_down_parts), whether
  // it forks or stays on st
  const int parts = chunks == 0 && !side ? shared_down_parts(h, L, T) : 1;
  const bool late_ok = (prep_done && L.bm_shared != kTileSrcCols && side_stream_ready(h, st)) ||
                       (x_from_route && shared_side_ready(h, T, L, st));
  if (rc == NKT_OK && allow_side && !side && h->Is > 0 && chunks == 0 && late_ok) {
    lk.lock();
    if (!check_hip(hipEventRecord(h->fork_ev, st), "fork event", err, len) ||
        !check_hip(hipStreamWaitEvent(h->side, h->fork_ev, 0), "fork wait", err, len))
      return NKT_ERR;
    const int rs = do_shared(h, x, T, ws, L, h->side, err, len, prep_done, parts);
    const hipError_t je = hipEventRecord(h->join_ev, h->side);
    if (je != hipSuccess) {
      if (rs == NKT_OK) check_hip(je, "join event", err, len);
      (void)hipStreamSynchronize(h->side);  // no event to wait on: drain the branch instead
      return NKT_ERR;
    }
    if (rs != NKT_OK) {
      (void)hipStreamWaitEvent(st, h->join_ev, 0);
      return NKT_ERR;
    }
    late = true;
  }
  if (rc == NKT_OK)
    rc = sr ? do_expert_phase(h, PHASE_DOWN, x, T, ws, L, st, err, len, nullptr, true, chunks)
            : do_experts(h, x, T, ws, L, st, err, len, true, chunks, prep_done);
  if (rc == NKT_OK && !side && !late && h->Is > 0 && chunks == 0)
    rc = do_shared(h, x, T, ws, L, st, err, len, prep_done, parts);
  if (side || late) {
    const hipError_t we = hipStreamWaitEvent(st, h->join_ev, 0);
    if (rc == NKT_OK && !check_hip(we, "join wait", err, len)) rc = NKT_ERR;
  }
  if (rc != NKT_OK) return rc;
  return do_combine(h, T, out, ws, L, st, err, len, nullptr, residual, true, parts > 1 ? parts : chunks);
}

// ---------------------------------------------------------------------------
// Static scratch of nkt_moe_forward_noalloc: the workspace of one layer call
// in a file-scope device array (each GPU that runs the library holds its own
// copy until the process ends).  Host code never passes the array's name to a
// kernel (on the host it is a stand-in symbol, not a device address): the
// device address comes from hipGetSymbolAddress, once per device, with that
// device current, and is kept per device.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = NKT_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxScratchDevices = 64;

}  // namespace

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// The current device's scratch address, looked up on the first call there.
void* device_scratch(char* err, size_t len) {
  int dev = -1;
  if (!check_hip(hipGetDevice(&dev), "hipGetDevice", err, len)) return nullptr;
  if (dev < 0 || dev >= kMaxScratchDevices) {
    set_err(err, len, "device %d outside the scratch table [0, %d)", dev, kMaxScratchDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (!check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)", err, len))
      return nullptr;
    if (!p) {
      set_err(err, len, "hipGetSymbolAddress(scratch) returned a null address");
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" {

void* nkt_moe_create(int num_experts, int top_k, int hidden_size, int moe_intermediate_size,
                     int shared_intermediate_size, int weight_format, int act_dtype,
                     unsigned route_flags, int max_tokens, char* err, size_t err_len) {
  if (num_experts < 1 || num_experts > kMaxExperts) {
    set_err(err, err_len, "num_experts=%d outside [1, %d]", num_experts, kMaxExperts);
    return nullptr;
  }
  if (top_k < 1 || top_k > kMaxTopK || top_k > num_experts) {
    set_err(err, err_len, "top_k=%d outside [1, min(%d, num_experts)]", top_k, kMaxTopK);
    return nullptr;
  }
  if (weight_format < NKT_WEIGHT_F32 || weight_format > NKT_WEIGHT_INT4_G128) {
    set_err(err, err_len, "unknown weight_format %d", weight_format);
    return nullptr;
  }
  if (act_dtype != NKT_DTYPE_F32 && act_dtype != NKT_DTYPE_BF16) {
    set_err(err, err_len, "unknown act_dtype %d", act_dtype);
    return nullptr;
  }
  if ((weight_format == NKT_WEIGHT_F32) != (act_dtype == NKT_DTYPE_F32)) {
    set_err(err, err_len, "fp32 weights require fp32 activations and the other formats bf16");
    return nullptr;
  }
  // the 128-wide K groups and 64-row down tiles need these multiples
  if (hidden_size < 128 || hidden_size % 128 != 0) {
    set_err(err, err_len, "hidden_size=%d must be a positive multiple of 128", hidden_size);
    return nullptr;
  }
  if (moe_intermediate_size < 128 || moe_intermediate_size % 128 != 0) {
    set_err(err, err_len, "moe_intermediate_size=%d must be a positive multiple of 128",
            moe_intermediate_size);
    return nullptr;
  }
  if (shared_intermediate_size < 0 || shared_intermediate_size % 128 != 0) {
    set_err(err, err_len, "shared_intermediate_size=%d must be 0 or a multiple of 128",
            shared_intermediate_size);
    return nullptr;
  }
  if (max_tokens < 1 || (int64_t)max_tokens * top_k > (1 << 24)) {
    set_err(err, err_len, "max_tokens=%d outside [1, 2^24 / top_k]", max_tokens);
    return nullptr;
  }
  {
    // the expert kernels address an activation matrix with 32-bit byte offsets
    const int64_t t = max_tokens, kmax = shared_intermediate_size > hidden_size ? shared_intermediate_size : hidden_size;
    const int64_t most = t * kmax * 2 > t * top_k * moe_intermediate_size * 2 ? t * kmax * 2
                                                                               : t * top_k * moe_intermediate_size * 2;
    if (most >= ((int64_t)1 << 32)) {
      set_err(err, err_len, "max_tokens=%d too large: activations would exceed 4 GiB", max_tokens);
      return nullptr;
    }
  }
  Handle* h = new (std::nothrow) Handle();
  if (!h) {
    set_err(err, err_len, "out of host memory");
    return nullptr;
  }
  h->E = num_experts;
  h->k = top_k;
  h->H = hidden_size;
  h->I = moe_intermediate_size;
  h->Is = shared_intermediate_size;
  h->wf = weight_format;
  h->act_bf16 = act_dtype == NKT_DTYPE_BF16;
  h->flags = route_flags;
  h->max_tokens = max_tokens;
  for (int i = 0; i < NKT_NUM_SLOTS; ++i) h->w[i] = nullptr;
  return h;
}

void nkt_moe_destroy(void* handle) { delete (Handle*)handle; }

int nkt_moe_weight_bytes(void* handle, int slot, size_t* bytes, char* err, size_t err_len) {
  Handle* h = (Handle*)handle;
  if (!h || !bytes || slot < 0 || slot >= NKT_NUM_SLOTS) {
    set_err(err, err_len, "bad arguments");
    return NKT_ERR;
  }
  *bytes = slot_bytes(h, slot);
  return NKT_OK;
}

int nkt_moe_pack_weight(void* handle, int slot, int expert, const void* src, const void* src_scales,
                        void* dst, void* dst_scales, void* stream, char* err, size_t err_len) {
  Handle* h = (Handle*)handle;
  if (!h) {
    set_err(err, err_len, "null handle");
    return NKT_ERR;
  }
  if (slot == NKT_SLOT_ROUTER) {
    if (!h->act_bf16) {
      set_err(err, err_len, "the fused router needs bf16 activations");
      return NKT_ERR;
    }
    if (expert != 0 || !src || !dst) {
      set_err(err, err_len, "router: expert must be 0 and src/dst non-null");
      return NKT_ERR;
    }
    if (!check_hip(launch_pack(WF_BF16, src, nullptr, router_rows(h), h->H, (uint8_t*)dst, nullptr,
                               (hipStream_t)stream, h->E),
                   "router pack kernel", err, err_len))
      return NKT_ERR;
    return NKT_OK;
  }
  if (slot != NKT_SLOT_GATE_UP && slot != NKT_SLOT_DOWN && slot != NKT_SLOT_SHARED_GATE_UP &&
      slot != NKT_SLOT_SHARED_DOWN) {
    set_err(err, err_len, "slot %d is not a packable projection", slot);
    return NKT_ERR;
  }
  int N, K, ne;
  if (!slot_shape(h, slot, &N, &K, &ne)) {
    set_err(err, err_len, "slot %d unused by this handle", slot);
    return NKT_ERR;
  }
  if (expert < 0 || expert >= ne) {
    set_err(err, err_len, "expert %d outside [0, %d)", expert, ne);
    return NKT_ERR;
  }
  const bool quant = h->wf == WF_I4 || h->wf == WF_I8;
  if (!src || !dst || (quant && (!src_scales || !dst_scales))) {
    set_err(err, err_len, "null source or destination pointer");
    return NKT_ERR;
  }
  uint8_t* d = (uint8_t*)dst + (int64_t)expert * code_bytes(h, N, K);
  uint16_t* ds = quant ? (uint16_t*)dst_scales + (int64_t)expert * scale_elems(h, N, K) : nullptr;
  if (!check_hip(launch_pack(h->wf, src, src_scales, N, K, d, ds, (hipStream_t)stream), "pack kernel",
                 err, err_len))
    return NKT_ERR;
  return NKT_OK;
}

int nkt_moe_bind_weights(void* handle, const void* const* ptrs, char* err, size_t err_len) {
  Handle* h = (Handle*)handle;
  if (!h || !ptrs) {
    set_err(err, err_len, "bad arguments");
    return NKT_ERR;
  }
  for (int i = 0; i < NKT_NUM_SLOTS; ++i) h->w[i] = ptrs[i];
  return NKT_OK;
}

int nkt_moe_workspace_bytes(void* handle, int num_tokens, size_t* bytes, char* err, size_t err_len) {
  Handle* h = (Handle*)handle;
  if (!h || !bytes) {
    set_err(err, err_len, "null handle or output pointer");
    return NKT_ERR;
  }
  if (num_tokens < 0 || num_tokens > h->max_tokens) {
    set_err(err, err_len, "num_tokens=%d outside [0, max_tokens=%d]", num_tokens, h->max_tokens);
    return NKT_ERR;
  }
  *bytes = ws_layout(h, num_tokens).total;
  return NKT_OK;
}

int nkt_moe_workspace_region(void* handle, int num_tokens, int region, size_t* offset, char* err,
                             size_t err_len) {
  Handle* h = (Handle*)handle;
  if (!h || !offset) {
    set_err(err, err_len, "null handle or output pointer");
    return NKT_ERR;
  }
  if (num_tokens < 0 || num_tokens > h->max_tokens) {
    set_err(err, err_len, "num_tokens=%d outside [0, max_tokens=%d]", num_tokens, h->max_tokens);
    return NKT_ERR;
  }
  if (region < 0 || region >= NKT_WS_NUM_REGIONS) {
    set_err(err, err_len, "region=%d outside [0, %d)", region, NKT_WS_NUM_REGIONS);
    return NKT_ERR;
  }
  *offset = ws_layout(h, num_tokens).off[region];
  return NKT_OK;
}

int nkt_moe_route(void* handle, const void* router_logits, int num_tokens, void* workspace,
                  size_t workspace_bytes, void* stream, char* err, size_t err_len) {
  Handle* h = (Handle*)handle;
  if (!check_call(h, num_tokens, workspace, workspace_bytes, err, err_len)) return NKT_ERR;
  if (num_tokens == 0) return NKT_OK;
  const WsLayout L = ws_layout(h, num_tokens);
  return do_route(h, router_logits, num_tokens, workspace, L, (hipStream_t)stream, err, err_len);
}

int nkt_moe_experts(void* handle, const void* hidden_states, int num_tokens, void* workspace,
                    size_t workspace_bytes, void* stream, char* err, size_t err_len) {
  Handle* h = (Handle*)handle;
  if (!check_call(h, num_tokens, workspace, workspace_bytes, err, err_len)) return NKT_ERR;
  if (num_tokens == 0) return NKT_OK;
  const WsLayout L = ws_layout(h, num_tokens);
  return do_experts(h, hidden_states, num_tokens, workspace, L, (hipStream_t)stream, err, err_len);
}

int nkt_moe_experts_phase(void* handle, int phase, const void* hidden_states, int num_tokens,
                          void* workspace, size_t workspace_bytes, void* stream, char* err,
                          size_t err_len) {
  Handle* h = (Handle*)handle;
  if (!check_call(h, num_tokens, workspace, workspace_bytes, err, err_len)) return NKT_ERR;
  if (phase != PHASE_GATE_UP && phase != PHASE_DOWN) {
    set_err(err, err_len, "phase must be 0 (gate_up) or 1 (down), got %d", phase);
    return NKT_ERR;
  }
  if (num_tokens == 0) return NKT_OK;
  const WsLayout L = ws_layout(h, num_tokens);
  return do_expert_phase(h, phase, hidden_states, num_tokens, workspace, L, (hipStream_t)stream, err,
                         err_len);
}

int nkt_moe_experts_phase_timed(void* handle, int phase, const void* hidden_states, int num_tokens,
                                void* workspace, size_t workspace_bytes, void* stream, void* start_event,
                                void* stop_event, char* err, size_t err_len) {
  Handle* h = (Handle*)handle;
  if (!check_call(h, num_tokens, workspace, workspace_bytes, err, err_len)) return NKT_ERR;
  if (phase != PHASE_GATE_UP && phase != PHASE_DOWN) {
    set_err(err, err_len, "phase must be 0 (gate_up) or 1 (down), got %d", phase);
    return NKT_ERR;
  }
  if (!start_event || !stop_event) {
    set_err(err, err_len, "null timing event");
    return NKT_ERR;
  }
  if (num_tokens == 0) return NKT_OK;
  const WsLayout L = ws_layout(h, num_tokens);
  const KernelTimer tm{(hipEvent_t)start_event, (hipEvent_t)stop_event};
  return do_expert_phase(h, phase, hidden_states, num_tokens, workspace, L, (hipStream_t)stream, err,
                         err_len, &tm);
}

int nkt_moe_shared(void* handle, const void* hidden_states, int num_tokens, void* workspace,
                   size_t workspace_bytes, void* stream, char* err, size_t err_len) {
  Handle* h = (Handle*)handle;
  if (!check_call(h, num_tokens, workspace, workspace_bytes, err, err_len)) return NKT_ERR;
  if (num_tokens == 0) return NKT_OK;
  const WsLayout L = ws_layout(h, num_tokens);
  return do_shared(h, hidden_states, num_tokens, workspace, L, (hipStream_t)stream, err, err_len);
}

int nkt_moe_combine(void* handle, int num_tokens, void* out, void* workspace, size_t workspace_bytes,
                    void* stream, char* err, size_t err_len) {
  Handle* h = (Handle*)handle;
  if (!check_call(h, num_tokens, workspace, workspace_bytes, err, err_len)) return NKT_ERR;
  if (num_tokens == 0) return NKT_OK;
  const WsLayout L = ws_layout(h, num_tokens);
  return do_combine(h, num_tokens, out, workspace, L, (hipStream_t)stream, err, err_len);
}

int nkt_moe_combine_extra(void* handle, int num_tokens, const void* extra, void* out, void* workspace,
                          size_t workspace_bytes, void* stream, char* err, size_t err_len) {
  Handle* h = (Handle*)handle;
  if (!check_call(h, num_tokens, workspace, workspace_bytes, err, err_len)) return NKT_ERR;
  if (num_tokens == 0) return NKT_OK;
  const WsLayout L = ws_layout(h, num_tokens);
  return do_combine(h, num_tokens, out, workspace, L, (hipStream_t)stream, err, err_len, extra);
}

int nkt_moe_bind_residency(void* handle, const void* resident, char* err, size_t err_len) {
  Handle* h = (Handle*)handle;
  if (!h) {
    set_err(err, err_len, "null handle");
    return NKT_ERR;
  }
  h->resident = (const uint8_t*)resident;
  return NKT_OK;
}

int nkt_moe_forward(void* handle, const void* hidden_states, const void* router_logits,
                    int num_tokens, void* out, void* workspace, size_t workspace_bytes, void* stream,
                    char* err, size_t err_len) {
  Handle* h = (Handle*)handle;
  if (!check_call(h, num_tokens, workspace, workspace_bytes, err, err_len)) return NKT_ERR;
  if (num_tokens == 0) return NKT_OK;
  if (!router_logits) {
    set_err(err, err_len, "null router_logits");
    return NKT_ERR;
  }
  const WsLayout L = ws_layout(h, num_tokens);
  hipStream_t st = (hipStream_t)stream;
  return run_layer(h, hidden_states, num_tokens, out, workspace, L, st, err, err_len,
                   [&] { return do_route(h, router_logits, num_tokens, workspace, L, st, err, err_len); }, nullptr,
                   true, router_logits);
}

int nkt_moe_route_given(void* handle, const int64_t* topk_ids, const float* topk_weights, int num_tokens,
                        void* workspace, size_t workspace_bytes, void* stream, char* err, size_t err_len) {
  Handle* h = (Handle*)handle;
  if (!check_call(h, num_tokens, workspace, workspace_bytes, err, err_len)) return NKT_ERR;
  if (num_tokens == 0) return NKT_OK;
  const WsLayout L = ws_layout(h, num_tokens);
  return do_route_given(h, topk_ids, topk_weights, num_tokens, workspace, L, (hipStream_t)stream, err, err_len);
}

int nkt_moe_forward_routed(void* handle, const void* hidden_states, const int64_t* topk_ids,
                           const float* topk_weights, int num_tokens, void* out, void* workspace,
                           size_t workspace_bytes, void* stream, char* err, size_t err_len) {
  Handle* h = (Handle*)handle;
  if (!check_call(h, num_tokens, workspace, workspace_bytes, err, err_len)) return NKT_ERR;
  if (num_tokens == 0) return NKT_OK;
  if (!topk_ids || !topk_weights) {
    set_err(err, err_len, "null topk_ids or topk_weights");
    return NKT_ERR;
  }
  const WsLayout L = ws_layout(h, num_tokens);
  hipStream_t st = (hipStream_t)stream;
  return run_layer(h, hidden_states, num_tokens, out, workspace, L, st, err, err_len, [&] {
    return do_route_given(h, topk_ids, topk_weights, num_tokens, workspace, L, st, err, err_len);
  });
}

int nkt_moe_forward_noalloc(void* handle, const void* hidden_states, const void* router_logits, int num_tokens,
                            void* out, void* stream, char* err, size_t err_len) {
  Handle* h = (Handle*)handle;
  if (!h) {
    set_err(err, err_len, "null handle");
    return NKT_ERR;
  }
  if (num_tokens < 0 || num_tokens > h->max_tokens) {
    set_err(err, err_len, "num_tokens=%d outside [0, max_tokens=%d]", num_tokens, h->max_tokens);
    return NKT_ERR;
  }
  if (num_tokens == 0) return NKT_OK;
  if (!router_logits) {
    set_err(err, err_len, "null router_logits");
    return NKT_ERR;
  }
  const WsLayout L = ws_layout(h, num_tokens);
  if (L.total > kScratchBytes) {
    set_err(err, err_len,
            "num_tokens=%d needs %zu bytes of workspace; the static scratch of nkt_moe_forward_noalloc holds %zu "
            "(use nkt_moe_forward with a caller-owned workspace)",
            num_tokens, L.total, kScratchBytes);
    return NKT_ERR;
  }
  void* ws = device_scratch(err, err_len);
  if (!ws) return NKT_ERR;
  hipStream_t st = (hipStream_t)stream;
  return run_layer(h, hidden_states, num_tokens, out, ws, L, st, err, err_len,
                   [&] { return do_route(h, router_logits, num_tokens, ws, L, st, err, err_len); }, nullptr,
                   /*allow_side=*/false, router_logits);
}

int nkt_moe_route_hidden(void* handle, const void* hidden_states, int num_tokens, void* workspace,
                         size_t workspace_bytes, void* stream, char* err, size_t err_len) {
  Handle* h = (Handle*)handle;
  if (!check_call(h, num_tokens, workspace, workspace_bytes, err, err_len)) return NKT_ERR;
  if (num_tokens == 0) return NKT_OK;
  const WsLayout L = ws_layout(h, num_tokens);
  return do_route_hidden(h, hidden_states, num_tokens, workspace, L, (hipStream_t)stream, err, err_len);
}

int nkt_moe_forward_hidden(void* handle, const void* hidden_states, int num_tokens, void* out, void* workspace,
                           size_t workspace_bytes, void* stream, char* err, size_t err_len) {
  Handle* h = (Handle*)handle;
  if (!check_call(h, num_tokens, workspace, workspace_bytes, err, err_len)) return NKT_ERR;
  if (num_tokens == 0) return NKT_OK;
  if (!check_route_hidden(h, hidden_states, err, err_len)) return NKT_ERR;
  const WsLayout L = ws_layout(h, num_tokens);
  hipStream_t st = (hipStream_t)stream;
  if (logits_first(h, num_tokens)) {
    // everything run_layer checks, checked before the router's launch
    if (!out) {
      set_err(err, err_len, "null output");
      return NKT_ERR;
    }
    if (!check_weights(h, h->Is > 0, err, err_len)) return NKT_ERR;
    if (do_router_logits(h, hidden_states, num_tokens, workspace, L, st, err, err_len) != NKT_OK) return NKT_ERR;
    const void* lg = ws_ptr<void>(workspace, L, NKT_WS_ROUTER_LOGITS);
    return run_layer(h, hidden_states, num_tokens, out, workspace, L, st, err, err_len,
                     [&] { return do_route(h, lg, num_tokens, workspace, L, st, err, err_len); }, nullptr, true, lg);
  }
  return run_layer(h, hidden_states, num_tokens, out, workspace, L, st, err, err_len,
                   [&] { return do_route_hidden(h, hidden_states, num_tokens, workspace, L, st, err, err_len); });
}

int nkt_moe_forward_block(void* handle, const void* hidden_states, const void* norm_weight, float eps,
                          int num_tokens, void* out, void* workspace, size_t workspace_bytes, void* stream,
                          char* err, size_t err_len) {
  Handle* h = (Handle*)handle;
  if (!check_call(h, num_tokens, workspace, workspace_bytes, err, err_len)) return NKT_ERR;
  if (num_tokens == 0) return NKT_OK;
  if (!h->act_bf16) {
    set_err(err, err_len, "the decoder-block form needs bf16 activations");
    return NKT_ERR;
  }
  if (!hidden_states || !norm_weight || !out) {
    set_err(err, err_len, "null hidden_states, norm_weight or output");
    return NKT_ERR;
  }
  if (!(eps >= 0.f)) {
    set_err(err, err_len, "eps must be >= 0");
    return NKT_ERR;
  }
  const WsLayout L = ws_layout(h, num_tokens);
  hipStream_t st = (hipStream_t)stream;
  void* x = ws_ptr<void>(workspace, L, NKT_WS_NORMED);
  if (!check_route_hidden(h, x, err, err_len) || !check_weights(h, h->Is > 0, err, err_len)) return NKT_ERR;
  if (logits_first(h, num_tokens)) {
    if (do_router_logits(h, hidden_states, num_tokens, workspace, L, st, err, err_len, norm_weight, eps) != NKT_OK)
      return NKT_ERR;
    const void* lg = ws_ptr<void>(workspace, L, NKT_WS_ROUTER_LOGITS);
    return run_layer(h, x, num_tokens, out, workspace, L, st, err, err_len,
                     [&] { return do_route(h, lg, num_tokens, workspace, L, st, err, err_len); }, hidden_states, true,
                     lg);
  }
  // the routing launch normalises x itself (and writes NKT_WS_NORMED, which
  // the experts read) whenever it takes the batch
  return run_layer(h, x, num_tokens, out, workspace, L, st, err, err_len,
                   [&] {
                     return do_route_hidden(h, hidden_states, num_tokens, workspace, L, st, err, err_len, norm_weight,
                                            eps);
                   },
                   hidden_states, true, nullptr, true);
}

const char* nkt_moe_version(void) { return "nkt_moe 0.4.0 gfx950"; }

}  // extern "C"
