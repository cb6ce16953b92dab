/*
 * nkt_moe.h -- C ABI of the MI355X (gfx950) MoE expert path.
 *
 * One handle describes one MoE layer shape.  All device buffers are owned by
 * the caller and passed as plain pointers; every entry point enqueues work on
 * the given HIP stream and returns without synchronising the host.  Entry
 * points return NKT_OK (0) or NKT_ERR (-1) and write a message into
 * err[0..err_len) on failure (the convention of the reference's native
 * bridge, nano_ktrans/kernels/pim_native/host_quantized_bridge.c:157-167,
 * 226-281, 640-648: handle + error buffer + int return code).
 *
 * Pair index: token t, top-k slot j  ->  p = t * top_k + j.
 * Position:   the rank of a pair in (expert ascending, token ascending) order.
 *
 * Weight formats (device layout written by nkt_moe_pack_weight):
 *   NKT_WEIGHT_F32        fp32 weights, fp32 activations
 *   NKT_WEIGHT_BF16       bf16 weights
 *   NKT_WEIGHT_INT8_PC    int8, one bf16 scale per output channel
 *   NKT_WEIGHT_INT4_G128  int4, one bf16 scale per output channel per 128 inputs
 * Source layout accepted by nkt_moe_pack_weight (device pointers):
 *   dense:  [N, K] row-major (nn.Linear.weight), fp32 or bf16
 *   int8:   int32 words [N, K/4],  byte j of word w is column 4w+j, stored q+128
 *   int4:   int32 words [N, K/8],  nibble j of word w is column 8w+j, stored q+8
 *           (GPTQLinearWeight.qweight, nano_ktrans/kernels/weight_loader.py:25-69)
 *   scales: bf16 [N, groups] (groups = K/128 for int4, 1 for int8)
 * "gate_up" is the packed [2I, H] projection (gate rows, then up rows;
 * nano_ktrans/layers/expert_mlp.py:26-41, 56-72); "down" is [H, I].
 */
#ifndef NKT_MOE_H
#define NKT_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NKT_OK 0
#define NKT_ERR (-1)

/* weight formats */
#define NKT_WEIGHT_F32 0
#define NKT_WEIGHT_BF16 1
#define NKT_WEIGHT_INT8_PC 2
#define NKT_WEIGHT_INT4_G128 3

/* activation / logits dtypes */
#define NKT_DTYPE_F32 0
#define NKT_DTYPE_BF16 1

/* routing flags (nano_ktrans/models/config.py:26-75 router_use_softmax,
 * normalize_topk_prob) */
#define NKT_ROUTE_SOFTMAX 1u
#define NKT_ROUTE_RENORM 2u

/* weight slots for nkt_moe_weight_bytes / nkt_moe_pack_weight / nkt_moe_bind_weights */
#define NKT_SLOT_GATE_UP 0        /* packed code blocks, all experts        */
#define NKT_SLOT_GATE_UP_SCALES 1 /* bf16 scales, all experts               */
#define NKT_SLOT_DOWN 2
#define NKT_SLOT_DOWN_SCALES 3
#define NKT_SLOT_SHARED_GATE_UP 4 /* shared expert (one expert)             */
#define NKT_SLOT_SHARED_GATE_UP_SCALES 5
#define NKT_SLOT_SHARED_DOWN 6
#define NKT_SLOT_SHARED_DOWN_SCALES 7
#define NKT_SLOT_SHARED_GATE 8 /* shared_expert_gate.weight [1, H], act dtype */
#define NKT_SLOT_ROUTER 9      /* router gate weight [E, H] (bf16 act only), packed */
#define NKT_NUM_SLOTS 10

/* workspace regions for nkt_moe_workspace_region */
#define NKT_WS_TOPK_IDS 0     /* int32 [T, k]            */
#define NKT_WS_TOPK_WEIGHTS 1 /* fp32  [T, k]            */
#define NKT_WS_COUNTS 2       /* int32 [E]               */
#define NKT_WS_OFFSETS 3      /* int32 [E + 1]           */
#define NKT_WS_PERM 4         /* int32 [T * k]  pos -> p */
#define NKT_WS_INV 5          /* int32 [T * k]  p -> pos */
#define NKT_WS_H 6            /* act dtype [T*k, I]  SwiGLU activations by position */
#define NKT_WS_Y 7            /* fp32 [T*k, H] expert outputs of nkt_moe_experts*: row = pair t*k + slot in the decode
                                 form (T*k / E up to 4.5 for int8 weights, 3.5 with a shared expert; 8 for int4, 6 for
                                 I >= 8192; 12 for the others), else position.  nkt_moe_forward* in the prefill form
                                 leaves it compact: fp16 [T*k, H] by position, each 256-column slab of a row times a
                                 power of two, then fp32 [T*k, H/256] with the inverse of each slab's factor; a
                                 one-token call (and a 2-4 token call with int4 weights and 4*T*k <= E), whose down
                                 projection and combine share one launch, does not write it */
#define NKT_WS_SHARED_GATE 8  /* fp32 [T] sigmoid(x . g)                              */
#define NKT_WS_SHARED_H 9     /* act dtype [T, I_s]                                    */
#define NKT_WS_SHARED_Y 10    /* fp32 [T, H]; not written by a decode-form nkt_moe_forward* whose shared expert
                                 runs inside the routed launches (I_s a multiple of I, I_s / I <= 8, bf16
                                 activations, up to 256 tokens) */
#define NKT_WS_ROUTER_LOGITS 11 /* bf16 [T, E] router logits of the *_hidden entry points */
#define NKT_WS_NORMED 12        /* bf16 [T, H] RMSNorm output of nkt_moe_forward_block    */
#define NKT_WS_SYNC 13          /* uint32 [32]: words 0 .. 16 the single-launch router's counters (zero
                                   between calls), word NKT_STATUS_BAD_ROUTING a status word */
#define NKT_WS_NUM_REGIONS 14

/* Status word (uint32 index into NKT_WS_SYNC), 0 unless a fault was seen
 * since the caller last cleared it: set to 1 by the call that sees the fault
 * (no entry point clears it); the caller reads it after synchronising and
 * writes 0 to clear it.  nkt_moe_route_given / nkt_moe_forward_routed
 * dropped a slot whose id was outside [0, E) or repeated an earlier slot's id
 * of the same token. */
#define NKT_STATUS_BAD_ROUTING 30

/* Create a handle for one layer shape.
 * Replaces the construction of HybridMoE's expert state
 * (nano_ktrans/layers/hybrid_moe.py:55-290).  shared_inter = 0: no shared
 * expert.  max_tokens bounds num_tokens of every later call.  Returns NULL on
 * failure. */
void* nkt_moe_create(int num_experts, int top_k, int hidden_size, int moe_intermediate_size,
                     int shared_intermediate_size, int weight_format, int act_dtype,
                     unsigned route_flags, int max_tokens, char* err, size_t err_len);

void nkt_moe_destroy(void* handle);

/* Bytes of device memory a weight slot needs (all experts of the layer). */
int nkt_moe_weight_bytes(void* handle, int slot, size_t* bytes, char* err, size_t err_len);

/* Repack one expert's projection from the source layout into the device
 * layout inside dst (a buffer of nkt_moe_weight_bytes(slot) bytes; dst_scales
 * likewise for the matching *_SCALES slot, NULL for dense formats).
 * slot: NKT_SLOT_GATE_UP / NKT_SLOT_DOWN (expert in [0, E)) or
 * NKT_SLOT_SHARED_GATE_UP / NKT_SLOT_SHARED_DOWN (expert 0), or
 * NKT_SLOT_ROUTER (expert 0; src = the gate weight [E, H] in bf16, rows
 * padded to a multiple of 32 with zeros).  Replaces the per-expert weight
 * load of nano_ktrans/layers/expert_mlp.py:56-85 and
 * nano_ktrans/kernels/weight_loader.py:278-325, 355-392. */
int nkt_moe_pack_weight(void* handle, int slot, int expert, const void* src, const void* src_scales,
                        void* dst, void* dst_scales, void* stream, char* err, size_t err_len);

/* Bind the device weight buffers used by later forward calls.  ptrs has
 * NKT_NUM_SLOTS entries (NULL where a slot does not apply). */
int nkt_moe_bind_weights(void* handle, const void* const* ptrs, char* err, size_t err_len);

/* Workspace size for num_tokens tokens, and the byte offset of each region.
 * The sync area -- the first NKT_SYNC_AREA_BYTES bytes of every workspace,
 * the same for every handle and token count (the NKT_WS_SYNC words and the
 * single-launch router's counters and published selection masks) -- must be
 * zero before a workspace's first use; every call of every handle leaves it
 * zero (the status word aside, when a call reports a fault), so one
 * workspace may serve several handles in turn. */
#define NKT_SYNC_AREA_BYTES 65792
int nkt_moe_workspace_bytes(void* handle, int num_tokens, size_t* bytes, char* err, size_t err_len);
int nkt_moe_workspace_region(void* handle, int num_tokens, int region, size_t* offset,
                             char* err, size_t err_len);

/* K1 + K2: router softmax / top-k / renormalise, then the deterministic
 * count / prefix-sum / permute.  Replaces nano_ktrans/layers/hybrid_moe.py:
 * 3321-3329 (routing) and 3384-3386, 3512-3526 (per-expert token lists).
 * router_logits: [T, E] in the handle's act dtype.  Results land in the
 * workspace regions NKT_WS_TOPK_IDS .. NKT_WS_INV. */
int nkt_moe_route(void* handle, const void* router_logits, int num_tokens, void* workspace,
                  size_t workspace_bytes, void* stream, char* err, size_t err_len);

/* K2 from routing the caller computed (K1 is not run): topk_ids int64
 * [T, k] and topk_weights fp32 [T, k] (device).  The expert side of the
 * reference's offload contract: ExpertOffloadBackend.submit_forward(
 * hidden_states, topk_ids, topk_weights, cuda_stream)
 * (nano_ktrans/kernels/offload_backend.py:40-52) and kt-kernel's
 * forward_task(bsz, k, expert_ids int64*, weights fp32*, ...)
 * (nano_ktrans/kernels/cpu_moe.py:570-592).  The slots of a token may come
 * in any order (the combine adds experts in ascending id).  Every id must be
 * in [0, E) and a token's k ids distinct: a slot breaking that is dropped (it
 * adds nothing) and status word NKT_STATUS_BAD_ROUTING is set.  Results land
 * in NKT_WS_TOPK_IDS .. NKT_WS_INV as after nkt_moe_route. */
int nkt_moe_route_given(void* handle, const int64_t* topk_ids, const float* topk_weights, int num_tokens,
                        void* workspace, size_t workspace_bytes, void* stream, char* err, size_t err_len);

/* K3: grouped SwiGLU expert GEMM for the routed experts (needs a prior
 * nkt_moe_route on the same workspace).  Replaces the per-expert loop
 * nano_ktrans/layers/hybrid_moe.py:3501-3533 / expert_mlp.py:20-41 and
 * nano_ktrans/kernels/cpu_moe.py:419-450.  Writes NKT_WS_H and NKT_WS_Y. */
int nkt_moe_experts(void* handle, const void* hidden_states, int num_tokens, void* workspace,
                    size_t workspace_bytes, void* stream, char* err, size_t err_len);

/* K3 as its two launches: phase 0 = gate_up GEMM + SwiGLU (reads
 * hidden_states, writes NKT_WS_H), phase 1 = down GEMM (reads NKT_WS_H,
 * writes NKT_WS_Y; hidden_states unused).  nkt_moe_experts is phase 0 then
 * phase 1; callers may enqueue other work between the two. */
int nkt_moe_experts_phase(void* handle, int phase, const void* hidden_states, int num_tokens,
                          void* workspace, size_t workspace_bytes, void* stream, char* err,
                          size_t err_len);

/* nkt_moe_experts_phase with the phase's expert-GEMM kernel stamped by two
 * hipEvent_t (start_event, stop_event) at its own start and end
 * (hipExtLaunchKernelGGL), so that hipEventElapsedTime gives that kernel's
 * duration without launch gaps.  No counterpart in the reference: a
 * measurement hook for benchmarks (bench.py's roofline). */
int nkt_moe_experts_phase_timed(void* handle, int phase, const void* hidden_states, int num_tokens,
                                void* workspace, size_t workspace_bytes, void* stream, void* start_event,
                                void* stop_event, char* err, size_t err_len);

/* K4 (+ K3 with one dense expert): shared expert and its sigmoid gate,
 * nano_ktrans/models/mixtral.py:170-179, 215-218.  Writes NKT_WS_SHARED_*. */
int nkt_moe_shared(void* handle, const void* hidden_states, int num_tokens, void* workspace,
                   size_t workspace_bytes, void* stream, char* err, size_t err_len);

/* K5: un-permute and weighted combine in ascending expert id order, plus the
 * gated shared expert when the handle has one; out [T, H] in the act dtype.
 * Replaces nano_ktrans/layers/hybrid_moe.py:3529-3533, 3570 and
 * nano_ktrans/kernels/cpu_moe.py:528-538. */
int nkt_moe_combine(void* handle, int num_tokens, void* out, void* workspace,
                    size_t workspace_bytes, void* stream, char* err, size_t err_len);

/* Mixed residency (nano_ktrans/layers/hybrid_moe.py:264-290, 3373-3378,
 * 3563-3570: experts whose gpu_experts_mask entry is False run in an offload
 * backend).  resident: device bytes [E], 0 = the expert's weights are not in
 * HBM; NULL (the default) = every expert resident.  Later route / experts
 * calls give non-resident experts no GEMM tiles (counts, offsets and the
 * permutation still cover every pair), and the combine skips their slots. */
int nkt_moe_bind_residency(void* handle, const void* resident, char* err, size_t err_len);

/* nkt_moe_combine plus extra [T, H] (act dtype, NULL for none): the sum the
 * offload backend's sync_forward returned for the non-resident experts
 * (nano_ktrans/kernels/offload_backend.py:40-52), added after the resident
 * experts and before the shared expert, in the same fp32 sum. */
int nkt_moe_combine_extra(void* handle, int num_tokens, const void* extra, void* out, void* workspace,
                          size_t workspace_bytes, void* stream, char* err, size_t err_len);

/* The whole layer: route, experts, shared expert, combine.  Replaces
 * HybridMoE.forward (nano_ktrans/layers/hybrid_moe.py:3310-3570) plus the
 * shared-expert add of nano_ktrans/models/mixtral.py:215-218. */
int nkt_moe_forward(void* handle, const void* hidden_states, const void* router_logits,
                    int num_tokens, void* out, void* workspace, size_t workspace_bytes,
                    void* stream, char* err, size_t err_len);

/* The whole layer from the caller's routing: nkt_moe_route_given, then the
 * experts, shared expert (when the handle has one) and combine of
 * nkt_moe_forward.  out[t] = sum over the token's slots, in ascending expert
 * id, of topk_weights[t, j] * expert_{topk_ids[t, j]}(x_t), in fp32 with one
 * rounding (experts that nkt_moe_bind_residency marks non-resident add
 * nothing), plus the gated shared expert.  Replaces the offload backend's
 * submit_forward / sync_forward pair (nano_ktrans/kernels/offload_backend.py:
 * 40-52, nano_ktrans/kernels/cpu_moe.py:491-539, 570-630): with residency
 * set to the experts a backend serves, out is that backend's sum. */
int nkt_moe_forward_routed(void* handle, const void* hidden_states, const int64_t* topk_ids,
                           const float* topk_weights, int num_tokens, void* out, void* workspace,
                           size_t workspace_bytes, void* stream, char* err, size_t err_len);

/* Router GEMV + K1 + K2: router_logits = hidden_states . gate^T (fp32
 * accumulation, rounded to bf16 as nn.Linear(H, E, bias=False) does in bf16),
 * written to NKT_WS_ROUTER_LOGITS, then routed as by nkt_moe_route.  Fuses the
 * decoder layer's gate (nano_ktrans/models/mixtral.py:127, 212) into the
 * expert path; needs bf16 activations and a packed NKT_SLOT_ROUTER.  Up to
 * 64 tokens (and top_k * tokens <= 1024, num_experts % 4 == 0, hidden_size <=
 * 8192) the GEMV, routing and grouping are one launch whose workgroups hand
 * their results on through counters in the sync area without waiting for
 * each other; larger batches take three launches. */
int nkt_moe_route_hidden(void* handle, const void* hidden_states, int num_tokens, void* workspace,
                         size_t workspace_bytes, void* stream, char* err, size_t err_len);

/* The whole layer from hidden states alone: nkt_moe_route_hidden, then the
 * experts, shared expert and combine of nkt_moe_forward.  Replaces
 * router_logits = self.gate(x); HybridMoE.forward(x, router_logits)
 * (nano_ktrans/models/mixtral.py:212-218).  Up to 16 tokens the router GEMV
 * is a launch of its own (the logits to NKT_WS_ROUTER_LOGITS, the sync area
 * untouched) and the layer then runs exactly as nkt_moe_forward on those
 * logits (the same launches and bits). */
int nkt_moe_forward_hidden(void* handle, const void* hidden_states, int num_tokens, void* out,
                           void* workspace, size_t workspace_bytes, void* stream, char* err,
                           size_t err_len);

/* The decoder layer's MoE half (nano_ktrans/models/mixtral.py:206-223):
 * x = RMSNorm(hidden_states) with norm_weight [H] (bf16, device) and eps as
 * nano_ktrans/layers/norm.py:11-17 computes it (written to NKT_WS_NORMED;
 * inside the router's launch -- the router GEMV alone up to 16 tokens,
 * nkt_moe_route_hidden's one-launch form up to 64), then the layer from x as
 * nkt_moe_forward_hidden, and out = hidden_states + that output (the
 * residual add inside the combine's fp32 sum).  bf16 only. */
int nkt_moe_forward_block(void* handle, const void* hidden_states, const void* norm_weight, float eps,
                          int num_tokens, void* out, void* workspace, size_t workspace_bytes, void* stream,
                          char* err, size_t err_len);

/* Largest workspace (bytes, per GPU) that nkt_moe_forward_noalloc serves
 * from the library's static scratch: compare nkt_moe_workspace_bytes. */
#define NKT_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/* nkt_moe_forward without a workspace argument and without any allocation:
 * the workspace is a static device array of NKT_NOALLOC_SCRATCH_BYTES
 * inside the library (one per GPU, held until the process ends), so the call
 * makes no hipMalloc / hipFree and creates no stream (the shared expert runs
 * on `stream`, after the routed experts).  No counterpart in the reference:
 * it is for callers that cannot allocate -- code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc.  Fails (NKT_ERR,
 * message in err) when nkt_moe_workspace_bytes(num_tokens) exceeds
 * NKT_NOALLOC_SCRATCH_BYTES (decode batches of every supported shape fit;
 * large prefill batches do not).  Every call on one GPU shares that GPU's
 * scratch: calls that overlap on one GPU (two streams, two handles, two
 * threads) race and must be serialised by the caller.  The scratch starts
 * zeroed (a static device array) and, as after every layer call, its sync
 * area (the NKT_WS_SYNC words and the router's published masks) is zero
 * again when the call ends: from given logits, batches of 17 .. 64 tokens
 * route in the several-workgroup launch, whose arrival counters and masks
 * live there; every other region is written before it is read. */
int nkt_moe_forward_noalloc(void* handle, const void* hidden_states, const void* router_logits,
                            int num_tokens, void* out, void* stream, char* err, size_t err_len);

/* Library version string (static storage). */
const char* nkt_moe_version(void);

#ifdef __cplusplus
}
#endif

#endif /* NKT_MOE_H */
