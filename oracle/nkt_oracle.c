/*
 * CPU oracle for the MoE router (softmax / top-k / renormalise) and the
 * token-by-expert grouping.  TEST INFRASTRUCTURE ONLY: this file is the
 * checker for the HIP kernels.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product never links it.
 *
 * What it restates (reference paths relative to the nano-ktrans tree):
 *   nano_ktrans/layers/hybrid_moe.py:3321-3329   routing block of HybridMoE.forward
 *       softmax arches:  p = softmax(logits, dtype=fp32).to(logits.dtype)
 *                        w, ids = topk(p, k);  if renorm: w = w / w.sum(-1)
 *       Mixtral arch:    w, ids = topk(logits, k);  w = softmax(w)
 *   nano_ktrans/layers/hybrid_moe.py:3384-3386, 3512-3526 and
 *   nano_ktrans/kernels/cpu_moe.py:515-523       per-expert token lists:
 *       experts visited in ascending id, tokens in ascending order.
 *
 * The reference leaves four things to torch's implementation; this oracle
 * (and the HIP kernel) fix them explicitly so that both sides agree bit for
 * bit:
 *   1. exp: range reduction x = n*ln2 + r (Cody & Waite split, fused
 *      multiply-adds), exp(r) by the degree-7 Taylor polynomial in Horner
 *      form, then an exact power-of-two scaling (two steps below 2^-126 so
 *      that subnormal results are rounded once).
 *   2. softmax reduction order: value i sits in lane i % 64 (64-lane
 *      wavefront); each lane adds its values in ascending i; the 64 lane sums
 *      are reduced by the xor butterfly (offsets 32, 16, 8, 4, 2, 1).
 *   3. top-k order: value descending, ties broken by the lower expert id;
 *      -0.0 counts as +0.0, NaN as the largest value.
 *   4. k-way sums (renormalisation, Mixtral softmax) add slots 0..k-1 in
 *      order; bf16 results are rounded to nearest-even from fp32 after every
 *      operation that torch performs in the logits dtype.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* ---- bf16 helpers (round to nearest even, NaN kept quiet) ------------- */
static float u32_as_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f32_as_u32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float orc_bf16_round(float x) {
    uint32_t u = f32_as_u32(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return u32_as_f32((u | 0x00400000u) & 0xffff0000u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return u32_as_f32(u & 0xffff0000u);
}

/* ---- exp ---------------------------------------------------------------- */
#define ORC_LOG2E   0x1.715476p+0f     /* nearest float to 1/ln 2            */
#define ORC_LN2_HI  0x1.62e430p-1f     /* nearest float to ln 2              */
#define ORC_LN2_LO  -0x1.05c610p-29f   /* nearest float to ln 2 - ORC_LN2_HI */
#define ORC_C2 0x1.000000p-1f          /* 1/2!  */
#define ORC_C3 0x1.555556p-3f          /* 1/3!  */
#define ORC_C4 0x1.555556p-5f          /* 1/4!  */
#define ORC_C5 0x1.111112p-7f          /* 1/5!  */
#define ORC_C6 0x1.6c16c2p-10f         /* 1/6!  */
#define ORC_C7 0x1.a01a02p-13f         /* 1/7!  */

float orc_expf(float x) {
    if (x != x) return x;
    if (x > 89.0f) return INFINITY;
    if (x < -110.0f) x = -110.0f;
    float t = x * ORC_LOG2E;
    float n = rintf(t);
    float r = fmaf(-n, ORC_LN2_HI, x);
    r = fmaf(-n, ORC_LN2_LO, r);
    float p = ORC_C7;
    p = fmaf(p, r, ORC_C6);
    p = fmaf(p, r, ORC_C5);
    p = fmaf(p, r, ORC_C4);
    p = fmaf(p, r, ORC_C3);
    p = fmaf(p, r, ORC_C2);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int ni = (int)n;
    if (ni > 127) return (p * u32_as_f32(254u << 23)) * 2.0f;
    if (ni >= -126) return p * u32_as_f32((uint32_t)(ni + 127) << 23);
    return (p * u32_as_f32((uint32_t)(ni + 127 + 64) << 23)) * u32_as_f32((uint32_t)(127 - 64) << 23);
}

void orc_expf_array(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_expf(x[i]);
}

/* ---- softmax over one row with the wavefront reduction order ------------ */
void orc_softmax_row(const float* x, int E, float* p) {
    float m = -INFINITY;
    for (int i = 0; i < E; ++i) m = (x[i] > m) ? x[i] : m;
    float lane[64];
    for (int l = 0; l < 64; ++l) lane[l] = 0.0f;
    for (int l = 0; l < 64; ++l) {
        int first = 1;
        for (int i = l; i < E; i += 64) {
            float e = orc_expf(x[i] - m);
            p[i] = e;
            if (first) { lane[l] = e; first = 0; }
            else lane[l] = lane[l] + e;
        }
    }
    for (int off = 32; off >= 1; off >>= 1)
        for (int l = 0; l < off; ++l) lane[l] = lane[l] + lane[l + off];
    float s = lane[0];
    for (int i = 0; i < E; ++i) p[i] = p[i] / s;
}

/* ---- ordering key: value descending, id ascending ----------------------- */
static uint64_t orc_key(float v, int id) {
    v = v + 0.0f;                                 /* -0.0 -> +0.0 */
    uint32_t u = f32_as_u32(v);
    if (v != v) u = 0x7fc00000u;                  /* NaN is the largest */
    uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - (uint32_t)id);
}

static void orc_topk(const float* v, int E, int k, int32_t* ids, float* vals) {
    /* selection by repeated maximum over the (value, -id) key */
    uint64_t taken_mask_words[(1024 + 63) / 64];
    memset(taken_mask_words, 0, sizeof(taken_mask_words));
    for (int j = 0; j < k; ++j) {
        uint64_t best = 0; int best_id = -1;
        for (int e = 0; e < E; ++e) {
            if (taken_mask_words[e >> 6] & (1ull << (e & 63))) continue;
            uint64_t key = orc_key(v[e], e);
            if (best_id < 0 || key > best) { best = key; best_id = e; }
        }
        taken_mask_words[best_id >> 6] |= 1ull << (best_id & 63);
        ids[j] = best_id;
        vals[j] = v[best_id];
    }
}

/*
 * Route T tokens.  logits: fp32 array [T, E] (bf16 logits are passed
 * upcast, exactly).  Outputs: ids [T, k] int32 in top-k order, weights
 * [T, k] fp32 (bf16-valued when bf16 != 0).  Returns 0, or -1 on bad args.
 */
int orc_route(const float* logits, int T, int E, int k, int use_softmax, int renorm, int bf16,
              int32_t* ids, float* w) {
    if (E < 1 || E > 1024 || k < 1 || k > E || T < 0) return -1;
    float p[1024];
    for (int t = 0; t < T; ++t) {
        const float* row = logits + (int64_t)t * E;
        int32_t* id = ids + (int64_t)t * k;
        float* wt = w + (int64_t)t * k;
        if (use_softmax) {
            orc_softmax_row(row, E, p);
            if (bf16)
                for (int e = 0; e < E; ++e) p[e] = orc_bf16_round(p[e]);
            orc_topk(p, E, k, id, wt);
            if (renorm) {
                float s = wt[0];
                for (int j = 1; j < k; ++j) s = s + wt[j];
                if (bf16) s = orc_bf16_round(s);
                for (int j = 0; j < k; ++j) {
                    float q = wt[j] / s;
                    wt[j] = bf16 ? orc_bf16_round(q) : q;
                }
            }
        } else {
            float sel[1024];
            orc_topk(row, E, k, id, sel);
            float m = sel[0];
            float s = 0.0f;
            for (int j = 0; j < k; ++j) {
                wt[j] = orc_expf(sel[j] - m);
                s = (j == 0) ? wt[j] : s + wt[j];
            }
            for (int j = 0; j < k; ++j) {
                float q = wt[j] / s;
                wt[j] = bf16 ? orc_bf16_round(q) : q;
            }
        }
    }
    return 0;
}

/*
 * Group the T*k (token, slot) pairs by expert.  Pair index p = t*k + j.
 * counts[e]   = number of pairs routed to e
 * offsets[e]  = exclusive prefix sum of counts (E+1 entries)
 * perm[pos]   = p, ordered by (expert ascending, token ascending)
 * inv[p]      = pos such that perm[pos] = p
 * Returns 0, or -1 when an id is out of range.
 */
int orc_group(const int32_t* ids, int T, int k, int E, int32_t* counts, int32_t* offsets,
              int32_t* perm, int32_t* inv) {
    int64_t P = (int64_t)T * k;
    for (int e = 0; e < E; ++e) counts[e] = 0;
    for (int64_t p = 0; p < P; ++p) {
        if (ids[p] < 0 || ids[p] >= E) return -1;
        counts[ids[p]]++;
    }
    offsets[0] = 0;
    for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int32_t fill[1024];
    for (int e = 0; e < E; ++e) fill[e] = offsets[e];
    for (int64_t p = 0; p < P; ++p) {
        int e = ids[p];
        perm[fill[e]] = (int32_t)p;
        inv[p] = fill[e];
        fill[e]++;
    }
    return 0;
}
