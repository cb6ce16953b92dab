// nkt_probe: a torch-free driver of the C ABI (include/nkt_moe.h) for
// hardware-counter runs (rocprofv3 --pmc) and kernel traces of the MoE layer.
//
//   nkt_probe <workload> <tokens> [copies] [passes] [layer]
//
// With "layer" each step is one nkt_moe_forward call (the layer's own launch
// sequence); otherwise the stage entry points run one by one.
//
// workload: qwen3_int4 | qwen3_int8 | mixtral_int4 | qwen15_int8 | tiny_f32.
// It first runs a calibration kernel of known traffic (fp32 negate over
// 256 MiB in and out, three launches), then `copies` distinct weight copies of
// the layer (quantized projections packed by nkt_moe_pack_weight from random
// codes with bf16 scales of 2^-7, dense ones random in the device layout, so
// every launch streams its weights from HBM) and `passes`
// passes of route -> gate_up -> down -> combine over them.  Activations are
// uniform in [-2, 2); router logits are Gaussian with the bench's spread
// (sd 0.905) plus, for the prefill workload qwen3_int8, the Zipf(1.1) bias
// -1.1 ln(e + 1) over expert ids.  Prints one line per pass (with the pass's time per layer, eager
// launches) so a long run shows progress.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include "../../include/nkt_moe.h"

#define CHECK(x)                                                                             \
  do {                                                                                       \
    hipError_t e_ = (x);                                                                     \
    if (e_ != hipSuccess) {                                                                  \
      fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_));      \
      exit(1);                                                                               \
    }                                                                                        \
  } while (0)

#define NKT(x)                                                        \
  do {                                                                \
    if ((x) != NKT_OK) {                                              \
      fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, err); \
      exit(1);                                                        \
    }                                                                 \
  } while (0)

static char err[512];

__device__ __forceinline__ uint32_t mix32(uint64_t x) {
  x ^= x >> 33;
  x *= 0xff51afd7ed558ccdull;
  x ^= x >> 33;
  x *= 0xc4ceb9fe1a85ec53ull;
  x ^= x >> 33;
  return (uint32_t)x;
}

// random bytes (weight codes); n32 words
__global__ void fill_random(uint32_t* p, size_t n32, uint64_t seed) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n32; i += (size_t)gridDim.x * blockDim.x)
    p[i] = mix32(seed * 0x9e3779b97f4a7c15ull + i);
}

// a constant 16-bit pattern (bf16 scales)
__global__ void fill_u16(uint16_t* p, size_t n, uint16_t v) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = v;
}

// activations uniform in [-2, 2): bf16 (or fp32 when f32 != 0)
__global__ void fill_act(void* p, size_t n, uint64_t seed, int f32) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const float v = (float)(mix32(seed * 0x9e3779b97f4a7c15ull + i) >> 8) * (4.0f / 16777216.0f) - 2.0f;
    if (f32)
      ((float*)p)[i] = v;
    else
      ((uint16_t*)p)[i] = (uint16_t)(__float_as_uint(v) >> 16);
  }
}

// calibration kernel: out = -in over n floats (reads and writes n * 4 bytes)
__global__ void neg_kernel(const float* in, float* out, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    out[i] = -in[i];
}

struct Workload {
  const char* name;
  int H, E, k, I, Is, wf, act;
  unsigned flags;
  float zipf;
};

static const Workload kWorkloads[] = {
    {"qwen3_int4", 2048, 128, 8, 768, 0, NKT_WEIGHT_INT4_G128, NKT_DTYPE_BF16, NKT_ROUTE_SOFTMAX | NKT_ROUTE_RENORM, 0.f},
    {"qwen3_int8", 2048, 128, 8, 768, 0, NKT_WEIGHT_INT8_PC, NKT_DTYPE_BF16, NKT_ROUTE_SOFTMAX | NKT_ROUTE_RENORM, 1.1f},
    {"mixtral_int4", 4096, 8, 2, 14336, 0, NKT_WEIGHT_INT4_G128, NKT_DTYPE_BF16, 0u, 0.f},
    {"qwen15_int8", 2048, 60, 4, 1408, 5632, NKT_WEIGHT_INT8_PC, NKT_DTYPE_BF16, NKT_ROUTE_SOFTMAX, 0.f},
    {"tiny_f32", 256, 8, 2, 512, 0, NKT_WEIGHT_F32, NKT_DTYPE_F32, NKT_ROUTE_SOFTMAX | NKT_ROUTE_RENORM, 0.f},
};

static uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

int main(int argc, char** argv) {
  if (argc < 3) {
    fprintf(stderr, "usage: %s <workload> <tokens> [copies=4] [passes=2] [layer]\n", argv[0]);
    return 2;
  }
  const Workload* w = nullptr;
  for (const Workload& c : kWorkloads)
    if (!strcmp(c.name, argv[1])) w = &c;
  if (!w) {
    fprintf(stderr, "unknown workload %s\n", argv[1]);
    return 2;
  }
  const int T = atoi(argv[2]);
  const int copies = argc > 3 ? atoi(argv[3]) : 4;
  const int passes = argc > 4 ? atoi(argv[4]) : 2;
  const bool layer = argc > 5 && !strcmp(argv[5], "layer");
  if (T < 1 || copies < 1 || passes < 1) {
    fprintf(stderr, "tokens, copies and passes must be positive\n");
    return 2;
  }
  hipStream_t st;
  CHECK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));

  // calibration: 256 MiB read and written, three launches
  {
    const size_t n = (size_t)64 << 20;
    float *a, *b;
    CHECK(hipMalloc(&a, n * 4));
    CHECK(hipMalloc(&b, n * 4));
    hipLaunchKernelGGL(fill_act, dim3(4096), dim3(256), 0, st, a, n, 7ull, 1);
    for (int r = 0; r < 3; ++r) hipLaunchKernelGGL(neg_kernel, dim3(8192), dim3(256), 0, st, a, b, n);
    CHECK(hipStreamSynchronize(st));
    CHECK(hipFree(a));
    CHECK(hipFree(b));
    printf("calibration done\n");
    fflush(stdout);
  }

  const int es = w->act == NKT_DTYPE_F32 ? 4 : 2;
  const bool quant = w->wf == NKT_WEIGHT_INT4_G128 || w->wf == NKT_WEIGHT_INT8_PC;
  // one projection's source codes and scales, reused for every pack
  const int max_i = w->I > w->Is ? w->I : w->Is;
  const size_t src_bytes = (size_t)2 * max_i * w->H;
  const size_t src_scale_elems = (size_t)2 * max_i * (w->H / 128 > 1 ? w->H / 128 : 1) + (size_t)w->H * (max_i / 128 + 1);
  void *src = nullptr, *src_scales = nullptr;
  if (quant) {
    CHECK(hipMalloc(&src, src_bytes));
    CHECK(hipMalloc(&src_scales, src_scale_elems * 2));
    hipLaunchKernelGGL(fill_u16, dim3(1024), dim3(256), 0, st, (uint16_t*)src_scales, src_scale_elems,
                       f32_to_bf16(0.0078125f));
  }
  std::vector<void*> handles(copies);
  std::vector<std::vector<void*>> slots(copies, std::vector<void*>(NKT_NUM_SLOTS, nullptr));
  for (int c = 0; c < copies; ++c) {
    handles[c] = nkt_moe_create(w->E, w->k, w->H, w->I, w->Is, w->wf, w->act, w->flags, T, err, sizeof(err));
    if (!handles[c]) {
      fprintf(stderr, "nkt_moe_create: %s\n", err);
      return 1;
    }
    for (int s = 0; s < NKT_NUM_SLOTS; ++s) {
      if (s == NKT_SLOT_ROUTER) continue;
      size_t bytes = 0;
      NKT(nkt_moe_weight_bytes(handles[c], s, &bytes, err, sizeof(err)));
      if (!bytes) continue;
      CHECK(hipMalloc(&slots[c][s], bytes));
      if (s == NKT_SLOT_SHARED_GATE || w->wf == NKT_WEIGHT_F32 || w->wf == NKT_WEIGHT_BF16)
        // dense weights in the activation dtype, uniform in [-2, 2)
        hipLaunchKernelGGL(fill_act, dim3(1024), dim3(256), 0, st, slots[c][s], bytes / es, (uint64_t)(1000 * c + s),
                           es == 4 ? 1 : 0);
    }
    if (quant) {
      // projections: (slot, rows, columns, experts)
      const int proj[4][4] = {{NKT_SLOT_GATE_UP, 2 * w->I, w->H, w->E},
                              {NKT_SLOT_DOWN, w->H, w->I, w->E},
                              {NKT_SLOT_SHARED_GATE_UP, 2 * w->Is, w->H, w->Is > 0 ? 1 : 0},
                              {NKT_SLOT_SHARED_DOWN, w->H, w->Is, w->Is > 0 ? 1 : 0}};
      for (const auto& pr : proj)
        for (int e = 0; e < pr[3]; ++e) {
          const size_t nq = (size_t)pr[1] * pr[2] / (w->wf == NKT_WEIGHT_INT4_G128 ? 2 : 1);
          const size_t ns = (size_t)pr[1] * (w->wf == NKT_WEIGHT_INT4_G128 ? pr[2] / 128 : 1);
          if (nq > src_bytes || ns > src_scale_elems) {
            fprintf(stderr, "source buffer too small\n");
            return 1;
          }
          hipLaunchKernelGGL(fill_random, dim3(4096), dim3(256), 0, st, (uint32_t*)src, nq / 4,
                             (uint64_t)(1000000 * c + 10000 * pr[0] + e));
          NKT(nkt_moe_pack_weight(handles[c], pr[0], e, src, src_scales, slots[c][pr[0]], slots[c][pr[0] + 1], st,
                                  err, sizeof(err)));
        }
    }
    NKT(nkt_moe_bind_weights(handles[c], (const void* const*)slots[c].data(), err, sizeof(err)));
  }
  size_t ws_bytes = 0;
  NKT(nkt_moe_workspace_bytes(handles[0], T, &ws_bytes, err, sizeof(err)));
  void *ws, *x, *logits, *out;
  CHECK(hipMalloc(&ws, ws_bytes));
  CHECK(hipMemset(ws, 0, ws_bytes));  // the workspace's sync area starts at zero
  CHECK(hipMalloc(&x, (size_t)T * w->H * es));
  CHECK(hipMalloc(&out, (size_t)T * w->H * es));
  CHECK(hipMalloc(&logits, (size_t)T * w->E * es));
  hipLaunchKernelGGL(fill_act, dim3(1024), dim3(256), 0, st, x, (size_t)T * w->H, 11ull, es == 4 ? 1 : 0);
  {
    std::vector<uint8_t> host((size_t)T * w->E * es);
    uint64_t r = 0x243f6a8885a308d3ull;
    for (int t = 0; t < T; ++t)
      for (int e = 0; e < w->E; ++e) {
        // Gaussian, sd 0.905: the spread of x . gate for x ~ N(0, 1) and
        // gate rows ~ N(0, 0.02^2) over H = 2048, as the bench's logits
        r = r * 6364136223846793005ull + 1442695040888963407ull;
        const float u1 = ((float)(r >> 40) + 0.5f) * (1.0f / 16777216.0f);
        r = r * 6364136223846793005ull + 1442695040888963407ull;
        const float u2 = (float)(r >> 40) * (1.0f / 16777216.0f);
        float v = 0.905f * sqrtf(-2.0f * logf(u1)) * cosf(6.28318530718f * u2);
        if (w->zipf > 0.f) v -= w->zipf * logf((float)e + 1.0f);
        if (es == 4)
          memcpy(&host[((size_t)t * w->E + e) * 4], &v, 4);
        else {
          const uint16_t b = f32_to_bf16(v);
          memcpy(&host[((size_t)t * w->E + e) * 2], &b, 2);
        }
      }
    CHECK(hipMemcpyAsync(logits, host.data(), host.size(), hipMemcpyHostToDevice, st));
    CHECK(hipStreamSynchronize(st));
  }
  printf("%s T=%d: %d copies, %zu workspace bytes\n", w->name, T, copies, ws_bytes);
  fflush(stdout);
  hipEvent_t ev0, ev1;
  CHECK(hipEventCreate(&ev0));
  CHECK(hipEventCreate(&ev1));
  for (int p = 0; p < passes; ++p) {
    CHECK(hipEventRecord(ev0, st));
    for (int c = 0; c < copies; ++c) {
      if (layer) {
        NKT(nkt_moe_forward(handles[c], x, logits, T, out, ws, ws_bytes, st, err, sizeof(err)));
        continue;
      }
      NKT(nkt_moe_route(handles[c], logits, T, ws, ws_bytes, st, err, sizeof(err)));
      NKT(nkt_moe_experts_phase(handles[c], 0, x, T, ws, ws_bytes, st, err, sizeof(err)));
      NKT(nkt_moe_experts_phase(handles[c], 1, x, T, ws, ws_bytes, st, err, sizeof(err)));
      if (w->Is > 0) NKT(nkt_moe_shared(handles[c], x, T, ws, ws_bytes, st, err, sizeof(err)));
      NKT(nkt_moe_combine(handles[c], T, out, ws, ws_bytes, st, err, sizeof(err)));
    }
    CHECK(hipEventRecord(ev1, st));
    CHECK(hipStreamSynchronize(st));
    float ms = 0.f;
    CHECK(hipEventElapsedTime(&ms, ev0, ev1));
    printf("pass %d done: %.2f us per layer (eager launches)\n", p, 1000.0f * ms / copies);
    fflush(stdout);
  }
  CHECK(hipEventDestroy(ev0));
  CHECK(hipEventDestroy(ev1));
  for (int c = 0; c < copies; ++c) {
    for (void* s : slots[c])
      if (s) CHECK(hipFree(s));
    nkt_moe_destroy(handles[c]);
  }
  if (src) CHECK(hipFree(src));
  if (src_scales) CHECK(hipFree(src_scales));
  CHECK(hipFree(ws));
  CHECK(hipFree(x));
  CHECK(hipFree(out));
  CHECK(hipFree(logits));
  CHECK(hipStreamDestroy(st));
  printf("probe done\n");
  return 0;
}
