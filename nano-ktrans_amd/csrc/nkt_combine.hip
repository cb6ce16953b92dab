// K4: shared-expert sigmoid gate, sigmoid(x . g) per token
//     (nano_ktrans/models/mixtral.py:170-179, 215-218).
// K5: un-permute and weighted combine.  For every token the k expert outputs
//     are added in ascending expert id (the visiting order of
//     nano_ktrans/layers/hybrid_moe.py:3512-3533 and cpu_moe.py:515-536),
//     in fp32, then the gated shared expert, then one rounding to the output
//     dtype.  No atomics: each output element is owned by one thread.
#include "nkt_common.h"
#include "nkt_internal.h"

namespace nkt {

__global__ void __launch_bounds__(256) shared_gate_kernel(const void* __restrict__ x,
                                                          const void* __restrict__ gw,
                                                          int act_bf16, int T, int H,
                                                          float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  float s = 0.f;
  if (act_bf16) {
    const uint16_t* xr = (const uint16_t*)x + (int64_t)t * H;
    const uint16_t* g = (const uint16_t*)gw;
    for (int i = lane; i < H; i += 64) s += bf16_bits_to_f32(xr[i]) * bf16_bits_to_f32(g[i]);
  } else {
    const float* xr = (const float*)x + (int64_t)t * H;
    const float* g = (const float*)gw;
    for (int i = lane; i < H; i += 64) s += xr[i] * g[i];
  }
  s = wave_sum_butterfly(s);
  if (lane == 0) out[t] = 1.0f / (1.0f + __expf(-s));
}

__global__ void __launch_bounds__(256) combine_kernel(
    const float* __restrict__ y, const int32_t* __restrict__ ids, const float* __restrict__ w,
    const int32_t* __restrict__ inv, const float* __restrict__ y_shared,
    const float* __restrict__ shared_gate, int num_tokens, int k, int H, void* __restrict__ out,
    int out_bf16) {
  const int t = blockIdx.x;
  // order the token's slots by expert id: rank[j] = #{i : id_i < id_j}
  // (ids of one token are distinct), then gather by rank with static indices
  int sid[kMaxTopK], spos[kMaxTopK], rank[kMaxTopK];
  float sw[kMaxTopK];
#pragma unroll
  for (int j = 0; j < kMaxTopK; ++j) {
    sid[j] = 0x7fffffff;
    spos[j] = 0;
    sw[j] = 0.f;
    if (j < k) {
      sid[j] = ids[(int64_t)t * k + j];
      // positions index y [T*k, H]; keep a corrupt entry from reading outside it
      spos[j] = min(max(inv[(int64_t)t * k + j], 0), num_tokens * k - 1);
      sw[j] = w[(int64_t)t * k + j];
    }
  }
#pragma unroll
  for (int j = 0; j < kMaxTopK; ++j) {
    int r = 0;
#pragma unroll
    for (int i = 0; i < kMaxTopK; ++i) r += (sid[i] < sid[j]) ? 1 : 0;
    rank[j] = r;
  }
  int order_pos[kMaxTopK];
  float order_w[kMaxTopK];
#pragma unroll
  for (int r = 0; r < kMaxTopK; ++r) {
    int p = 0;
    float wt = 0.f;
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) {
      if (j < k && rank[j] == r) {
        p = spos[j];
        wt = sw[j];
      }
    }
    order_pos[r] = p;
    order_w[r] = wt;
  }
  const int n = k;
  const float sg = shared_gate ? shared_gate[t] : 0.f;
  const int H4 = H / 4;
  for (int c = threadIdx.x; c < H4; c += blockDim.x) {
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) {
      if (j < n) {
        const f32x4 v = *(const f32x4*)(y + (int64_t)order_pos[j] * H + 4 * c);
        acc += order_w[j] * v;
      }
    }
    if (y_shared) {
      const f32x4 v = *(const f32x4*)(y_shared + (int64_t)t * H + 4 * c);
      acc += sg * v;
    }
    if (out_bf16) {
      u32x2 pk;
      pk[0] = pack_bf16x2(acc[0], acc[1]);
      pk[1] = pack_bf16x2(acc[2], acc[3]);
      *(u32x2*)((uint16_t*)out + (int64_t)t * H + 4 * c) = pk;
    } else {
      *(f32x4*)((float*)out + (int64_t)t * H + 4 * c) = acc;
    }
  }
}

hipError_t launch_shared_gate(const void* x, const void* gate_w, int act_bf16, int T, int H,
                              float* gate_out, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  hipLaunchKernelGGL(shared_gate_kernel, dim3((T + 3) / 4), dim3(256), 0, stream, x, gate_w,
                     act_bf16, T, H, gate_out);
  return hipGetLastError();
}

hipError_t launch_combine(const float* y, const int32_t* ids, const float* w, const int32_t* inv,
                          const float* y_shared, const float* shared_gate, int T, int k, int H,
                          void* out, int out_bf16, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  hipLaunchKernelGGL(combine_kernel, dim3(T), dim3(256), 0, stream, y, ids, w, inv, y_shared,
                     shared_gate, T, k, H, out, out_bf16);
  return hipGetLastError();
}

}  // namespace nkt
