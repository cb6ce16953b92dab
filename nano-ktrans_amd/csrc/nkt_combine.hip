// K4: shared-expert sigmoid gate, sigmoid(x . g) per token
//     (nano_ktrans/models/mixtral.py:170-179, 215-218).
// K5: un-permute and weighted combine.  For every token the k expert outputs
//     are added in ascending expert id (the visiting order of
//     nano_ktrans/layers/hybrid_moe.py:3512-3533 and cpu_moe.py:515-536),
//     in fp32, then the sum an offload backend returned for the experts that
//     are not HBM-resident (hybrid_moe.py:3563-3570; their slots are skipped),
//     then the gated shared expert, then (decoder-block form) the residual
//     stream, then one rounding to the output dtype.  No atomics: each output
//     element is owned by one thread.
// Decoder-block form: RMSNorm of the residual stream before the path
//     (nano_ktrans/layers/norm.py:11-17), one wave per token.
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
  const float v = shared_gate_value(x, gw, act_bf16, t, H, lane);
  if (lane == 0) out[t] = v;
}

// One workgroup per (token, 1024-column slice); one thread per 4 columns.
// y holds the k expert rows of token t at rows t k .. t k + k - 1 (pair
// order; inv == nullptr) or at rows inv[t k + j] (position order); in pair
// order every load is issued at once.  The terms are added in ascending
// expert id through the thread's own LDS slots.
// The end of one token's four output columns: + the offload backend's sum,
// + gate x shared expert row, + the residual, one rounding, store.
// (shared: whether the gated shared expert row vs is added; by value, so
// the row stays in registers)
__device__ __forceinline__ void combine_tail(f32x4 acc, int t, int col, int H, const void* extra, bool shared,
                                             f32x4 vs, float sg, const void* residual, void* out, int out_bf16) {
#pragma clang fp contract(off)
  const int64_t o = (int64_t)t * H + col;
  if (extra) {
    if (out_bf16)
      acc += bf16x4_to_f32(*(const u32x2*)((const uint16_t*)extra + o));
    else
      acc += *(const f32x4*)((const float*)extra + o);
  }
  if (shared) acc += sg * vs;
  if (residual) {
    if (out_bf16)
      acc += bf16x4_to_f32(*(const u32x2*)((const uint16_t*)residual + o));
    else
      acc += *(const f32x4*)((const float*)residual + o);
  }
  if (out_bf16) {
    u32x2 pk;
    pk[0] = pack_bf16x2(acc[0], acc[1]);
    pk[1] = pack_bf16x2(acc[2], acc[3]);
    *(u32x2*)((uint16_t*)out + o) = pk;
  } else {
    *(f32x4*)((float*)out + o) = acc;
  }
}

template <int K>
__global__ void __launch_bounds__(256) combine_kernel(
    const float* __restrict__ y, const int32_t* __restrict__ ids, const float* __restrict__ w,
    const int32_t* __restrict__ inv, const float* __restrict__ y_shared, const float* __restrict__ shared_gate, const uint8_t* __restrict__ resident,
    const void* __restrict__ extra, const void* __restrict__ residual, int num_tokens, int H,
    void* __restrict__ out, int out_bf16, int sh_rows) {
  __shared__ f32x4 terms[K][256];
  const int t = blockIdx.x;
  const int c = blockIdx.y * blockDim.x + threadIdx.x;  // float4 column index
  if (4 * c >= H) return;
  // every load first: the k rows, the gated shared row, ids and weights
  f32x4 v[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    // a corrupt position never reads outside y
    const int64_t row = inv ? min(max(inv[(int64_t)t * K + j], 0), num_tokens * K - 1) : (int64_t)t * K + j;
    v[j] = *(const f32x4*)(y + row * H + 4 * c);
  }
  f32x4 vs = f32x4{0.f, 0.f, 0.f, 0.f};
  float sg = 0.f;
  if (y_shared) {
    // the shared row (or its chunks' rows, added in chunk order)
    vs = *(const f32x4*)(y_shared + (int64_t)t * H + 4 * c);
    for (int j = 1; j < sh_rows; ++j) vs += *(const f32x4*)(y_shared + ((int64_t)j * num_tokens + t) * H + 4 * c);
    sg = shared_gate[t];
  }
  int sid[K];
  float sw[K];
  bool sres[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    sid[j] = ids[(int64_t)t * K + j];
    sw[j] = w[(int64_t)t * K + j];
    sres[j] = resident ? resident[sid[j]] != 0 : true;
  }
  // slot j's term goes to place rank_j = #{i : id_i < id_j} (ids of one token
  // are distinct); slots of experts that are not resident have no y row this
  // call: their (stale) values are selected away, never multiplied
  const f32x4 zero = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < K; ++j) {
    int r = 0;
#pragma unroll
    for (int i = 0; i < K; ++i) r += (sid[i] < sid[j]) ? 1 : 0;
    terms[r][threadIdx.x] = sres[j] ? sw[j] * v[j] : zero;
  }
  f32x4 acc = terms[0][threadIdx.x];
#pragma unroll
  for (int r = 1; r < K; ++r) acc += terms[r][threadIdx.x];
  combine_tail(acc, t, 4 * c, H, extra, y_shared != nullptr, vs, sg, residual, out, out_bf16);
}

// The same sum over the prefill layer's compact y (fp16 rows, one fp32
// inverse scale per row and 256-column slab in yscale), eight columns per
// thread so every row load is 16 bytes: each half of four columns goes
// through the thread's LDS slots in turn, with combine_kernel's order and
// arithmetic on the expanded values.  The shared row: the sum of its
// sh_rows part rows (the shared down's K parts) in part order.
template <int K>
__global__ void __launch_bounds__(256) combine16_kernel(
    const uint16_t* __restrict__ y16, const float* __restrict__ yscale, const int32_t* __restrict__ ids,
    const float* __restrict__ w, const int32_t* __restrict__ inv, const float* __restrict__ y_shared,
    const float* __restrict__ shared_gate, const uint8_t* __restrict__ resident, const void* __restrict__ extra,
    const void* __restrict__ residual, int num_tokens, int H, void* __restrict__ out, int out_bf16, int sh_rows) {
  __shared__ f32x4 terms[K][256];
  const int t = blockIdx.x;
  const int c = blockIdx.y * blockDim.x + threadIdx.x;  // 8-column group
  if (8 * c >= H) return;
  u32x4 hv[K];
  float sc[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    const int64_t row = inv ? min(max(inv[(int64_t)t * K + j], 0), num_tokens * K - 1) : (int64_t)t * K + j;
    hv[j] = *(const u32x4*)(y16 + row * H + 8 * c);
    sc[j] = yscale[row * (H / 256) + (8 * c) / 256];
  }
  int sid[K];
  float sw[K];
  bool sres[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    sid[j] = ids[(int64_t)t * K + j];
    sw[j] = w[(int64_t)t * K + j];
    sres[j] = resident ? resident[sid[j]] != 0 : true;
  }
  int rk[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    int r = 0;
#pragma unroll
    for (int i = 0; i < K; ++i) r += (sid[i] < sid[j]) ? 1 : 0;
    rk[j] = r;
  }
  const float sg = y_shared ? shared_gate[t] : 0.f;
  const f32x4 zero = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int half = 0; half < 2; ++half) {
#pragma unroll
    for (int j = 0; j < K; ++j) {
      f32x4 v;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t word = hv[j][2 * half + q];
        v[2 * q] = (float)__builtin_bit_cast(_Float16, (uint16_t)(word & 0xffffu));
        v[2 * q + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(word >> 16));
      }
      v *= sc[j];
      terms[rk[j]][threadIdx.x] = sres[j] ? sw[j] * v : zero;
    }
    f32x4 acc = terms[0][threadIdx.x];
#pragma unroll
    for (int r = 1; r < K; ++r) acc += terms[r][threadIdx.x];
    const int col = 8 * c + 4 * half;
    f32x4 vs = zero;
    if (y_shared) {
      // the shared row (or its parts' rows, added in order)
      vs = *(const f32x4*)(y_shared + (int64_t)t * H + col);
      for (int j = 1; j < sh_rows; ++j) vs += *(const f32x4*)(y_shared + ((int64_t)j * num_tokens + t) * H + col);
    }
    combine_tail(acc, t, col, H, extra, y_shared != nullptr, vs, sg, residual, out, out_bf16);
  }
}

// RMSNorm as nano_ktrans/layers/norm.py:11-17 computes it: in fp32,
// x * rsqrt(mean(x^2) + eps), rounded to bf16, then times the bf16 weight,
// rounded again.  Lane l holds the 8-column chunks l, l + 64, ...; the sum of
// squares adds a lane's chunks in order, then a fixed butterfly.
constexpr int kNormMaxChunks = 8;  // rows up to 4096 wide stay in registers

__global__ void __launch_bounds__(256) rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                      const uint16_t* __restrict__ w, float eps, int T,
                                                      int H, uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const uint16_t* xr = x + (int64_t)t * H;
  uint16_t* orow = out + (int64_t)t * H;
  if (H <= kNormMaxChunks * 512) {
    // the row and the weight in registers, every load issued at once; the
    // same summation order as below (chunks past H add +0)
    u32x4 v[kNormMaxChunks], g[kNormMaxChunks];
#pragma unroll
    for (int ch = 0; ch < kNormMaxChunks; ++ch) {
      const int c = lane * 8 + ch * 512;
      v[ch] = c < H ? *(const u32x4*)(xr + c) : u32x4{0u, 0u, 0u, 0u};
      g[ch] = c < H ? *(const u32x4*)(w + c) : u32x4{0u, 0u, 0u, 0u};
    }
    float ss = 0.f;
#pragma unroll
    for (int ch = 0; ch < kNormMaxChunks; ++ch) {
      if (lane * 8 + ch * 512 >= H) continue;
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const float a = __uint_as_float(v[ch][h] << 16), b = __uint_as_float(v[ch][h] & 0xffff0000u);
        ss += a * a;
        ss += b * b;
      }
    }
    ss = wave_sum_butterfly(ss);
    const float inv = 1.0f / sqrtf(ss / (float)H + eps);
#pragma unroll
    for (int ch = 0; ch < kNormMaxChunks; ++ch) {
      const int c = lane * 8 + ch * 512;
      if (c >= H) continue;
      u32x4 o;
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const float a = bf16_round(__uint_as_float(v[ch][h] << 16) * inv);
        const float b = bf16_round(__uint_as_float(v[ch][h] & 0xffff0000u) * inv);
        o[h] = pack_bf16x2(a * __uint_as_float(g[ch][h] << 16), b * __uint_as_float(g[ch][h] & 0xffff0000u));
      }
      *(u32x4*)(orow + c) = o;
    }
    return;
  }
  float ss = 0.f;
  for (int c = lane * 8; c < H; c += 512) {
    const u32x4 v = *(const u32x4*)(xr + c);
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const float a = __uint_as_float(v[h] << 16), b = __uint_as_float(v[h] & 0xffff0000u);
      ss += a * a;
      ss += b * b;
    }
  }
  ss = wave_sum_butterfly(ss);
  const float inv = 1.0f / sqrtf(ss / (float)H + eps);
  for (int c = lane * 8; c < H; c += 512) {
    const u32x4 v = *(const u32x4*)(xr + c);
    const u32x4 g = *(const u32x4*)(w + c);
    u32x4 o;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const float a = bf16_round(__uint_as_float(v[h] << 16) * inv);
      const float b = bf16_round(__uint_as_float(v[h] & 0xffff0000u) * inv);
      o[h] = pack_bf16x2(a * __uint_as_float(g[h] << 16), b * __uint_as_float(g[h] & 0xffff0000u));
    }
    *(u32x4*)(orow + c) = o;
  }
}

hipError_t launch_rmsnorm(const void* x, const void* w, float eps, int T, int H, void* out, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  if (H % 8 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((T + 3) / 4), dim3(256), 0, stream, (const uint16_t*)x,
                     (const uint16_t*)w, eps, T, H, (uint16_t*)out);
  return hipGetLastError();
}

hipError_t launch_shared_gate(const void* x, const void* gate_w, int act_bf16, int T, int H,
                              float* gate_out, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  hipLaunchKernelGGL(shared_gate_kernel, dim3((T + 3) / 4), dim3(256), 0, stream, x, gate_w,
                     act_bf16, T, H, gate_out);
  return hipGetLastError();
}

hipError_t launch_combine(const float* y, const int32_t* ids, const float* w, const int32_t* inv, const float* y_shared, const float* shared_gate, const uint8_t* resident,
                          const void* extra, const void* residual, int T, int k, int H, void* out,
                          int out_bf16, hipStream_t stream, const uint16_t* y16, const float* yscale, int sh_rows) {
  if (T <= 0) return hipSuccess;
  if (y16 && (!yscale || H % 256 != 0)) return hipErrorInvalidValue;
  if (sh_rows < 1 || sh_rows > kMaxSharedChunks || (sh_rows > 1 && !y_shared)) return hipErrorInvalidValue;
  dim3 grid(T, (H / 4 + 255) / 256), grid16(T, (H / 8 + 255) / 256), block(256);
#define NKT_COMBINE_CASE(KK)                                                                              \
  case KK:                                                                                                \
    if (y16)                                                                                              \
      hipLaunchKernelGGL(combine16_kernel<KK>, grid16, block, 0, stream, y16, yscale, ids, w, inv, y_shared, \
                         shared_gate, resident, extra, residual, T, H, out, out_bf16, sh_rows);           \
    else                                                                                                  \
      hipLaunchKernelGGL(combine_kernel<KK>, grid, block, 0, stream, y, ids, w, inv, y_shared, shared_gate,  \
                         resident, extra, residual, T, H, out, out_bf16, sh_rows);                        \
    break;
  switch (k) {
    NKT_COMBINE_CASE(1)
    NKT_COMBINE_CASE(2)
    NKT_COMBINE_CASE(3)
    NKT_COMBINE_CASE(4)
    NKT_COMBINE_CASE(5)
    NKT_COMBINE_CASE(6)
    NKT_COMBINE_CASE(7)
    NKT_COMBINE_CASE(8)
    NKT_COMBINE_CASE(9)
    NKT_COMBINE_CASE(10)
    NKT_COMBINE_CASE(11)
    NKT_COMBINE_CASE(12)
    NKT_COMBINE_CASE(13)
    NKT_COMBINE_CASE(14)
    NKT_COMBINE_CASE(15)
    NKT_COMBINE_CASE(16)
    default:
      return hipErrorInvalidValue;
  }
#undef NKT_COMBINE_CASE
  return hipGetLastError();
}

}  // namespace nkt
