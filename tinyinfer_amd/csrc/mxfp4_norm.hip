// RMSNorm of the MLP's input rows: the decoder layer's post_attention_layernorm
// in front of the MXFP4 MLP (tinyinfer/models/qwen3.py:210-216 ->
// tinyinfer/layers/layernorm.py:15-23 -> tinyinfer/csrc/rmsnorm.cu:10-54).
//
// Per row: s = sum(x^2) in fp32, inv = rsqrt(s / hidden + eps), out =
// round(w * x * inv) with the reference's evaluation order ((w * x) * inv).
// One 256-thread workgroup per row, 16-byte chunks (8 activations); the sum
// is a fixed-order tree (per thread, then over the wave, then over the four
// waves), so a row's result does not depend on scheduling.  The streaming
// gate_up kernel applies the same formula to its LDS copy of x when the MLP
// is called with a norm weight (mxfp4_stream.hip).
#include "mxfp4_common.hpp"
#include "mxfp4_launch.hpp"

namespace tinyinfer {

namespace {

constexpr int kNormThreads = 256;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <int DT>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                               const uint16_t* __restrict__ w, float eps,
                                                               int64_t hidden, uint16_t* __restrict__ out) {
  __shared__ float part[kNormThreads / 64];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * hidden;
  uint16_t* orow = out + row * hidden;
  const int64_t chunks = hidden / 8;
  float s = 0.f;
  for (int64_t c = threadIdx.x; c < chunks; c += kNormThreads) {
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xr + 8 * c);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = act_to_f32<DT>((uint16_t)(v[j] & 0xffffu)), hi = act_to_f32<DT>((uint16_t)(v[j] >> 16));
      s += lo * lo;
      s += hi * hi;
    }
  }
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += part[i];
  const float inv = rsqrtf(tot / (float)hidden + eps);
  for (int64_t c = threadIdx.x; c < chunks; c += kNormThreads) {
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xr + 8 * c);
    const u32x4_t g = *reinterpret_cast<const u32x4_t*>(w + 8 * c);
    u32x4_t o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = act_to_f32<DT>((uint16_t)(g[j] & 0xffffu)) * act_to_f32<DT>((uint16_t)(v[j] & 0xffffu)) * inv;
      const float hi = act_to_f32<DT>((uint16_t)(g[j] >> 16)) * act_to_f32<DT>((uint16_t)(v[j] >> 16)) * inv;
      o[j] = (uint32_t)f32_to_act<DT>(lo) | ((uint32_t)f32_to_act<DT>(hi) << 16);
    }
    *reinterpret_cast<u32x4_t*>(orow + 8 * c) = o;
  }
}

}  // namespace

hipError_t launch_rmsnorm(const void* x, const void* w, float eps, int64_t n, int64_t hidden, void* out, int dtype,
                          hipStream_t stream) {
  if (n < 1 || hidden < 8 || hidden % 8 != 0 || n > 0x7fffffff) return hipErrorInvalidValue;
  const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                       reinterpret_cast<uintptr_t>(out);
  if (al & 15u) return hipErrorInvalidValue;
  const uint16_t* xs = static_cast<const uint16_t*>(x);
  const uint16_t* ws = static_cast<const uint16_t*>(w);
  uint16_t* os = static_cast<uint16_t*>(out);
  if (dtype == kBF16) rmsnorm_kernel<kBF16><<<(unsigned)n, kNormThreads, 0, stream>>>(xs, ws, eps, hidden, os);
  else rmsnorm_kernel<kF16><<<(unsigned)n, kNormThreads, 0, stream>>>(xs, ws, eps, hidden, os);
  return hipGetLastError();
}

}  // namespace tinyinfer
