// MXFP4 codec kernels: device dequantization and quantization.
//
// dequant  : reference dequantize_chunk (quantize_mxfp4.py:67-85) / GPU decode
//            (utils.h:87-127); bit-exact, uses the same dq8_bf16 decode as the
//            MLP kernels so its exhaustive test covers theirs.
// quantize : reference quantize_chunk (quantize_mxfp4.py:28-64), bit-exact,
//            including the exponent choice of torch's fp32 log2 (which is
//            correctly rounded) at powers of two.
//
// One thread per 32-element block; adjacent threads touch adjacent blocks,
// so a wave reads/writes one contiguous span.
#include "mxfp4_common.hpp"
#include "mxfp4_launch.hpp"

namespace tinyinfer {

namespace {

constexpr int kCodecThreads = 256;

template <int OUT>
__global__ __launch_bounds__(kCodecThreads) void dequant_kernel(const uint8_t* __restrict__ packed,
                                                                const uint8_t* __restrict__ scale,
                                                                int64_t nblocks,
                                                                void* __restrict__ out) {
  for (int64_t blk = blockIdx.x * (int64_t)kCodecThreads + threadIdx.x; blk < nblocks;
       blk += (int64_t)gridDim.x * kCodecThreads) {
    const u32x4_t w = *reinterpret_cast<const u32x4_t*>(packed + blk * 16);
    const uint32_t b = scale[blk];
    if constexpr (OUT == kBF16) {
      u32x4_t* dst = reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(out) + blk * 32);
      dst[0] = dq8_bf16(w.x, b);
      dst[1] = dq8_bf16(w.y, b);
      dst[2] = dq8_bf16(w.z, b);
      dst[3] = dq8_bf16(w.w, b);
    } else {
      float* dst = static_cast<float*>(out) + blk * 32;
      float v[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        dq8_f32(w[j], b, v);
        f32x4_t* d4 = reinterpret_cast<f32x4_t*>(dst + 8 * j);
        d4[0] = f32x4_t{v[0], v[1], v[2], v[3]};
        d4[1] = f32x4_t{v[4], v[5], v[6], v[7]};
      }
    }
  }
}

// ceil(log2(y)) where log2 is evaluated as a correctly rounded fp32 function,
// y > 0 finite (normal or subnormal).
//
// Write y = 2^k (1 + u), u in [0, 1).  The exact ceil is k for u == 0 and
// k + 1 otherwise.  A correctly rounded fp32 log2 instead returns exactly k
// while d = log2(1 + u) is below half an ulp of the result near k:
//   * k > 0, or k < 0 with |k| not a power of two: half ulp = 2^(p-24),
//   * k < 0 with |k| == 2^p: k + d lies in the binade below, half ulp 2^(p-25),
//   with p = floor(log2 |k|); k == 0 never rounds back (d > 0 is representable).
// d < 2^-h  <=>  u < 2^(2^-h) - 1, and with u in units of 2^-23 the bound is
// 2^j ln 2 (1 + O(2^-18)) for j = 23 - h, never within 0.08 of an integer, so
// the test is  u23 <= floor(2^j ln 2).
__device__ __forceinline__ int ceil_log2_cr(float y) {
  const uint32_t bits = __float_as_uint(y);
  const uint32_t ef = bits >> 23;
  const uint32_t f = bits & 0x7fffffu;
  int k;
  uint32_t u23;
  if (ef != 0u) {
    k = (int)ef - 127;
    u23 = f;
  } else {
    const int q = 31 - __builtin_clz(f);          // top bit of the subnormal
    k = q - 149;
    u23 = (f - (1u << q)) << (23 - q);
  }
  if (u23 == 0u) return k;
  if (k == 0) return 1;
  const int a = k < 0 ? -k : k;
  const int p = 31 - __builtin_clz((uint32_t)a);
  const int j = p - 1 - ((k < 0 && (a & (a - 1)) == 0) ? 1 : 0);
  // floor(2^j ln 2) for j = 1..6; 0 for j <= 0
  const uint32_t thr = j <= 0 ? 0u : (j == 1 ? 1u : j == 2 ? 2u : j == 3 ? 5u : j == 4 ? 11u : j == 5 ? 22u : 44u);
  return (u23 <= thr) ? k : k + 1;
}

template <int IN>
__device__ __forceinline__ void load_block_f32(const void* w, int64_t blk, float* v) {
  if constexpr (IN == kF32) {
    const f32x4_t* s = reinterpret_cast<const f32x4_t*>(static_cast<const float*>(w) + blk * 32);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      f32x4_t t = s[j];
      v[4 * j] = t.x; v[4 * j + 1] = t.y; v[4 * j + 2] = t.z; v[4 * j + 3] = t.w;
    }
  } else {
    const u32x4_t* s = reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(w) + blk * 32);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4_t t = s[j];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint32_t d = t[e];
        if constexpr (IN == kBF16) {
          v[8 * j + 2 * e] = __uint_as_float(d << 16);
          v[8 * j + 2 * e + 1] = __uint_as_float(d & 0xffff0000u);
        } else {
          f16x2_t h = __builtin_bit_cast(f16x2_t, d);
          v[8 * j + 2 * e] = static_cast<float>(h.x);
          v[8 * j + 2 * e + 1] = static_cast<float>(h.y);
        }
      }
    }
  }
}

template <int IN>
__global__ __launch_bounds__(kCodecThreads) void quantize_kernel(const void* __restrict__ w,
                                                                 int64_t nblocks,
                                                                 uint8_t* __restrict__ packed,
                                                                 uint8_t* __restrict__ scale,
                                                                 uint32_t* __restrict__ flags) {
  uint32_t flag = 0;
  for (int64_t blk = blockIdx.x * (int64_t)kCodecThreads + threadIdx.x; blk < nblocks;
       blk += (int64_t)gridDim.x * kCodecThreads) {
    float v[32];
    load_block_f32<IN>(w, blk, v);
    float amax = 0.0f;
    bool finite = true;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const float a = fabsf(v[j]);
      finite = finite && (a <= 3.4028234663852886e38f);   // false for NaN and Inf
      amax = fmaxf(amax, a);
    }
    int e = 0;
    if (!finite) {
      flag |= 1u;  // TI_QFLAG_NONFINITE
    } else if (amax > 0.0f) {
      e = ceil_log2_cr(__fdiv_rn(amax, 6.0f));
    }
    if (e < -127 || e > 127) {
      flag |= 2u;  // TI_QFLAG_EXP_RANGE
      e = 0;
    }
    // x / 2^e == x * 2^-e exactly (2^-e is representable for |e| <= 127,
    // including the subnormal 2^-127), so the product rounds as the
    // reference's fp32 division does.
    const float inv = (e == 127) ? __uint_as_float(0x00400000u) : __uint_as_float((uint32_t)(127 - e) << 23);
    u32x4_t out;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      uint32_t word = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float x = v[8 * d + j];
        const float s = __fmul_rn(x, inv);
        const float m = fminf(fabsf(s), 6.0f);
        // nearest e2m1 magnitude, ties to the even code: midpoints whose
        // upper code is even (0.75, 1.75, 3.5) round up on a tie.
        uint32_t c = (m > 0.25f) + (m >= 0.75f) + (m > 1.25f) + (m >= 1.75f) + (m > 2.5f) +
                     (m >= 3.5f) + (m > 5.0f);
        c |= (__float_as_uint(s) >> 28) & 8u;  // sign of the scaled value (keeps -0)
        word |= c << (4 * j);
      }
      out[d] = word;
    }
    *reinterpret_cast<u32x4_t*>(packed + blk * 16) = out;
    scale[blk] = (uint8_t)(e + 127);
  }
  if (flag) atomicOr(flags, flag);
}

__global__ void clear_flags_kernel(uint32_t* flags) { *flags = 0u; }

int grid_for(int64_t nblocks) {
  int64_t g = (nblocks + kCodecThreads - 1) / kCodecThreads;
  if (g > 65536) g = 65536;
  return (int)(g < 1 ? 1 : g);
}

}  // namespace

hipError_t launch_dequant(const uint8_t* packed, const uint8_t* scale, int64_t rows, int64_t k,
                          void* out, int out_dtype, hipStream_t stream) {
  const int64_t nblocks = rows * (k / 32);
  if (nblocks == 0) return hipSuccess;
  const int grid = grid_for(nblocks);
  if (out_dtype == kBF16)
    dequant_kernel<kBF16><<<grid, kCodecThreads, 0, stream>>>(packed, scale, nblocks, out);
  else
    dequant_kernel<kF32><<<grid, kCodecThreads, 0, stream>>>(packed, scale, nblocks, out);
  return hipGetLastError();
}

hipError_t launch_quantize(const void* w, int in_dtype, int64_t rows, int64_t k, uint8_t* packed,
                           uint8_t* scale, uint32_t* flags, hipStream_t stream) {
  // A one-thread kernel instead of hipMemsetAsync: safe under graph capture.
  clear_flags_kernel<<<1, 1, 0, stream>>>(flags);
  const int64_t nblocks = rows * (k / 32);
  if (nblocks == 0) return hipGetLastError();
  const int grid = grid_for(nblocks);
  if (in_dtype == kF32)
    quantize_kernel<kF32><<<grid, kCodecThreads, 0, stream>>>(w, nblocks, packed, scale, flags);
  else if (in_dtype == kBF16)
    quantize_kernel<kBF16><<<grid, kCodecThreads, 0, stream>>>(w, nblocks, packed, scale, flags);
  else
    quantize_kernel<kF16><<<grid, kCodecThreads, 0, stream>>>(w, nblocks, packed, scale, flags);
  return hipGetLastError();
}

}  // namespace tinyinfer
