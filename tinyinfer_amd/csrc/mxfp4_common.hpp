// Device helpers shared by the MXFP4 kernels (gfx950 / CDNA4 only).
//
// Format: e2m1 codes packed two per byte (element 2j in the low nibble of byte
// j), one e8m0 byte per 32 consecutive input features, value
// (-1)^s * {0,.5,1,1.5,2,3,4,6}[m] * 2^(byte-127); byte 255 is NaN.
// (Reference: tinyinfer/quantization/quantize_mxfp4.py:20-85,
//  tinyinfer/csrc/utils.h:87-127.)
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace tinyinfer {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kBlock = 32;          // elements per e8m0 scale
constexpr int kWave = 64;           // CDNA wavefront width

// Activation dtype codes at the C ABI (same meaning as the reference's
// dtype_code, tinyinfer/csrc/mlp_fp4.cu:481-515), plus fp32 for the codec.
enum DType : int { kF16 = 0, kBF16 = 1, kF32 = 2 };

// ---------------------------------------------------------------- decode

// e8m0 byte -> fp32 2^(b-127); byte 0 is the subnormal 2^-127, 255 is NaN.
__device__ __forceinline__ float e8m0_to_f32(uint32_t b) {
  uint32_t bits = (b == 0u) ? 0x00400000u : (b == 255u ? 0x7fc00000u : (b << 23));
  return __uint_as_float(bits);
}

// e2m1 code -> fp32, exact; code 8 -> -0.0.
__device__ __forceinline__ float e2m1_to_f32(uint32_t c) {
  // magnitude bits m2m1m0: m=1 -> 0.5 (exp 126), m>=2 -> exp 126 + (m>>1),
  // mantissa top bit = m & 1.
  uint32_t m = c & 7u;
  uint32_t bits = (m == 0u) ? 0u
                            : (((126u + (m >> 1)) << 23) | ((m >= 2u ? (m & 1u) : 0u) << 22));
  return __uint_as_float(bits | ((c & 8u) << 28));
}

// Scale bytes for which every e2m1 value times 2^(b-127) is a finite normal
// number in bf16/fp32: min |v| = 2^(b-128) >= 2^-126 and max 6*2^(b-127) <=
// 1.5*2^127.  Inside this range the hardware conversion is exact.
__device__ __forceinline__ bool e8m0_fast_ok(uint32_t b) { return (b - 2u) <= 250u; }

__device__ __forceinline__ uint32_t bf16x2_bits(bf16x2_t v) {
  return __builtin_bit_cast(uint32_t, v);
}

// Exact slow path: two codes (byte `byte`) times the scale as fp32, then the
// top 16 bits (every such product has <= 2 significant bits, so the low 16
// bits are zero and truncation is exact; fp32 subnormals and +-inf carry over).
__device__ __forceinline__ uint32_t dq_byte_bf16_exact(uint32_t byte, uint32_t b) {
  float s = e8m0_to_f32(b);
  float lo = e2m1_to_f32(byte & 15u) * s;
  float hi = e2m1_to_f32(byte >> 4) * s;
  return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
}

// 8 codes in one dword (elements 0..7, element 0 in the low nibble) -> 8 bf16
// as four dwords, `b` being the e8m0 byte of their block.
//
// dq8_bf16_fast: hardware conversion with the block scale folded in
// (v_cvt_scalef32_pk_bf16_fp4); exact only when e8m0_fast_ok(b).
__device__ __forceinline__ u32x4_t dq8_bf16_fast(uint32_t w, uint32_t b) {
  u32x4_t r;
  const float s = __uint_as_float(b << 23);
  r.x = bf16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 0));
  r.y = bf16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 1));
  r.z = bf16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 2));
  r.w = bf16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 3));
  return r;
}

// Scale bytes for which every e2m1 value times 2^(b-127) is exactly an fp16
// number: the smallest, 2^(b-128), at least fp16's smallest subnormal 2^-24
// (all values are multiples of it, with at most 4 significant bits), the
// largest, 6 * 2^(b-127), at most 49152 < 65504.  (Kernels keep fp16
// denormals: the code object's fp16/fp64 denormal mode preserves them.)
__device__ __forceinline__ bool e8m0_f16_ok(uint32_t b) { return (b - 104u) <= 36u; }

// dq8_f16_fast: eight codes times the block scale as fp16, by the hardware
// conversion (v_cvt_scalef32_pk_f16_fp4); exact only when e8m0_f16_ok(b).
__device__ __forceinline__ u32x4_t dq8_f16_fast(uint32_t w, uint32_t b) {
  u32x4_t r;
  const float s = __uint_as_float(b << 23);
  r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 0));
  r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 1));
  r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 2));
  r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 3));
  return r;
}

// dq8_bf16_exact: exact for every scale byte (subnormal products, +-inf, NaN).
__device__ __forceinline__ u32x4_t dq8_bf16_exact(uint32_t w, uint32_t b) {
  u32x4_t r;
  r.x = dq_byte_bf16_exact(w & 0xffu, b);
  r.y = dq_byte_bf16_exact((w >> 8) & 0xffu, b);
  r.z = dq_byte_bf16_exact((w >> 16) & 0xffu, b);
  r.w = dq_byte_bf16_exact(w >> 24, b);
  return r;
}

// Per-lane choice of the two (for code where lanes' scales are independent).
// Hot loops instead decide once per wave with wave_all_fast() and call
// dq8_bf16_fast / dq8_bf16_exact directly: a per-dword branch costs more
// than the conversion.
__device__ __forceinline__ u32x4_t dq8_bf16(uint32_t w, uint32_t b) {
  return __builtin_expect(e8m0_fast_ok(b), 1) ? dq8_bf16_fast(w, b) : dq8_bf16_exact(w, b);
}

// True (uniformly across the wave) when every active lane's flag is true.
__device__ __forceinline__ bool wave_all(bool ok) { return !__any(!ok); }

// Sum over the 64 lanes (all active), the same bits in every lane.  Within
// each row of 16 lanes by DPP exchanges (xor 1 and xor 2 as quad permutes,
// then the half-row and row mirrors): a pair's two lanes add the same two
// values, so they agree; then the four row sums are read into scalars and
// added in a fixed order.  No LDS round trips (a shuffle is one each).
template <int kCtrl>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kCtrl, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_sum64(float v) {
  v = dpp_add<0xb1>(v);     // quad_perm [1,0,3,2]
  v = dpp_add<0x4e>(v);     // quad_perm [2,3,0,1]
  v = dpp_add<0x141>(v);    // row_half_mirror
  v = dpp_add<0x140>(v);    // row_mirror
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

// 8 codes -> 8 fp32 (exact, all scale bytes).
__device__ __forceinline__ void dq8_f32(uint32_t w, uint32_t b, float* out) {
  float s = e8m0_to_f32(b);
#pragma unroll
  for (int j = 0; j < 8; ++j) out[j] = e2m1_to_f32((w >> (4 * j)) & 15u) * s;
}

// ---------------------------------------------------------------- numerics

// SiLU as the reference writes it (utils.h:76-78), with ROCm's expf.
__device__ __forceinline__ float silu_f32(float v) { return v / (1.0f + expf(-v)); }

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}
template <int DT>
__device__ __forceinline__ uint16_t f32_to_act(float f) {
  if constexpr (DT == kBF16) return f32_to_bf16_rne(f);
  else return f32_to_f16_rne(f);
}

template <int DT>
__device__ __forceinline__ float act_to_f32(uint16_t v) {
  if constexpr (DT == kBF16) return __uint_as_float((uint32_t)v << 16);
  else return static_cast<float>(__builtin_bit_cast(_Float16, v));
}

// A stored down-stage output: the MLP value already rounded to the
// activation dtype, plus the residual (when there is one) in fp32, rounded
// again -- what torch computes for `x + mlp(x)` on two activation-dtype
// tensors (the reference's residual add, tinyinfer/models/qwen3.py:219).
template <int DT>
__device__ __forceinline__ uint16_t with_residual(uint16_t v, const uint16_t* res, int64_t idx) {
  return res ? f32_to_act<DT>(act_to_f32<DT>(res[idx]) + act_to_f32<DT>(v)) : v;
}
// The same for four consecutive outputs packed in two dwords (res + idx
// 8-byte aligned).
template <int DT>
__device__ __forceinline__ u32x2_t with_residual4(u32x2_t v, const uint16_t* res, int64_t idx) {
  if (!res) return v;
  const u32x2_t r = *reinterpret_cast<const u32x2_t*>(res + idx);
  u32x2_t o;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float lo = act_to_f32<DT>((uint16_t)(r[h] & 0xffffu)) + act_to_f32<DT>((uint16_t)(v[h] & 0xffffu));
    const float hi = act_to_f32<DT>((uint16_t)(r[h] >> 16)) + act_to_f32<DT>((uint16_t)(v[h] >> 16));
    o[h] = (uint32_t)f32_to_act<DT>(lo) | ((uint32_t)f32_to_act<DT>(hi) << 16);
  }
  return o;
}

// fp16x8 (as 4 dwords) -> exact bf16 hi/lo split: x = hi + lo with both bf16
// (fp16's 11 significant bits over two 8-bit halves).  An infinite or NaN x
// goes whole into hi with lo = 0, so w * hi + w * lo is w * x as IEEE has it
// (inf - inf would make lo a NaN).
__device__ __forceinline__ void f16x8_split_bf16(u32x4_t v, u32x4_t& hi, u32x4_t& lo) {
  f16x8_t h = __builtin_bit_cast(f16x8_t, v);
  bf16x8_t a, c;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float f = static_cast<float>(h[j]);
    __bf16 t = static_cast<__bf16>(f);
    a[j] = t;
    const float r = f - static_cast<float>(t);
    c[j] = static_cast<__bf16>(r == r ? r : 0.f);
  }
  hi = __builtin_bit_cast(u32x4_t, a);
  lo = __builtin_bit_cast(u32x4_t, c);
}

// ---------------------------------------------------------------- MFMA

__device__ __forceinline__ f32x4_t mfma16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mfma16x16x32_f16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16_t mfma32x32x16(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16_t mfma32x32x16_f16(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

}  // namespace tinyinfer
