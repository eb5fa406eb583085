// Split-K tile kernels for small batches (up to 80 bf16 or fp16 tokens): the
// reference's per-token GEMV stages mlp_stage1_mxfp4 / mlp_stage2_mxfp4
// (tinyinfer/csrc/mlp_fp4.cu:79-142, 365-426) for a batch whose activations
// are too many for the decode kernels' registers (or whose K they decline,
// e.g. a 25600-element down stage beyond two tokens) and too few for the
// prefill GEMM's 64-token tiles to stream the weights at HBM speed.
//
// Work: a workgroup owns one K range of 1024 elements and a strided list of
// 16-row weight groups (gate and up rows are separate groups).  The range's
// activations for all tokens (padded to a multiple of 16) go to LDS once,
// 16-byte chunks XOR-swizzled by token so the MFMA operand reads of 16
// tokens hit distinct banks.  Each wave streams its groups, two in flight:
// lane l loads 16 bytes (one 32-element block) of row l % 16 at block
// 4c + l / 16 of the range (c = 0..7), so one load instruction covers 16 rows
// x 64 contiguous bytes and the lane's registers are already the A operand
// of v_mfma_f32_16x16x32_bf16: k-group l / 16 of MFMA (c, quarter q) is block
// 4c + l / 16, quarter q, for weights and activations alike.  The e8m0 bytes
// of a lane's row come as two 16-byte loads (the range's 32 blocks); block
// 4c + g's byte is byte g of dword c.  The fp32 partial tile goes to a
// workspace [K range][token][matrix * R + row]; tile_reduce adds the ranges
// in order (bit-reproducible) and applies SiLU * up, or the residual.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "mxfp4_common.hpp"
#include "mxfp4_launch.hpp"

namespace tinyinfer {

namespace {

constexpr int kTW = 8;                     // waves per workgroup
constexpr int kTThreads = kTW * 64;
constexpr int kRangeK = 1024;              // K elements per workgroup range
constexpr int kRangeLoads = kRangeK / 128; // 16-byte loads per lane per group (16 rows x 64 B each)
constexpr int kTokenLds = kRangeK * 2;     // LDS bytes per token of the range
constexpr int kTileMaxM = 80;              // five 16-token column tiles: 160 KB of activations in LDS

struct TileArgs {
  const uint16_t* x;       // [M, K]
  const uint8_t* w0;       // [R, K/2] gate (or down)
  const uint8_t* s0;       // [R, K/32]
  const uint8_t* w1;       // [R, K/2] up (gate_up only; else = w0)
  const uint8_t* s1;
  float* ws;               // [nkr][mpad][nmat * R] fp32 partials
  int M, K, R;
  int mpad;                // tokens padded to 16 * MT
  int nmat;                // 2: gate_up, 1: down
  int nkr;                 // K / 1024
  int wpk;                 // workgroups per K range
  int ngroups;             // nmat * R / 16
  int nblk;                // K / 32
};

struct TileBuf {
  u32x4_t w[kRangeLoads];
  u32x4_t s[2];            // the row's 32 scale bytes of the range
};

// Loads of row group G for K range kr.  Scales first.
__device__ __forceinline__ void tile_issue(const TileArgs& a, int G, int kr, TileBuf& b) {
  const int lane = threadIdx.x & 63;
  const int rg = a.R / 16;
  const int m = G / rg;
  const int64_t row = (int64_t)(G - m * rg) * 16 + (lane & 15);
  const uint8_t* sp = (m ? a.s1 : a.s0) + row * a.nblk + kr * 32;
  b.s[0] = *reinterpret_cast<const u32x4_t*>(sp);
  b.s[1] = *reinterpret_cast<const u32x4_t*>(sp + 16);
  const uint8_t* wp = (m ? a.w1 : a.w0) + row * (a.K / 2) + (int64_t)kr * (kRangeK / 2) + 16 * (lane >> 4);
  // plain loads: the non-temporal hint measured slower for this pattern (8B
  // down at 16 tokens 14.8 against 13.0 us, 64 tokens 26.6 against 22.1)
#pragma unroll
  for (int c = 0; c < kRangeLoads; ++c) b.w[c] = *reinterpret_cast<const u32x4_t*>(wp + 64 * c);
  __builtin_amdgcn_sched_barrier(0);
}

__device__ __forceinline__ uint32_t tile_scale(const TileBuf& b, int c) {
  return (b.s[c >> 2][c & 3] >> (8 * ((threadIdx.x >> 4) & 3))) & 0xffu;
}

// lds: the K range's activations, token t at lds + t * tstride.  MODE 0:
// bf16 activations, hardware conversion; 1: bf16, exact conversion; 2: fp16
// activations, weights converted to fp16 by the hardware (exact when every
// scale byte is e8m0_f16_ok), fp16 MFMAs; 3: fp16 activations, exact bf16
// weights against the activations' exact bf16 hi and lo parts (two MFMAs).
template <int MT, int MODE>
__device__ __forceinline__ void tile_mma(const TileBuf& b, const uint8_t* lds, int tstride, f32x4_t (&acc)[MT]) {
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
#pragma unroll
  for (int c = 0; c < kRangeLoads; ++c) {
    const uint32_t sb = tile_scale(b, c);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x4_t wa = MODE == 0   ? dq8_bf16_fast(b.w[c][q], sb)
                         : MODE == 2 ? dq8_f16_fast(b.w[c][q], sb)
                                     : dq8_bf16_exact(b.w[c][q], sb);
      const int ch = (4 * c + g) * 4 + q;   // 16-byte chunk of the range
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const u32x4_t xb = *reinterpret_cast<const u32x4_t*>(lds + (16 * mt + n) * tstride + 16 * (ch ^ n));
        if constexpr (MODE == 2) {
          acc[mt] = mfma16x16x32_f16(wa, xb, acc[mt]);
        } else if constexpr (MODE == 3) {
          u32x4_t xh, xl;
          f16x8_split_bf16(xb, xh, xl);
          acc[mt] = mfma16x16x32(wa, xl, mfma16x16x32(wa, xh, acc[mt]));
        } else {
          acc[mt] = mfma16x16x32(wa, xb, acc[mt]);
        }
      }
    }
  }
}

// The group's multiply: per wave, the faster exact form its scale bytes allow.
template <int MT, int DT>
__device__ __forceinline__ void tile_group_mma(const TileBuf& b, const uint8_t* lds, int tstride,
                                               f32x4_t (&acc)[MT]) {
  bool ok = true;
#pragma unroll
  for (int c = 0; c < kRangeLoads; ++c)
    ok = ok && (DT == kBF16 ? e8m0_fast_ok(tile_scale(b, c)) : e8m0_f16_ok(tile_scale(b, c)));
  if (wave_all(ok)) tile_mma<MT, DT == kBF16 ? 0 : 2>(b, lds, tstride, acc);
  else tile_mma<MT, DT == kBF16 ? 1 : 3>(b, lds, tstride, acc);
}

// NG groups at once: each activation operand read from LDS serves all NG
// groups' MFMAs (1 / NG of the LDS reads of NG tile_group_mma calls; the
// same products and sums, so the same bits).  One form for all: the fast
// conversion only when every scale byte of every group allows it.
template <int MT, int MODE, int NG>
__device__ __forceinline__ void tile_mma_multi(const TileBuf (&b)[NG], const uint8_t* lds, int tstride,
                                               f32x4_t (&acc)[NG][MT]) {
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
#pragma unroll
  for (int c = 0; c < kRangeLoads; ++c) {
    uint32_t sc[NG];
#pragma unroll
    for (int i = 0; i < NG; ++i) sc[i] = tile_scale(b[i], c);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      u32x4_t w[NG];
#pragma unroll
      for (int i = 0; i < NG; ++i)
        w[i] = MODE == 0   ? dq8_bf16_fast(b[i].w[c][q], sc[i])
               : MODE == 2 ? dq8_f16_fast(b[i].w[c][q], sc[i])
                           : dq8_bf16_exact(b[i].w[c][q], sc[i]);
      const int ch = (4 * c + g) * 4 + q;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const u32x4_t xb = *reinterpret_cast<const u32x4_t*>(lds + (16 * mt + n) * tstride + 16 * (ch ^ n));
        if constexpr (MODE == 3) {
          u32x4_t xh, xl;
          f16x8_split_bf16(xb, xh, xl);
#pragma unroll
          for (int i = 0; i < NG; ++i) acc[i][mt] = mfma16x16x32(w[i], xl, mfma16x16x32(w[i], xh, acc[i][mt]));
        } else {
#pragma unroll
          for (int i = 0; i < NG; ++i)
            acc[i][mt] = MODE == 2 ? mfma16x16x32_f16(w[i], xb, acc[i][mt]) : mfma16x16x32(w[i], xb, acc[i][mt]);
        }
      }
      // one quarter at a time: the compiler would otherwise hoist every
      // quarter's operand reads and spill
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

template <int MT, int DT, int NG>
__device__ __forceinline__ void tile_multi_mma(const TileBuf (&b)[NG], const uint8_t* lds, int tstride,
                                               f32x4_t (&acc)[NG][MT]) {
  bool ok = true;
#pragma unroll
  for (int c = 0; c < kRangeLoads; ++c)
#pragma unroll
    for (int i = 0; i < NG; ++i)
      ok = ok && (DT == kBF16 ? e8m0_fast_ok(tile_scale(b[i], c)) : e8m0_f16_ok(tile_scale(b[i], c)));
  if (wave_all(ok)) tile_mma_multi<MT, DT == kBF16 ? 0 : 2, NG>(b, lds, tstride, acc);
  else tile_mma_multi<MT, DT == kBF16 ? 1 : 3, NG>(b, lds, tstride, acc);
}

// NG > 0: every wave owns exactly NG groups (ngroups = NG * wpk * 8; 8B down
// at every token count: 2, 8B gate_up at 17..64 tokens: 3): all of them are
// loaded at once and multiplied together, one LDS read of each activation
// operand for all.  Kernels of their own, so that the loop form's (NG = 0)
// registers are not raised by them.
template <int MT, int DT, int NG>
__global__ __launch_bounds__(kTThreads, 1) void tile_kernel(TileArgs a) {
  constexpr int kXPre = MT * 16 * (kRangeK / 8) / kTThreads;   // 16-byte x chunks per thread
  extern __shared__ __align__(16) uint8_t lds[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int kr = blockIdx.x % a.nkr;
  const int wi = blockIdx.x / a.nkr;
  const int nslots = a.wpk * kTW;
  const int slot = wi * kTW + wave;
  const int units = slot < a.ngroups ? (a.ngroups - slot + nslots - 1) / nslots : 0;

  // the range's activations: token t = c / 128, chunk c % 128 (clamped rows
  // past M are loaded and replaced by zeros)
  u32x4_t xv[kXPre];
#pragma unroll
  for (int p = 0; p < kXPre; ++p) {
    const int c = threadIdx.x + p * kTThreads;
    const int t = c >> 7;
    const int tr = t < a.M ? t : a.M - 1;
    xv[p] = *reinterpret_cast<const u32x4_t*>(a.x + (int64_t)tr * a.K + (int64_t)kr * kRangeK + 8 * (c & 127));
  }
  TileBuf b0, b1, bx;
  auto group_of = [&](int j) { return units > 0 ? slot + (j < units ? j : units - 1) * nslots : slot % a.ngroups; };
  tile_issue(a, group_of(0), kr, b0);
  tile_issue(a, group_of(1), kr, b1);
  if constexpr (NG == 3) tile_issue(a, group_of(2), kr, bx);
#pragma unroll
  for (int p = 0; p < kXPre; ++p) {
    const int c = threadIdx.x + p * kTThreads;
    const int t = c >> 7;
    const u32x4_t v = t < a.M ? xv[p] : u32x4_t{0u, 0u, 0u, 0u};
    *reinterpret_cast<u32x4_t*>(lds + t * kTokenLds + 16 * ((c & 127) ^ (t & 15))) = v;
  }
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);    // lgkmcnt(0): LDS only, not the weights in flight
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  const int nmr = a.nmat * a.R;
  // lane l holds rows 4 (l / 16) + v of the group, token 16 mt + l % 16
  auto store = [&](int G, const f32x4_t (&acc)[MT]) __attribute__((always_inline)) {
    const int rg = a.R / 16;
    const int m = G / rg;
    const int col = m * a.R + (G - m * rg) * 16 + 4 * (lane >> 4);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int t = 16 * mt + (lane & 15);
      *reinterpret_cast<f32x4_t*>(a.ws + ((int64_t)kr * a.mpad + t) * nmr + col) = acc[mt];
    }
  };
  auto step = [&](TileBuf& b, int j, auto issue_tag) __attribute__((always_inline)) {
    const int G = group_of(j);
    f32x4_t acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    tile_group_mma<MT, DT>(b, lds, kTokenLds, acc);
    if constexpr (decltype(issue_tag)::value) tile_issue(a, group_of(j + 2), kr, b);
    store(G, acc);
  };
  if constexpr (NG > 0) {
    // the wave's whole share: the groups in b0, b1 and (NG = 3) bx
    TileBuf bs[NG];
    bs[0] = b0;
    bs[1] = b1;
    if constexpr (NG == 3) bs[2] = bx;
    f32x4_t acc[NG][MT];
#pragma unroll
    for (int i = 0; i < NG; ++i)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[i][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    tile_multi_mma<MT, DT, NG>(bs, lds, kTokenLds, acc);
#pragma unroll
    for (int i = 0; i < NG; ++i) store(group_of(i), acc[i]);
    return;
  }
  constexpr std::true_type kIssue{};
  constexpr std::false_type kLast{};
  // every load issued is a group the wave multiplies (tails peeled; an issue
  // under a condition inside the loop would drain the load queue each step)
  int j = 0;
  for (; j + 3 < units; j += 2) {
    step(b0, j, kIssue);
    step(b1, j + 1, kIssue);
  }
  const int left = units - j;
  if (left == 3) {
    step(b0, j, kIssue);
    step(b1, j + 1, kLast);
    step(b0, j + 2, kLast);
  } else if (left == 2) {
    step(b0, j, kLast);
    step(b1, j + 1, kLast);
  } else if (left == 1) {
    step(b0, j, kLast);
  }
}

// out[m][n] = epilogue(sum over kr of ws[kr][m][n] (and [R + n] for up)), in
// kr order; four outputs per thread.
template <int NMAT, int DT>
__global__ __launch_bounds__(256) void tile_reduce(const float* __restrict__ ws, uint16_t* out, const uint16_t* res,
                                                   int M, int mpad, int R, int nkr) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)M * R / 4;
  if (q >= total) return;
  const int64_t m = q / (R / 4);
  const int n = (int)(q - m * (R / 4)) * 4;
  // loads in batches of 16 ranges (issued together, then added in range order):
  // one memory round trip for up to 16 ranges (8B down: 12)
  constexpr int kBatch = 16;
  f32x4_t g = {0.f, 0.f, 0.f, 0.f}, u = {0.f, 0.f, 0.f, 0.f};
  const int64_t stride = (int64_t)mpad * (NMAT * R);
  const float* base = ws + m * (NMAT * R) + n;
  for (int k0 = 0; k0 < nkr; k0 += kBatch) {
    f32x4_t pg[kBatch], pu[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int kr = k0 + i < nkr ? k0 + i : nkr - 1;
      pg[i] = *reinterpret_cast<const f32x4_t*>(base + kr * stride);
      if constexpr (NMAT == 2) pu[i] = *reinterpret_cast<const f32x4_t*>(base + kr * stride + R);
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      if (k0 + i < nkr) {
        g += pg[i];
        if constexpr (NMAT == 2) u += pu[i];
      }
    }
  }
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = NMAT == 2 ? silu_f32(g[e]) * u[e] : g[e];
  const uint32_t lo = (uint32_t)f32_to_act<DT>(v[0]) | ((uint32_t)f32_to_act<DT>(v[1]) << 16);
  const uint32_t hi = (uint32_t)f32_to_act<DT>(v[2]) | ((uint32_t)f32_to_act<DT>(v[3]) << 16);
  *reinterpret_cast<u32x2_t*>(out + m * R + n) = with_residual4<DT>(u32x2_t{lo, hi}, res, m * R + n);
}

// gate_up without the K split, when all of x fits LDS (S = K / 1024 ranges,
// MT * S <= 4): a workgroup iteration takes 4 / S blocks of 16 gate rows and
// the 16 matching up rows; wave w multiplies matrix (w / S) % 2 of block
// w / (2 S) over K range w % S.  The partial tiles meet in LDS (two buffers,
// so one barrier per iteration), and the workgroup adds each output's ranges
// in order, applies SiLU * up and stores h: no workspace round trip and no
// reduce launch.  Every wave runs the same iterations (the barrier); blocks
// past the end repeat the last one and store to `dummy` instead.
// NI = 3: every workgroup runs exactly three iterations (8B at up to 16
// tokens: 768 row blocks over 256 workgroups).  Each wave then loads its
// three groups at once (same K range, so each activation operand read from
// LDS feeds all three), and the three iterations' partial tiles meet in LDS
// behind one barrier instead of three.  NI = 0: the loop.
template <int MT, int S, int DT, int NI>
__global__ __launch_bounds__(kTThreads, 1) void tile_gu_kernel(TileArgs a, uint16_t* out, uint16_t* dummy) {
  static_assert(S == 1 || S == 2 || S == 4, "8 waves = (4 / S) blocks x 2 matrices x S ranges");
  constexpr int kBlocks = 4 / S;
  constexpr int kMpad = 16 * MT;
  constexpr int kXPre = kMpad * S * (kRangeK / 8) / kTThreads;
  constexpr int kOut = kBlocks * 16 * kMpad;                  // outputs per iteration
  constexpr int kOutTrips = kOut >= kTThreads ? kOut / kTThreads : 1;
  extern __shared__ __align__(16) uint8_t lds[];
  const int tstride = S * kRangeK * 2;                         // LDS bytes per token (all of K)
  float* part = reinterpret_cast<float*>(lds + kMpad * tstride);   // [2][8 waves][MT][64 lanes][4]
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int rbl = wave / (2 * S), mat = (wave / S) & 1, sp = wave % S;
  const int nrb = a.R / 16;
  const int per_iter = (int)gridDim.x * kBlocks;
  const int niter = (nrb + per_iter - 1) / per_iter;
  auto rb_of = [&](int it) {
    const int rb = (it * (int)gridDim.x + (int)blockIdx.x) * kBlocks + rbl;
    return rb < nrb ? rb : nrb - 1;
  };

  // all of x: token t = c / (K / 8), 16-byte chunk c % (K / 8); per K range
  // the split kernel's swizzle
  const int nxr = a.K / 8;
  u32x4_t xv[kXPre];
#pragma unroll
  for (int p = 0; p < kXPre; ++p) {
    const int c = threadIdx.x + p * kTThreads;
    const int t = c / nxr;
    const int tr = t < a.M ? t : a.M - 1;
    xv[p] = *reinterpret_cast<const u32x4_t*>(a.x + (int64_t)tr * a.K + 8 * (c - t * nxr));
  }
  TileBuf b0, b1;
  tile_issue(a, mat * nrb + rb_of(0), sp, b0);
  tile_issue(a, mat * nrb + rb_of(1), sp, b1);
#pragma unroll
  for (int p = 0; p < kXPre; ++p) {
    const int c = threadIdx.x + p * kTThreads;
    const int t = c / nxr, cc = c - t * nxr;
    const u32x4_t v = t < a.M ? xv[p] : u32x4_t{0u, 0u, 0u, 0u};
    *reinterpret_cast<u32x4_t*>(lds + t * tstride + (cc >> 7) * kTokenLds + 16 * ((cc & 127) ^ (t & 15))) = v;
  }
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);    // lgkmcnt(0): LDS only, not the weights in flight
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // iteration it's outputs from its partial tiles at pr: o = (block, token,
  // row), row fastest, so a token's 16 rows are one 32-byte store run
  auto emit = [&](int it, const float* pr) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < kOutTrips; ++k) {
      const int o = kOut >= kTThreads ? (int)threadIdx.x + k * kTThreads : (int)threadIdx.x % kOut;
      const int i = o & 15, t = (o >> 4) % kMpad, bl = (o >> 4) / kMpad;
      const int ln = 16 * (i >> 2) + (t & 15), v = i & 3, mt = t >> 4;
      float g = 0.f, u = 0.f;
#pragma unroll
      for (int s2 = 0; s2 < S; ++s2) {
        g += pr[(((bl * 2 * S + s2) * MT + mt) * 64 + ln) * 4 + v];
        u += pr[(((bl * 2 * S + S + s2) * MT + mt) * 64 + ln) * 4 + v];
      }
      const int rb = (it * (int)gridDim.x + (int)blockIdx.x) * kBlocks + bl;
      const bool valid = rb < nrb && t < a.M && (kOut >= kTThreads || (int)threadIdx.x < kOut);
      uint16_t* dst = valid ? out + (int64_t)t * a.R + rb * 16 + i : dummy + threadIdx.x;
      *dst = f32_to_act<DT>(silu_f32(g) * u);
    }
  };
  if constexpr (NI == 3) {
    TileBuf bs[3];
    bs[0] = b0;
    bs[1] = b1;
    tile_issue(a, mat * nrb + rb_of(2), sp, bs[2]);   // after x left the registers
    f32x4_t acc[3][MT];
#pragma unroll
    for (int j = 0; j < 3; ++j)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[j][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    tile_multi_mma<MT, DT, 3>(bs, lds + sp * kTokenLds, tstride, acc);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      float* pw = part + (j * kTW + wave) * MT * 256;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) *reinterpret_cast<f32x4_t*>(pw + (mt * 64 + lane) * 4) = acc[j][mt];
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int j = 0; j < 3; ++j) emit(j, part + j * kTW * MT * 256);
    return;
  }
  auto step = [&](TileBuf& b, int it, auto issue_tag) __attribute__((always_inline)) {
    f32x4_t acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    tile_group_mma<MT, DT>(b, lds + sp * kTokenLds, tstride, acc);
    if constexpr (decltype(issue_tag)::value) tile_issue(a, mat * nrb + rb_of(it + 2), sp, b);
    float* pw = part + ((it & 1) * kTW + wave) * MT * 256;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) *reinterpret_cast<f32x4_t*>(pw + (mt * 64 + lane) * 4) = acc[mt];
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    emit(it, part + (it & 1) * kTW * MT * 256);
  };
  constexpr std::true_type kIssue{};
  constexpr std::false_type kLast{};
  int it = 0;
  for (; it + 3 < niter; it += 2) {
    step(b0, it, kIssue);
    step(b1, it + 1, kIssue);
  }
  const int left = niter - it;
  if (left == 3) {
    step(b0, it, kIssue);
    step(b1, it + 1, kLast);
    step(b0, it + 2, kLast);
  } else if (left == 2) {
    step(b0, it, kLast);
    step(b1, it + 1, kLast);
  } else if (left == 1) {
    step(b0, it, kLast);
  }
}

int tile_cus() { return device_info().cus; }

// Workgroups per K range: about one workgroup per CU over all ranges, at
// least one group per wave, then as few as give every wave the same largest
// number of groups (8B down at 16 tokens: 16 instead of 21 per range, two
// groups per wave; 12.4 -> 12.1 us).
bool tile_plan(int64_t M, int64_t K, int64_t R, bool gateup, TileArgs& a, int& grid, int& mt, size_t& ws_bytes) {
  const int cus = tile_cus();
  if (cus < 1 || M < 1 || M > kTileMaxM || K < kRangeK || K % kRangeK != 0 || K > (1 << 20) || R < 16 || R % 16 != 0 ||
      R > (1 << 22))
    return false;
  mt = (int)((M + 15) / 16);
  a.M = (int)M;
  a.K = (int)K;
  a.R = (int)R;
  a.mpad = 16 * mt;
  a.nmat = gateup ? 2 : 1;
  a.nkr = (int)(K / kRangeK);
  a.ngroups = (int)(a.nmat * R / 16);
  a.nblk = (int)(K / kBlock);
  int wpk = std::max(1, cus / a.nkr);
  wpk = std::min(wpk, (a.ngroups + kTW - 1) / kTW);
  const int umax = (a.ngroups + wpk * kTW - 1) / (wpk * kTW);
  wpk = (a.ngroups + umax * kTW - 1) / (umax * kTW);
  a.wpk = wpk;
  grid = a.nkr * wpk;
  ws_bytes = (size_t)a.nkr * a.mpad * a.nmat * (size_t)R * sizeof(float);
  return true;
}

bool aligned_tile(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; }

template <int MT, int DT>
hipError_t tile_launch(const TileArgs& a, int grid, hipStream_t st) {
  const int lds = MT * 16 * kTokenLds;
  const int nslots = a.wpk * kTW;
  auto k = a.ngroups == 2 * nslots   ? tile_kernel<MT, DT, 2>
           : a.ngroups == 3 * nslots ? tile_kernel<MT, DT, 3>
                                     : tile_kernel<MT, DT, 0>;
  if (lds > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, lds) !=
          hipSuccess)
    return hipErrorNotSupported;
  hipLaunchKernelGGL(k, dim3(grid), dim3(kTThreads), (size_t)lds, st, a);
  return hipGetLastError();
}

// gate_up in one launch (tile_gu_kernel): S = K / 1024 ranges in {1, 2, 4},
// at most two column tiles, all of x plus the partial buffers within LDS.
bool tile_gu_fits(const TileArgs& a, int mt) {
  const int S = a.nkr;
  return (S == 1 || S == 2 || S == 4) && mt <= 2 && mt * S <= 4 && a.R % 16 == 0;
}

bool tile_gu_enabled() { return option(kOptTileGu) != 0; }

template <int MT, int S, int DT>
hipError_t tile_gu_launch(const TileArgs& a, int grid, uint16_t* out, hipStream_t st) {
  const int nrb = a.R / 16;
  const int niter = (nrb + grid * (4 / S) - 1) / (grid * (4 / S));
  // three iterations' partial tiles at once when each workgroup runs three
  const int part_tile = kTW * MT * 256 * (int)sizeof(float);
  const int lds3 = 16 * MT * S * kTokenLds + 3 * part_tile;
  const bool three = niter == 3 && lds3 <= device_info().lds_per_block;
  auto k = three ? tile_gu_kernel<MT, S, DT, 3> : tile_gu_kernel<MT, S, DT, 0>;
  const int lds_k = three ? lds3 : 16 * MT * S * kTokenLds + 2 * part_tile;
  if (lds_k > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, lds_k) !=
          hipSuccess)
    return hipErrorNotSupported;
  // stores of outputs past the end go to the (otherwise unused) workspace
  hipLaunchKernelGGL(k, dim3(grid), dim3(kTThreads), (size_t)lds_k, st, a, out, reinterpret_cast<uint16_t*>(a.ws));
  return hipGetLastError();
}

template <bool GATEUP, int DT>
hipError_t tile_stage(const MlpArgs& m, hipStream_t st) {
  TileArgs a;
  int grid = 0, mt = 0;
  size_t bytes = 0;
  const int64_t K = GATEUP ? m.hidden : m.inter;
  const int64_t R = GATEUP ? m.inter : m.hidden;
  if (m.dtype != DT || !tile_plan(m.n, K, R, GATEUP, a, grid, mt, bytes)) return hipErrorNotSupported;
  a.ws = m.ws ? (bytes <= m.ws_bytes ? m.ws : nullptr) : gemm_split_workspace(bytes, st);
  if (!a.ws) return hipErrorNotSupported;
  a.x = static_cast<const uint16_t*>(GATEUP ? m.x : m.tmp);
  a.w0 = GATEUP ? m.gate : m.down;
  a.s0 = GATEUP ? m.gate_scale : m.down_scale;
  a.w1 = GATEUP ? m.up : a.w0;
  a.s1 = GATEUP ? m.up_scale : a.s0;
  if constexpr (GATEUP) {
    if (tile_gu_fits(a, mt) && tile_gu_enabled()) {
      const int S = a.nkr;
      const int kblocks = 4 / S;
      const int nrb = a.R / 16;
      const int g2 = std::min(tile_cus(), (nrb + kblocks - 1) / kblocks);
      switch (mt * 8 + S) {
        case 8 + 1: return tile_gu_launch<1, 1, DT>(a, g2, static_cast<uint16_t*>(m.tmp), st);
        case 8 + 2: return tile_gu_launch<1, 2, DT>(a, g2, static_cast<uint16_t*>(m.tmp), st);
        case 8 + 4: return tile_gu_launch<1, 4, DT>(a, g2, static_cast<uint16_t*>(m.tmp), st);
        case 16 + 1: return tile_gu_launch<2, 1, DT>(a, g2, static_cast<uint16_t*>(m.tmp), st);
        case 16 + 2: return tile_gu_launch<2, 2, DT>(a, g2, static_cast<uint16_t*>(m.tmp), st);
        default: break;
      }
    }
  }
  hipError_t e = hipErrorNotSupported;
  switch (mt) {
    case 1: e = tile_launch<1, DT>(a, grid, st); break;
    case 2: e = tile_launch<2, DT>(a, grid, st); break;
    case 3: e = tile_launch<3, DT>(a, grid, st); break;
    case 4: e = tile_launch<4, DT>(a, grid, st); break;
    case 5: e = tile_launch<5, DT>(a, grid, st); break;
    default: break;
  }
  if (e != hipSuccess) return e;
  uint16_t* out = static_cast<uint16_t*>(GATEUP ? m.tmp : m.out);
  const uint16_t* res = GATEUP ? nullptr : static_cast<const uint16_t*>(m.residual);
  const int64_t groups = m.n * R / 4;
  tile_reduce<GATEUP ? 2 : 1, DT><<<(unsigned)((groups + 255) / 256), 256, 0, st>>>(a.ws, out, res, a.M, a.mpad, a.R,
                                                                                 a.nkr);
  return hipGetLastError();
}

}  // namespace

bool tile_enabled() { return option(kOptTile) != 0; }

size_t tile_workspace_need(const MlpArgs& m, int stage) {
  if (m.dtype != kBF16 && m.dtype != kF16) return 0;
  if ((stage & kStageGateUp) && m.norm_w != nullptr) return 0;
  TileArgs a;
  int grid = 0, mt = 0;
  size_t bytes = 0, need = 0;
  if (stage & kStageGateUp) {
    if (!tile_plan(m.n, m.hidden, m.inter, true, a, grid, mt, bytes)) return 0;
    need = std::max(need, bytes);
  }
  if (stage & kStageDown) {
    if (!tile_plan(m.n, m.inter, m.hidden, false, a, grid, mt, bytes)) return 0;
    need = std::max(need, bytes);
  }
  // 16-byte loads of activations, weights and scale runs; 8-byte output stores
  const void* p16[] = {m.x, m.gate, m.up, m.down, m.gate_scale, m.up_scale, m.down_scale, m.tmp};
  for (const void* p : p16)
    if (p && !aligned_tile(p, 16)) return 0;
  const void* p8[] = {m.out, m.residual};
  for (const void* p : p8)
    if (p && !aligned_tile(p, 8)) return 0;
  return need;
}

bool tile_supported(const MlpArgs& m, int stage, hipStream_t st) {
  const size_t need = tile_workspace_need(m, stage);
  if (need == 0) return false;
  if (m.ws) return need <= m.ws_bytes;
  return gemm_split_workspace(need, st) != nullptr;
}

hipError_t launch_tile_mlp(const MlpArgs& m, int stage, hipStream_t st) {
  const bool f16 = m.dtype == kF16;
  if (stage & kStageGateUp) {
    const hipError_t e = f16 ? tile_stage<true, kF16>(m, st) : tile_stage<true, kBF16>(m, st);
    if (e != hipSuccess) return e;
  }
  if (stage & kStageDown) return f16 ? tile_stage<false, kF16>(m, st) : tile_stage<false, kBF16>(m, st);
  return hipSuccess;
}

}  // namespace tinyinfer
