// Streaming MXFP4 GEMV for decode (M <= 8 tokens): one kernel per MLP stage.
//
// Replaces, for small token counts, the reference's per-token GEMV kernels
// mlp_stage1_mxfp4 / mlp_stage2_mxfp4 (tinyinfer/csrc/mlp_fp4.cu:79-142,
// 365-426): gate_up with the SiLU*up epilogue writes h, down writes out.
//
// Memory order is what decides HBM efficiency here, so the work is laid out
// around the load stream (each choice measured on MI355X):
//   * an item is 8 weight rows x 128 contiguous bytes (256 K elements): one
//     dwordx4 load per lane, 8 full cache lines per instruction;
//   * a row group is 8 rows x all of K (x both matrices for gate_up).
//     Workgroup g takes row groups g, g+G, g+2G, ...; wave w of it takes a
//     contiguous run of the row group's K segments (1/8 of K), so the whole
//     chip reads one band of each matrix at a time;
//   * a wave's share of a row group is cut into units of SPU segments; the
//     wave keeps two units in flight (loads of unit u+2 are issued as soon as
//     unit u has been multiplied);
//   * one 8-wave workgroup per CU and no workgroup barrier in the stream: at
//     the end of a row group a wave stores its partial sums in an LDS slot of
//     the row group and bumps an LDS counter; the last wave to get there sums
//     the slots in a fixed order (bit-reproducible) and runs the epilogue;
//   * x and the e8m0 bytes of all of the workgroup's row groups are staged in
//     LDS by a prologue, with whole-line loads issued before the first
//     weights (loads complete in issue order, so anything issued after the
//     weights would wait for them).  Scale bytes fetched per unit instead cost
//     about as many cache-line requests as the weights themselves.
//
// MFMA mapping ("8 rows x 128 B"): lane l holds weight row l&7, 32-element K
// block l>>3 of the item.  With these as the A operand of
// v_mfma_f32_16x16x32_bf16, MFMA row i is weight row i&7 over K blocks
// {2g + (i>>3)}; the B operand in lane l carries token (l%16)&7 at lane l's
// own K block, so y[row r][token t] = C[r][t] + C[r+8][t+8] (r, t < 8).
#include <cstdlib>
#include <type_traits>

#include "mxfp4_common.hpp"
#include "mxfp4_launch.hpp"

namespace tinyinfer {

namespace {

constexpr int kNW = 8;            // waves per workgroup
constexpr int kItemK = 256;       // K elements per item (one 128-byte segment per row)
constexpr int kMaxSpw = 32;       // max K segments per wave per row group (K <= 65536)
constexpr int kXPre = 4;          // x chunks per thread loaded ahead of the weights
constexpr int kSPre = 4;          // scale chunks per thread loaded ahead of the weights

struct StreamArgs {
  const uint16_t* x;      // [M, K] activations (x for gate_up, h for down)
  const uint8_t* w0;      // [R, K/2] gate (or down)
  const uint8_t* s0;      // [R, K/32]
  const uint8_t* w1;      // [R, K/2] up (gate_up only)
  const uint8_t* s1;
  uint16_t* out;          // [M, R]
  int M, K, R;
  int segs;               // K / kItemK
  int spu;                // segments per unit
  int parts;              // units per row group per wave
  int rgroups;            // R / 8
  int nrg_max;            // max row groups per workgroup
  int xs_stride;          // LDS bytes per staged token row
  int ss_stride;          // LDS bytes per staged scale row (K/32 + 16: rows fall in different banks)
  int xreg;               // activations in VGPRs (else staged in LDS)
  int lds_scl, lds_red, lds_cnt, lds_out;   // LDS byte offsets
  const uint16_t* res;    // down only: residual [M, R] added to out, or null
  const uint16_t* norm_w; // gate_up only: RMSNorm weight [K] applied to x in LDS, or null
  float eps;
  uint16_t* xn;           // with norm_w: workgroup 0 writes the normalized x here [M, K]
  int lds_nw, lds_nsum;   // with norm_w: LDS copy of the weight, partial sums
};


// Wave w's segment run [lo, hi) of a row group (same for both matrices).
__device__ __forceinline__ void seg_run(const StreamArgs& a, int wave, int& lo, int& hi) {
  lo = a.segs * wave / kNW;
  hi = a.segs * (wave + 1) / kNW;
}

// Segments [s0, s0 + nu) of the wave's run belong to unit `part`.
__device__ __forceinline__ void unit_segs(const StreamArgs& a, int wave, int part, int spu, int& s0, int& nu) {
  int lo, hi;
  seg_run(a, wave, lo, hi);
  s0 = lo + part * spu;
  const int e = s0 + spu < hi ? s0 + spu : hi;
  nu = e > s0 ? e - s0 : 0;
}

// A unit's weight items (matrix-major).  A fixed instruction count: a slot
// outside the unit repeats the load of a segment the unit (or a neighbouring
// wave) does read, and is not used.  Repeats of real addresses hit in cache;
// a common dummy address instead would send every wave of the chip to one L2
// channel.
template <int SPU, bool GATEUP>
__device__ __forceinline__ void issue_unit(const StreamArgs& a, int rg, int part, int wave,
                                           u32x4_t (&wv)[(GATEUP ? 2 : 1) * SPU]) {
  constexpr int kMats = GATEUP ? 2 : 1;
  const int lane = threadIdx.x & 63;
  const int r8 = lane & 7, q8 = lane >> 3;
  int s0, nu;
  unit_segs(a, wave, part, SPU, s0, nu);
  if (nu == 0) {                 // a wave with a shorter run: repeat its first segment
    int hi;
    seg_run(a, wave, s0, hi);
  }
  const int last = nu > 0 ? nu - 1 : 0;
  const int64_t row = (int64_t)rg * 8 + r8;
#pragma unroll
  for (int k = 0; k < kMats * SPU; ++k) {
    const int mat = GATEUP ? k / SPU : 0;
    const int sg = k - mat * SPU < last ? k - mat * SPU : last;
    const uint8_t* w = mat ? a.w1 : a.w0;
    const uint8_t* wp = w + row * (a.K / 2) + (int64_t)(s0 + sg) * (kItemK / 2) + 16 * q8;
    wv[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wp));
  }
  // units complete in issue order only if they are issued in program order:
  // keep the scheduler from interleaving two units' loads
  __builtin_amdgcn_sched_barrier(0);
}

// Multiply one unit's items into acc (FAST: every scale byte in the
// hardware-exact range -- for fp16 activations e8m0_f16_ok, the weights then
// converted to fp16 on fp16 MFMAs, otherwise exact bf16 weights against the
// activations' exact bf16 hi and lo parts; chosen once outside this body so
// each conversion sits in the same basic block as its MFMA).  Every item goes through the
// MFMA: a branch around the slots outside the unit would leave some loads
// unconsumed on one path, and the compiler then drains the whole load queue
// (vmcnt(0)) before the next issue, which serialises the pipeline.  FULL
// units (all slots inside, the common case) take no masking: a wave64 select
// costs as much as one of the four conversions an MFMA needs.  Otherwise the
// outside slots multiply zero weights by zero activations.
// xf(sg, t) returns the activation operand of segment sg of the unit, MFMA t.
template <int DT, int SPU, bool GATEUP, bool FAST, bool FULL, typename XF>
__device__ __forceinline__ void mma_unit(int nu, const u32x4_t (&wv)[(GATEUP ? 2 : 1) * SPU],
                                         const uint32_t (&sb)[(GATEUP ? 2 : 1) * SPU], const XF& xf,
                                         f32x4_t (&acc)[2]) {
  constexpr int kMats = GATEUP ? 2 : 1;
#pragma unroll
  for (int mat = 0; mat < kMats; ++mat) {
#pragma unroll
    for (int sg = 0; sg < SPU; ++sg) {
      const int k = mat * SPU + sg;
      const bool live = FULL || sg < nu;                    // wave-uniform
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t wq = live ? wv[k][t] : 0u;           // e2m1 code 0 is +0
        const u32x4_t wa = !FAST ? dq8_bf16_exact(wq, sb[k])
                                 : DT == kBF16 ? dq8_bf16_fast(wq, sb[k]) : dq8_f16_fast(wq, sb[k]);
        const u32x4_t xr = xf(live ? sg : 0, t);
        const u32x4_t xb = live ? xr : u32x4_t{0u, 0u, 0u, 0u};   // 0 * (inf or nan in x) stays out
        if constexpr (DT == kBF16) {
          acc[mat] = mfma16x16x32(wa, xb, acc[mat]);
        } else if constexpr (FAST) {
          acc[mat] = mfma16x16x32_f16(wa, xb, acc[mat]);
        } else {
          u32x4_t xh, xlo;
          f16x8_split_bf16(xb, xh, xlo);
          acc[mat] = mfma16x16x32(wa, xlo, mfma16x16x32(wa, xh, acc[mat]));
        }
      }
    }
  }
}

// Scale bytes of unit `part` of the workgroup's li-th row group, from the
// LDS copy ([li][mat][row] rows of ss_stride bytes), then the multiply.
// The activations come from xf(segment of the unit, t).
template <int DT, int SPU, bool GATEUP, typename XF>
__device__ __forceinline__ void compute_unit(const StreamArgs& a, int wave, int li, int part,
                                             const u32x4_t (&wv)[(GATEUP ? 2 : 1) * SPU], const uint8_t* scl,
                                             const XF& xf, f32x4_t (&acc)[2]) {
  constexpr int kMats = GATEUP ? 2 : 1;
  const int lane = threadIdx.x & 63;
  const int r8 = lane & 7, q8 = lane >> 3;
  int s0, nu;
  unit_segs(a, wave, part, SPU, s0, nu);
  uint32_t sb[kMats * SPU];
  bool ok = true;
#pragma unroll
  for (int k = 0; k < kMats * SPU; ++k) {
    const int mat = GATEUP ? k / SPU : 0;
    const int sg = k - mat * SPU;
    const uint8_t* srow = scl + ((li * kMats + mat) * 8 + r8) * a.ss_stride;
    sb[k] = sg < nu ? (uint32_t)srow[(s0 + sg) * 8 + q8] : 127u;
    ok = ok && (DT == kBF16 ? e8m0_fast_ok(sb[k]) : e8m0_f16_ok(sb[k]));
  }
  if (wave_all(ok)) {
    if (nu == SPU) mma_unit<DT, SPU, GATEUP, true, true>(nu, wv, sb, xf, acc);
    else mma_unit<DT, SPU, GATEUP, true, false>(nu, wv, sb, xf, acc);
  } else {
    mma_unit<DT, SPU, GATEUP, false, false>(nu, wv, sb, xf, acc);
  }
}

// Fold C[r][t] + C[r+8][t+8] and store this wave's partial (rows 4g..4g+3,
// token t) into LDS.
__device__ __forceinline__ void store_partial(const f32x4_t& acc, float* red, int M) {
  const int lane = threadIdx.x & 63;
  f32x4_t part;
#pragma unroll
  for (int v = 0; v < 4; ++v) part[v] = acc[v] + __shfl_down(acc[v], 40, 64);
  const int c = lane & 15, g = lane >> 4;
  if (c < 8 && g < 2 && c < M) *reinterpret_cast<f32x4_t*>(red + c * 8 + 4 * g) = part;
}

// XREG: the wave's activations (its K range of every token, up to PMAX
// units' worth) are copied from LDS into VGPRs once: a wave's K range is the
// same in every row group, and reading them from LDS for every MFMA moves
// twice the bytes the MFMAs consume (64 lanes x 16 B per instruction, 8 waves
// sharing one LDS), which made gate_up's multiply LDS-bound.  The down stage
// (longer K range per wave, more registers) measured faster reading LDS.
// D units in flight per wave: 2 measured best (3 was slower everywhere).
template <int DT, int SPU, bool GATEUP, int D, bool XREG, int PMAX>
__global__ __launch_bounds__(kNW * 64, 1) void stream_kernel(StreamArgs a) {
  static_assert(D == 2 || D == 3, "units in flight per wave");
  static_assert(PMAX == 1 || PMAX == 2, "units per row group with activations in registers");
  static_assert(!XREG || DT == kBF16, "fp16 activations are split into two bf16 operands in LDS");
  constexpr int kMats = GATEUP ? 2 : 1;
  constexpr int kItems = kMats * SPU;
  constexpr int kThreads = kNW * 64;
  constexpr int kNX = XREG ? PMAX * SPU : 1;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int G = gridDim.x;
  const int g = blockIdx.x;
  uint8_t* scl = lds + a.lds_scl;                                           // [nrg_max][kMats][8][ss_stride]
  float* red = reinterpret_cast<float*>(lds + a.lds_red);                   // [nrg_max][kNW][kMats][64]
  unsigned int* cnt = reinterpret_cast<unsigned int*>(lds + a.lds_cnt);    // [nrg_max]
  uint16_t* outs = reinterpret_cast<uint16_t*>(lds + a.lds_out);           // [nrg_max][M][8]
  const int P = a.parts;
  const int nrg = (a.rgroups - g + G - 1) / G;
  const int units = nrg * P;
  const int q8 = lane >> 3;
  const int tok = ((lane & 15) & 7) < a.M ? ((lane & 15) & 7) : a.M - 1;   // MFMA columns >= M are discarded
  int lo, hi;
  seg_run(a, wave, lo, hi);

  for (int i = threadIdx.x; i < a.nrg_max; i += kThreads) cnt[i] = 0u;

  // Prologue: x and the scale bytes of all of this workgroup's row groups go
  // to LDS, loaded before the first weights (loads complete in issue order,
  // so anything issued after the weights would wait for them).
  // LDS x chunk c (16 bytes): token c / (K/8), elements 8 (c % (K/8)).
  const int x_row = a.K / 8;
  const int nxc = a.M * x_row;
  auto x_src = [&](int c) {
    const int cc = c < nxc ? c : nxc - 1;
    const int t = cc / x_row, k8 = cc - t * x_row;
    return reinterpret_cast<const u32x4_t*>(a.x + (int64_t)t * a.K + 8 * k8);
  };
  auto x_dst = [&](int c) {
    const int t = c / x_row, k8 = c - t * x_row;
    return reinterpret_cast<u32x4_t*>(lds + t * a.xs_stride + 16 * k8);
  };
  // scale chunk c (16 bytes): block (li, mat) = c / (K/64), which is rows
  // rg*8 .. rg*8+7 of that matrix's scales, contiguous in memory
  const int s_blk = a.K / 64;
  const int nsc = nrg * kMats * s_blk;
  auto s_src = [&](int c) {
    const int cc = c < nsc ? c : nsc - 1;
    const int blk = cc / s_blk, off = 16 * (cc - blk * s_blk);
    const int li = blk / kMats, mat = blk - li * kMats;
    const uint8_t* sp = mat ? a.s1 : a.s0;
    return reinterpret_cast<const u32x4_t*>(sp + (int64_t)(g + li * G) * 8 * (a.K / 32) + off);
  };
  auto s_dst = [&](int c) {
    const int blk = c / s_blk, off = 16 * (c - blk * s_blk);
    const int row = off / (a.K / 32), col = off - row * (a.K / 32);
    return reinterpret_cast<u32x4_t*>(scl + (blk * 8 + row) * a.ss_stride + col);
  };
  // chunks beyond the per-thread preload (large M, many row groups per
  // workgroup): these wait for their own loads, before any weight is issued
  for (int c0 = threadIdx.x + kXPre * kThreads; c0 < nxc; c0 += 4 * kThreads) {
    u32x4_t v[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) v[b] = *x_src(c0 + b * kThreads);
#pragma unroll
    for (int b = 0; b < 4; ++b)
      if (c0 + b * kThreads < nxc) *x_dst(c0 + b * kThreads) = v[b];
  }
  for (int c0 = threadIdx.x + kSPre * kThreads; c0 < nsc; c0 += 4 * kThreads) {
    u32x4_t v[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) v[b] = *s_src(c0 + b * kThreads);
#pragma unroll
    for (int b = 0; b < 4; ++b)
      if (c0 + b * kThreads < nsc) *s_dst(c0 + b * kThreads) = v[b];
  }
  u32x4_t xv[kXPre], sv[kSPre];
#pragma unroll
  for (int b = 0; b < kXPre; ++b) xv[b] = *x_src(threadIdx.x + b * kThreads);
#pragma unroll
  for (int b = 0; b < kSPre; ++b) sv[b] = *s_src(threadIdx.x + b * kThreads);
  // RMSNorm weights (gate_up with a norm): LDS chunk c = elements 8c .. 8c+7,
  // loaded before the first weights like x
  const bool norm = GATEUP && a.norm_w != nullptr;
  const int nwc = a.K / 8;
  u32x4_t nv[2];
  if (norm) {
    for (int c0 = threadIdx.x + 2 * kThreads; c0 < nwc; c0 += kThreads)
      *reinterpret_cast<u32x4_t*>(lds + a.lds_nw + 16 * c0) = *reinterpret_cast<const u32x4_t*>(a.norm_w + 8 * c0);
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int c = threadIdx.x + b * kThreads;
      nv[b] = *reinterpret_cast<const u32x4_t*>(a.norm_w + 8 * (c < nwc ? c : nwc - 1));
    }
  }

  // the first D units in flight (separate named buffers: an array indexed by
  // the pipeline slot ends up in scratch)
  struct Buf {
    u32x4_t w[kItems];
  };
  Buf b0, b1, b2;
  auto issue = [&](Buf& b, int u) {
    const int uu = u < units ? u : units - 1;    // past the end: repeat the last unit's loads
    const int rgi = uu / P, part = uu - rgi * P;
    issue_unit<SPU, GATEUP>(a, g + rgi * G, part, wave, b.w);
  };
  issue(b0, 0);
  issue(b1, 1);
  if constexpr (D > 2) issue(b2, 2);

#pragma unroll
  for (int b = 0; b < kXPre; ++b)
    if (threadIdx.x + b * kThreads < nxc) *x_dst(threadIdx.x + b * kThreads) = xv[b];
#pragma unroll
  for (int b = 0; b < kSPre; ++b)
    if (threadIdx.x + b * kThreads < nsc) *s_dst(threadIdx.x + b * kThreads) = sv[b];
  if (norm) {
#pragma unroll
    for (int b = 0; b < 2; ++b)
      if (threadIdx.x + b * kThreads < nwc) *reinterpret_cast<u32x4_t*>(lds + a.lds_nw + 16 * (threadIdx.x + b * kThreads)) = nv[b];
  }
  // every wave's LDS stores (counters, x, scales) are done before any wave
  // reads them: wait for LDS only (a full __syncthreads would also wait for
  // the weights in flight)
  auto lds_barrier = [] {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);    // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  lds_barrier();

  // RMSNorm of x in LDS while the first weights are in flight (the
  // reference's post_attention_layernorm, tinyinfer/csrc/rmsnorm.cu:10-54):
  // per token the sum of squares in fp32 (per thread, over the wave, then
  // over the waves in order), inv = rsqrt(sum / K + eps), x <- round(w * x *
  // inv).  Every workgroup normalizes its own copy.
  if (norm) {
    float* nsum = reinterpret_cast<float*>(lds + a.lds_nsum);   // [kNW][8] partials, then [8] inverse rms
    for (int t = 0; t < a.M; ++t) {
      float sq = 0.f;
      for (int c = threadIdx.x; c < nwc; c += kThreads) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(lds + t * a.xs_stride + 16 * c);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float lo = act_to_f32<DT>((uint16_t)(v[j] & 0xffffu)), hi = act_to_f32<DT>((uint16_t)(v[j] >> 16));
          sq += lo * lo;
          sq += hi * hi;
        }
      }
      sq = wave_sum64(sq);
      if (lane == 0) nsum[wave * 8 + t] = sq;
    }
    lds_barrier();
    if (threadIdx.x < a.M) {
      float tot = 0.f;
      for (int w = 0; w < kNW; ++w) tot += nsum[w * 8 + threadIdx.x];
      nsum[kNW * 8 + threadIdx.x] = rsqrtf(tot / (float)a.K + a.eps);
    }
    lds_barrier();
    for (int t = 0; t < a.M; ++t) {
      const float inv = nsum[kNW * 8 + t];
      for (int c = threadIdx.x; c < nwc; c += kThreads) {
        u32x4_t* xp = reinterpret_cast<u32x4_t*>(lds + t * a.xs_stride + 16 * c);
        const u32x4_t v = *xp;
        const u32x4_t gw = *reinterpret_cast<const u32x4_t*>(lds + a.lds_nw + 16 * c);
        u32x4_t o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float lo = act_to_f32<DT>((uint16_t)(gw[j] & 0xffffu)) * act_to_f32<DT>((uint16_t)(v[j] & 0xffffu)) * inv;
          const float hi = act_to_f32<DT>((uint16_t)(gw[j] >> 16)) * act_to_f32<DT>((uint16_t)(v[j] >> 16)) * inv;
          o[j] = (uint32_t)f32_to_act<DT>(lo) | ((uint32_t)f32_to_act<DT>(hi) << 16);
        }
        *xp = o;
      }
    }
    lds_barrier();
  }

  // XREG: segment j of the wave's run, MFMA t: x[tok][256 (lo + j) + 32 q8 + 8 t],
  // copied once from LDS; segments past the run read a valid address and are
  // never used unmasked.
  const uint8_t* xrow = lds + tok * a.xs_stride;
  u32x4_t xr[kNX][4];
  if constexpr (XREG) {
#pragma unroll
    for (int j = 0; j < kNX; ++j) {
      const int seg = lo + j < a.segs ? lo + j : a.segs - 1;
#pragma unroll
      for (int t = 0; t < 4; ++t)
        xr[j][t] = *reinterpret_cast<const u32x4_t*>(xrow + 2 * (seg * kItemK + 32 * q8 + 8 * t));
    }
  }

  // after a row group: partials into its slot, count, and the last wave of
  // the workgroup to get here runs the epilogue into LDS
  auto finish_rg = [&](int li, const f32x4_t (&acc)[2]) {
    float* slot = red + (int64_t)li * (kNW * kMats * 64);
#pragma unroll
    for (int m = 0; m < kMats; ++m) store_partial(acc[m], slot + (wave * kMats + m) * 64, a.M);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    unsigned int old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(&cnt[li], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
    old = __shfl(old, 0, 64);
    if (old == kNW - 1) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
      // epilogue: 8 rows x M tokens, one lane each, fixed-order sum over the waves
      if (lane < 8 * a.M) {
        const int t = lane >> 3, r = lane & 7;
        float y0 = 0.f, y1 = 0.f;
        for (int w = 0; w < kNW; ++w) {
          y0 += slot[(w * kMats + 0) * 64 + t * 8 + r];
          if (GATEUP) y1 += slot[(w * kMats + 1) * 64 + t * 8 + r];
        }
        const float v = GATEUP ? silu_f32(y0) * y1 : y0;
        outs[(li * a.M + t) * 8 + r] = f32_to_act<DT>(v);
      }
    }
  };

  // unit u = (row group g + (u / P) G, part u % P) uses buffer u % D
  f32x4_t acc[2];
  auto compute = [&](Buf& b, int rgi, int part) {
    if constexpr (XREG) {
      // part selects which of the wave's segments: a compile-time index into
      // the activation registers
      auto run = [&](auto part_tag) {
        constexpr int PT = decltype(part_tag)::value;
        auto xf = [&](int sg, int t) { return xr[PT * SPU + sg][t]; };
        compute_unit<DT, SPU, GATEUP>(a, wave, rgi, PT, b.w, scl, xf, acc);
      };
      if (PMAX == 1 || part == 0) run(std::integral_constant<int, 0>{});
      else run(std::integral_constant<int, PMAX - 1>{});
    } else {
      auto xf = [&](int sg, int t) {
        int s0, nu;
        unit_segs(a, wave, part, SPU, s0, nu);
        return *reinterpret_cast<const u32x4_t*>(xrow + 2 * ((s0 + sg) * kItemK + 32 * q8 + 8 * t));
      };
      compute_unit<DT, SPU, GATEUP>(a, wave, rgi, part, b.w, scl, xf, acc);
    }
  };
  // multiply unit u from buffer b; with ISSUE, then load unit u + D into b
  auto step = [&](Buf& b, int u, auto issue_tag) {
    const int rgi = u / P, part = u - rgi * P;
    if (part == 0) acc[0] = acc[1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    compute(b, rgi, part);
    if constexpr (decltype(issue_tag)::value) issue(b, u + D);
    if (part == P - 1) finish_rg(rgi, acc);
  };
  constexpr std::true_type kIssue{};
  constexpr std::false_type kLast{};
  // One exit, at the top: a break between the steps would join the loop's
  // back edge with a path on which the buffers were issued in another order,
  // and the compiler's load-queue bookkeeping would then wait for all of them
  // at the top of every iteration.
  int u = 0;
  if constexpr (D == 2) {
    // every load issued is a unit the wave multiplies: the loop runs while
    // units u + 2 and u + 3 exist and the last two or three units are peeled
    // into straight-line tails (loads past the end cost their bytes and one
    // more memory latency before the wave can end; an issue under a condition
    // inside the loop would drain the load queue at every step)
    for (; u + 3 < units; u += 2) {
      step(b0, u, kIssue);
      step(b1, u + 1, kIssue);
    }
    const int left = units - u;
    if (left == 3) {
      step(b0, u, kIssue);
      step(b1, u + 1, kLast);
      step(b0, u + 2, kLast);
    } else if (left == 2) {
      step(b0, u, kLast);
      step(b1, u + 1, kLast);
    } else if (left == 1) {
      step(b0, u, kLast);
    }
  } else {
    for (; u + D - 1 < units; u += D) {
      step(b0, u, kIssue);
      step(b1, u + 1, kIssue);
      step(b2, u + 2, kIssue);
    }
    if (u < units) step(b0, u, kIssue);
    if (u + 1 < units) step(b1, u + 1, kIssue);
  }

  // the row groups' outputs, staged in LDS by their last waves (a global
  // store inside the stream would make the load-queue accounting
  // path-dependent, see mma_unit)
  __syncthreads();
  for (int i = threadIdx.x; i < nrg * a.M * 8; i += kThreads) {
    const int li = i / (a.M * 8), rem = i - li * a.M * 8;
    const int t = rem >> 3, r = rem & 7;
    const int64_t idx = (int64_t)t * a.R + (int64_t)(g + li * G) * 8 + r;
    a.out[idx] = with_residual<DT>(outs[i], a.res, idx);
  }
  if (norm && g == 0 && a.xn) {
    for (int c = threadIdx.x; c < a.M * nwc; c += kThreads) {
      const int t = c / nwc, cc = c - t * nwc;
      *reinterpret_cast<u32x4_t*>(a.xn + (int64_t)t * a.K + 8 * cc) =
          *reinterpret_cast<const u32x4_t*>(lds + t * a.xs_stride + 16 * cc);
    }
  }
}

struct DevCaps {
  int cus = 0;
  int64_t max_lds = 0;
};

DevCaps caps() {
  const DeviceInfo i = device_info();
  DevCaps d;
  d.cus = i.cus;
  d.max_lds = i.lds_per_block;
  return d;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }


// Segments per unit for a wave run of up to `spw` segments: the least of
// load slots (units x segments per unit, the last unit padded) plus 0.8 slot
// per unit (its issue, scale reads and pipeline step), at most 3 segments per
// gate_up unit (6 weight items; 2 for fp16 activations, whose split operands
// need more registers) and 4 per down unit.  Measured at K = 5120 (3
// segments per wave): one 3-segment unit beats a 2 + 1 split by 17%.
// TINYINFER_STREAM_SPU_GU / _DN override it for tuning.
int stream_spu(bool gateup, bool bf16, int spw) {
  const int forced = option(gateup ? kOptStreamSpuGu : kOptStreamSpuDn);
  if (forced > 0) return gateup && !bf16 && forced > 2 ? 2 : forced;
  const int cap = gateup ? (bf16 ? 3 : 2) : 4;
  int best = 1;
  double best_cost = 1.8 * spw;
  for (int spu = 2; spu <= cap; ++spu) {
    const int units = (spw + spu - 1) / spu;
    const double cost = units * spu + 0.8 * units;
    if (cost < best_cost) {
      best = spu;
      best_cost = cost;
    }
  }
  return best;
}

constexpr int kDepth = 2;         // units in flight per wave

// Activations in registers for gate_up (TINYINFER_STREAM_XREG=0 turns it off).
bool stream_xreg_allowed(bool gateup) {
  return option(kOptStreamXreg) == 1 && gateup;
}

// Geometry of one stage; false when the streaming kernel does not apply.
// force_grid > 0 fixes the grid (the fused decode kernel runs both stages on
// the gate_up stage's grid).
bool plan(int64_t M, int64_t K, int64_t R, bool gateup, bool bf16, const DevCaps& d, StreamArgs& a, int& grid,
          int64_t& lds, int force_grid = 0, bool norm = false) {
  // K % 512: a row group's scale rows split into whole 16-byte chunks
  if (d.cus < 1 || M < 1 || M > 8 || K % (2 * kItemK) != 0 || R % 8 != 0) return false;
  if (K > (1 << 20) || R > (1 << 24)) return false;
  const int mats = gateup ? 2 : 1;
  a.M = (int)M;
  a.K = (int)K;
  a.R = (int)R;
  a.segs = (int)(K / kItemK);
  const int spw = (a.segs + kNW - 1) / kNW;
  if (spw > kMaxSpw) return false;
  a.spu = stream_spu(gateup, bf16, spw);
  a.parts = (spw + a.spu - 1) / a.spu;
  a.rgroups = (int)(R / 8);
  grid = force_grid > 0 ? force_grid : (d.cus < a.rgroups ? d.cus : a.rgroups);
  a.nrg_max = (a.rgroups + grid - 1) / grid;
  a.xs_stride = (int)(2 * K + 16);
  a.ss_stride = (int)(K / 32 + 16);
  // register budget (2 waves per SIMD, 256 VGPRs each): one unit's activations
  a.xreg = bf16 && stream_xreg_allowed(gateup) && a.parts == 1;
  a.lds_scl = (int)(M * a.xs_stride);
  a.lds_red = a.lds_scl + a.nrg_max * mats * 8 * a.ss_stride;
  a.lds_cnt = a.lds_red + a.nrg_max * kNW * mats * 64 * 4;
  a.lds_out = a.lds_cnt + 4 * ((a.nrg_max + 3) & ~3);
  lds = a.lds_out + a.nrg_max * (int)M * 8 * 2;
  a.norm_w = nullptr;
  a.eps = 0.f;
  a.xn = nullptr;
  a.lds_nw = a.lds_nsum = 0;
  if (norm) {
    a.lds_nw = (int)((lds + 15) & ~int64_t(15));
    a.lds_nsum = a.lds_nw + (int)(2 * K);
    lds = a.lds_nsum + 4 * (kNW * 8 + 8);
  }
  return lds <= d.max_lds;
}

template <int DT, bool GATEUP>
hipError_t launch(const StreamArgs& a, int64_t lds, int grid, hipStream_t st) {
  auto go = [&](auto kern) -> hipError_t {
    if (lds > 64 * 1024 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess) {
      (void)hipGetLastError();
      return hipErrorNotSupported;
    }
    kern<<<grid, kNW * 64, (size_t)lds, st>>>(a);
    return hipGetLastError();
  };
  auto depth = [&](auto spu_tag) -> hipError_t {
    constexpr int S = decltype(spu_tag)::value;
    if constexpr (DT == kBF16 && GATEUP) {
      if (a.xreg) return go(stream_kernel<DT, S, GATEUP, kDepth, true, 1>);
    }
    return go(stream_kernel<DT, S, GATEUP, kDepth, false, 1>);
  };
  if (a.spu <= 1) return depth(std::integral_constant<int, 1>{});
  if constexpr (GATEUP) {
    if (a.spu == 3) return depth(std::integral_constant<int, 3>{});
    return depth(std::integral_constant<int, 2>{});
  } else {
    if (a.spu == 2) return depth(std::integral_constant<int, 2>{});
    if (a.spu == 3) return depth(std::integral_constant<int, 3>{});
    return depth(std::integral_constant<int, 4>{});
  }
}

template <int DT, bool GATEUP>
hipError_t run_stage(const uint16_t* x, const uint8_t* w0, const uint8_t* s0, const uint8_t* w1,
                     const uint8_t* s1, int64_t M, int64_t K, int64_t R, uint16_t* out, hipStream_t st,
                     const uint16_t* res = nullptr, const uint16_t* norm_w = nullptr, float eps = 0.f,
                     uint16_t* xn = nullptr) {
  StreamArgs a;
  int grid = 0;
  int64_t lds = 0;
  const bool norm = GATEUP && norm_w != nullptr;
  if (!plan(M, K, R, GATEUP, DT == kBF16, caps(), a, grid, lds, 0, norm)) return hipErrorNotSupported;
  if (norm) {
    a.norm_w = norm_w;
    a.eps = eps;
    a.xn = xn;
  }
  a.x = x;
  a.w0 = w0;
  a.s0 = s0;
  a.w1 = GATEUP ? w1 : w0;
  a.s1 = GATEUP ? s1 : s0;
  a.out = out;
  a.res = GATEUP ? nullptr : res;
  return launch<DT, GATEUP>(a, lds, grid, st);
}

// ===================================================================== fused
//
// Fused decode (TI_PATH_DECODE, and AUTO for M <= 4): both stages in one
// launch, one workgroup per CU, all resident.  Phase 1 is the gate_up stream
// above; each workgroup then publishes its rows of h with agent-scope stores
// (performed at the device's coherence point, so other XCDs' L2s never hold
// them) and, once they have completed, sets its flag to the launch's epoch.
// Before waiting for the other workgroups' flags it issues all of its down
// weight loads (at most 4 units per wave, registers only), so the down
// weights stream while the slowest workgroups finish gate_up.  It then reads
// h with agent-scope loads into LDS and runs the down stream from registers.
//
// The flags hold the epoch of the last launch that reached them, so they are
// never reset: a launch reads the epoch E, waits for flag == E + 1, and
// workgroup 0 stores E + 1 as the new epoch after its own wait (by then every
// workgroup has read E).  The wait is a bounded spin: if it ever gives up
// (workgroups not all resident), the timeout is counted, the launch's
// results are invalid, but the kernel ends; the wait also sets a sticky
// poison word, so a workgroup that starts late, and every later launch,
// exits at entry without writing anything (a late workgroup would otherwise
// read the advanced epoch and publish a flag the next launch takes for its
// own) until decode_reset() clears the state.  Launches must not overlap on
// a device.
constexpr int kFusedMaxGrid = 1024;
constexpr int kFusedMaxUnits2 = 4;
__device__ uint32_t g_fused_flags[kFusedMaxGrid];
// [0] epoch of the last completed launch, [1] poisoned (nonzero after a wait
// gave up): read together as one 64-bit word at kernel entry
__device__ __attribute__((aligned(8))) uint32_t g_fused_ctl[2];
__device__ uint32_t g_fused_timeouts;

struct FusedArgs {
  StreamArgs g;           // gate_up: x -> h (g.out is tmp)
  StreamArgs d;           // down: h -> out
  uint32_t spin_limit;
};

__device__ __forceinline__ uint32_t agent_load(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// After a row group: partials into its LDS slot, count, and the last wave of
// the workgroup to get here runs the epilogue into outs.
template <int DT, bool GATEUP>
__device__ __forceinline__ void finish_row_group(const StreamArgs& a, float* red, unsigned int* cnt,
                                                 uint16_t* outs, int li, int wave, const f32x4_t (&acc)[2]) {
  constexpr int kMats = GATEUP ? 2 : 1;
  const int lane = threadIdx.x & 63;
  float* slot = red + (int64_t)li * (kNW * kMats * 64);
#pragma unroll
  for (int m = 0; m < kMats; ++m) store_partial(acc[m], slot + (wave * kMats + m) * 64, a.M);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  unsigned int old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(&cnt[li], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
  old = __shfl(old, 0, 64);
  if (old == kNW - 1) {
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    if (lane < 8 * a.M) {
      const int t = lane >> 3, r = lane & 7;
      float y0 = 0.f, y1 = 0.f;
      for (int w = 0; w < kNW; ++w) {
        y0 += slot[(w * kMats + 0) * 64 + t * 8 + r];
        if (GATEUP) y1 += slot[(w * kMats + 1) * 64 + t * 8 + r];
      }
      const float v = GATEUP ? silu_f32(y0) * y1 : y0;
      outs[(li * a.M + t) * 8 + r] = f32_to_act<DT>(v);
    }
  }
}

template <int DT, int SPU1, int SPU2, bool XREG1>
__global__ __launch_bounds__(kNW * 64, 1) void fused_kernel(FusedArgs f) {
  constexpr int kItems1 = 2 * SPU1;
  constexpr int kItems2 = SPU2;
  constexpr int kThreads = kNW * 64;
  const StreamArgs& A = f.g;
  const StreamArgs& B = f.d;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int G = gridDim.x;
  const int g = blockIdx.x;
  const int q8 = lane >> 3;
  const uint64_t ctl = __hip_atomic_load(reinterpret_cast<const uint64_t*>(g_fused_ctl), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
  // after a wait that gave up, every later launch leaves its outputs alone
  // (the flags can no longer be trusted) until the host resets the state
  if (__builtin_amdgcn_readfirstlane((uint32_t)(ctl >> 32)) != 0u) return;
  const uint32_t epoch = __builtin_amdgcn_readfirstlane((uint32_t)ctl);

  // phase 1 LDS (x, scales, partials, counters, outputs) from 0; phase 2's
  // scale rows at B.lds_scl (past both phases' other areas); phase 2's x (h),
  // partials, counters and outputs from 0 again once phase 1 is done.
  uint8_t* scl1 = lds + A.lds_scl;
  float* red1 = reinterpret_cast<float*>(lds + A.lds_red);
  unsigned int* cnt1 = reinterpret_cast<unsigned int*>(lds + A.lds_cnt);
  uint16_t* outs1 = reinterpret_cast<uint16_t*>(lds + A.lds_out);
  uint8_t* scl2 = lds + B.lds_scl;
  float* red2 = reinterpret_cast<float*>(lds + B.lds_red);
  unsigned int* cnt2 = reinterpret_cast<unsigned int*>(lds + B.lds_cnt);
  uint16_t* outs2 = reinterpret_cast<uint16_t*>(lds + B.lds_out);

  const int P1 = A.parts, P2 = B.parts;
  const int nrg1 = (A.rgroups - g + G - 1) / G;
  const int units1 = nrg1 * P1;
  const int nrg2 = g < B.rgroups ? (B.rgroups - g + G - 1) / G : 0;
  const int units2 = nrg2 * P2;
  const int tok = ((lane & 15) & 7) < A.M ? ((lane & 15) & 7) : A.M - 1;
  int lo1, hi1;
  seg_run(A, wave, lo1, hi1);

  for (int i = threadIdx.x; i < A.nrg_max; i += kThreads) cnt1[i] = 0u;

  // ---- prologue: x, phase 1 and phase 2 scale rows -> LDS ---------------
  const int x_row = A.K / 8;
  const int nxc = A.M * x_row;
  auto x_src = [&](int c) {
    const int cc = c < nxc ? c : nxc - 1;
    const int t = cc / x_row, k8 = cc - t * x_row;
    return reinterpret_cast<const u32x4_t*>(A.x + (int64_t)t * A.K + 8 * k8);
  };
  auto x_dst = [&](int c) {
    const int t = c / x_row, k8 = c - t * x_row;
    return reinterpret_cast<u32x4_t*>(lds + t * A.xs_stride + 16 * k8);
  };
  // scale chunk c of a stage: block (li, mat) = c / (K/64): rows rg*8 ..
  // rg*8+7 of that matrix, contiguous in memory
  const int sb1 = A.K / 64, nsc1 = nrg1 * 2 * sb1;
  const int sb2 = B.K / 64, nsc2 = nrg2 * sb2;
  auto s1_src = [&](int c) {
    const int cc = c < nsc1 ? c : nsc1 - 1;
    const int blk = cc / sb1, off = 16 * (cc - blk * sb1);
    const int li = blk >> 1, mat = blk & 1;
    return reinterpret_cast<const u32x4_t*>((mat ? A.s1 : A.s0) + (int64_t)(g + li * G) * 8 * (A.K / 32) + off);
  };
  auto s1_dst = [&](int c) {
    const int blk = c / sb1, off = 16 * (c - blk * sb1);
    const int row = off / (A.K / 32), col = off - row * (A.K / 32);
    return reinterpret_cast<u32x4_t*>(scl1 + (blk * 8 + row) * A.ss_stride + col);
  };
  auto s2_src = [&](int c) {
    const int cc = c < nsc2 ? c : (nsc2 > 0 ? nsc2 - 1 : 0);
    const int li = cc / sb2, off = 16 * (cc - li * sb2);
    const int rg = nsc2 > 0 ? g + li * G : 0;
    return reinterpret_cast<const u32x4_t*>(B.s0 + (int64_t)rg * 8 * (B.K / 32) + off);
  };
  auto s2_dst = [&](int c) {
    const int li = c / sb2, off = 16 * (c - li * sb2);
    const int row = off / (B.K / 32), col = off - row * (B.K / 32);
    return reinterpret_cast<u32x4_t*>(scl2 + (li * 8 + row) * B.ss_stride + col);
  };
  auto sync_copy = [&](int n, int pre, auto src, auto dst) {
    for (int c0 = threadIdx.x + pre * kThreads; c0 < n; c0 += 4 * kThreads) {
      u32x4_t v[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) v[b] = *src(c0 + b * kThreads);
#pragma unroll
      for (int b = 0; b < 4; ++b)
        if (c0 + b * kThreads < n) *dst(c0 + b * kThreads) = v[b];
    }
  };
  sync_copy(nxc, kXPre, x_src, x_dst);
  sync_copy(nsc1, kSPre, s1_src, s1_dst);
  sync_copy(nsc2, 2, s2_src, s2_dst);
  u32x4_t xv[kXPre], sv1[kSPre], sv2[2];
#pragma unroll
  for (int b = 0; b < kXPre; ++b) xv[b] = *x_src(threadIdx.x + b * kThreads);
#pragma unroll
  for (int b = 0; b < kSPre; ++b) sv1[b] = *s1_src(threadIdx.x + b * kThreads);
  if (nsc2 > 0) {
#pragma unroll
    for (int b = 0; b < 2; ++b) sv2[b] = *s2_src(threadIdx.x + b * kThreads);
  }

  struct Buf1 {
    u32x4_t w[kItems1];
  };
  Buf1 a0, a1;
  auto issue1 = [&](Buf1& b, int u) {
    const int uu = u < units1 ? u : units1 - 1;    // past the end: repeat the last unit's loads
    const int rgi = uu / P1, part = uu - rgi * P1;
    issue_unit<SPU1, true>(A, g + rgi * G, part, wave, b.w);
  };
  issue1(a0, 0);
  issue1(a1, 1);

#pragma unroll
  for (int b = 0; b < kXPre; ++b)
    if (threadIdx.x + b * kThreads < nxc) *x_dst(threadIdx.x + b * kThreads) = xv[b];
#pragma unroll
  for (int b = 0; b < kSPre; ++b)
    if (threadIdx.x + b * kThreads < nsc1) *s1_dst(threadIdx.x + b * kThreads) = sv1[b];
  if (nsc2 > 0) {
#pragma unroll
    for (int b = 0; b < 2; ++b)
      if (threadIdx.x + b * kThreads < nsc2) *s2_dst(threadIdx.x + b * kThreads) = sv2[b];
  }
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);    // lgkmcnt(0): LDS stores done, weights stay in flight
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // ---- phase 1: gate_up -------------------------------------------------
  const uint8_t* xrow1 = lds + tok * A.xs_stride;
  constexpr int kNX = XREG1 ? SPU1 : 1;
  u32x4_t xr[kNX][4];
  if constexpr (XREG1) {
#pragma unroll
    for (int j = 0; j < kNX; ++j) {
      const int seg = lo1 + j < A.segs ? lo1 + j : A.segs - 1;
#pragma unroll
      for (int t = 0; t < 4; ++t)
        xr[j][t] = *reinterpret_cast<const u32x4_t*>(xrow1 + 2 * (seg * kItemK + 32 * q8 + 8 * t));
    }
  }
  f32x4_t acc[2];
  auto step1 = [&](Buf1& b, int u) {
    const int rgi = u / P1, part = u - rgi * P1;
    if (part == 0) acc[0] = acc[1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    if constexpr (XREG1) {
      auto xf = [&](int sg, int t) { return xr[sg][t]; };
      compute_unit<DT, SPU1, true>(A, wave, rgi, 0, b.w, scl1, xf, acc);
    } else {
      auto xf = [&](int sg, int t) {
        int s0, nu;
        unit_segs(A, wave, part, SPU1, s0, nu);
        return *reinterpret_cast<const u32x4_t*>(xrow1 + 2 * ((s0 + sg) * kItemK + 32 * q8 + 8 * t));
      };
      compute_unit<DT, SPU1, true>(A, wave, rgi, part, b.w, scl1, xf, acc);
    }
    issue1(b, u + 2);
    if (part == P1 - 1) finish_row_group<DT, true>(A, red1, cnt1, outs1, rgi, wave, acc);
  };
  int u = 0;
  for (; u + 1 < units1; u += 2) {
    step1(a0, u);
    step1(a1, u + 1);
  }
  if (u < units1) step1(a0, u);

  // ---- publish this workgroup's rows of h, then its flag ---------------
  __syncthreads();
  {
    // outs1 [li][t][8 rows] bf16: 16 bytes per (li, t), two 8-byte stores
    const int n8 = nrg1 * A.M * 2;
    for (int i = threadIdx.x; i < n8; i += kThreads) {
      const int lt = i >> 1, half = i & 1;
      const int li = lt / A.M, t = lt - li * A.M;
      const uint64_t v = *reinterpret_cast<const uint64_t*>(outs1 + lt * 8 + 4 * half);
      uint64_t* dst = reinterpret_cast<uint64_t*>(A.out + (int64_t)t * A.R + (int64_t)(g + li * G) * 8 + 4 * half);
      __hip_atomic_store(dst, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);     // this thread's stores (and loads) have completed
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_store(&g_fused_flags[g], epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (units2 == 0) return;           // no down rows here; workgroup 0 always has some

  // ---- phase 2: down ------------------------------------------------------
  for (int i = threadIdx.x; i < B.nrg_max; i += kThreads) cnt2[i] = 0u;
  struct Buf2 {
    u32x4_t w[kItems2];
  };
  Buf2 b0, b1, b2, b3;
  auto issue2 = [&](Buf2& b, int v) {
    const int vv = v < units2 ? v : units2 - 1;
    const int rgi = vv / P2, part = vv - rgi * P2;
    issue_unit<SPU2, false>(B, g + rgi * G, part, wave, b.w);
  };
  // Waves 1..7 put their down loads in flight now; wave 0 first polls the
  // flags, since its poll loads would otherwise return only after its own
  // down loads (loads complete in issue order).
  if (wave != 0) {
    issue2(b0, 0);
    issue2(b1, 1);
    issue2(b2, 2);
    issue2(b3, 3);
  }

  // every workgroup's h rows: wave 0 polls the flags (bounded)
  if (wave == 0) {
    const uint32_t want = epoch + 1u;
    for (uint32_t it = 0;; ++it) {
      bool done = true;
      for (int i = lane; i < G; i += 64) done = done && agent_load(&g_fused_flags[i]) == want;
      if (wave_all(done)) break;
      if (it >= f.spin_limit) {
        if (lane == 0) {
          __hip_atomic_fetch_add(&g_fused_timeouts, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(&g_fused_ctl[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    issue2(b0, 0);
    issue2(b1, 1);
    issue2(b2, 2);
    issue2(b3, 3);
  }
  __syncthreads();
  if (g == 0 && threadIdx.x == 0)
    __hip_atomic_store(&g_fused_ctl[0], epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // h [M, I] -> LDS rows of B.xs_stride bytes, 8-byte agent-scope loads
  {
    const int per_row = B.K / 4;
    const int n8 = B.M * per_row;
    for (int i = threadIdx.x; i < n8; i += kThreads) {
      const int t = i / per_row, c = i - t * per_row;
      const uint64_t v = __hip_atomic_load(reinterpret_cast<const uint64_t*>(B.x + (int64_t)t * B.K + 4 * c),
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *reinterpret_cast<uint64_t*>(lds + t * B.xs_stride + 8 * c) = v;
    }
  }
  __syncthreads();

  // down's activations for this wave's K range (at most 2 parts of SPU2
  // segments) in VGPRs, copied once: reading LDS per MFMA made the multiply
  // LDS-bound.  With 4-segment units that would not fit; those read LDS.
  constexpr bool kXReg2 = SPU2 <= 3;
  const uint8_t* xrow2 = lds + tok * B.xs_stride;
  int lo2, hi2;
  seg_run(B, wave, lo2, hi2);
  u32x4_t xr2[kXReg2 ? 2 * SPU2 : 1][4];
  if constexpr (kXReg2) {
#pragma unroll
    for (int j = 0; j < 2 * SPU2; ++j) {
      const int seg = lo2 + j < B.segs ? lo2 + j : B.segs - 1;
#pragma unroll
      for (int t = 0; t < 4; ++t)
        xr2[j][t] = *reinterpret_cast<const u32x4_t*>(xrow2 + 2 * (seg * kItemK + 32 * q8 + 8 * t));
    }
  }
  auto step2 = [&](Buf2& b, int v) {
    const int rgi = v / P2, part = v - rgi * P2;
    if (part == 0) acc[0] = acc[1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    if constexpr (kXReg2) {
      auto run = [&](auto part_tag) {
        constexpr int PT = decltype(part_tag)::value;
        auto xf = [&](int sg, int t) { return xr2[PT * SPU2 + sg][t]; };
        compute_unit<DT, SPU2, false>(B, wave, rgi, PT, b.w, scl2, xf, acc);
      };
      if (part == 0) run(std::integral_constant<int, 0>{});
      else run(std::integral_constant<int, 1>{});
    } else {
      auto xf = [&](int sg, int t) {
        int s0, nu;
        unit_segs(B, wave, part, SPU2, s0, nu);
        return *reinterpret_cast<const u32x4_t*>(xrow2 + 2 * ((s0 + sg) * kItemK + 32 * q8 + 8 * t));
      };
      compute_unit<DT, SPU2, false>(B, wave, rgi, part, b.w, scl2, xf, acc);
    }
    if (part == P2 - 1) finish_row_group<DT, false>(B, red2, cnt2, outs2, rgi, wave, acc);
  };
  step2(b0, 0);
  if (units2 > 1) step2(b1, 1);
  if (units2 > 2) step2(b2, 2);
  if (units2 > 3) step2(b3, 3);

  __syncthreads();
  for (int i = threadIdx.x; i < nrg2 * B.M * 8; i += kThreads) {
    const int li = i / (B.M * 8), rem = i - li * B.M * 8;
    const int t = rem >> 3, r = rem & 7;
    const int64_t idx = (int64_t)t * B.R + (int64_t)(g + li * G) * 8 + r;
    B.out[idx] = with_residual<DT>(outs2[i], B.res, idx);
  }
}

// Geometry of a fused launch; false when it does not apply.
bool plan_fused(const MlpArgs& m, const DevCaps& d, FusedArgs& f, int& grid, int64_t& lds) {
  if (m.n < 1 || m.n > 4 || d.cus < 1) return false;
  const bool bf = m.dtype == kBF16;
  int64_t l1 = 0, l2 = 0;
  if (!plan(m.n, m.hidden, m.inter, true, bf, d, f.g, grid, l1)) return false;
  if (grid > kFusedMaxGrid) return false;
  int grid2 = 0;
  if (!plan(m.n, m.inter, m.hidden, false, bf, d, f.d, grid2, l2, grid)) return false;
  if (f.d.nrg_max * f.d.parts > kFusedMaxUnits2 || f.d.parts > 2) return false;
  // phase 1: [x][scl1][red1][cnt1][out1] as planned; phase 2 reuses the start
  // for [h][red2][cnt2][out2]; phase 2's scale rows after both
  StreamArgs& B = f.d;
  const int64_t p1 = l1;
  const int64_t h_bytes = (int64_t)m.n * B.xs_stride;
  B.lds_red = (int)h_bytes;
  B.lds_cnt = B.lds_red + B.nrg_max * kNW * 64 * 4;
  B.lds_out = B.lds_cnt + 4 * ((B.nrg_max + 3) & ~3);
  const int64_t p2 = B.lds_out + (int64_t)B.nrg_max * m.n * 8 * 2;
  B.lds_scl = (int)(((p1 > p2 ? p1 : p2) + 15) & ~int64_t(15));
  lds = B.lds_scl + (int64_t)B.nrg_max * 8 * B.ss_stride;
  if (lds > d.max_lds) return false;
  f.spin_limit = (uint32_t)option(kOptDecodeSpin);
  return true;
}

template <int DT>
hipError_t run_fused(const MlpArgs& m, hipStream_t st) {
  const DevCaps d = caps();
  FusedArgs f;
  int grid = 0;
  int64_t lds = 0;
  if (!plan_fused(m, d, f, grid, lds)) return hipErrorNotSupported;
  const void* p16[] = {m.x, m.gate, m.up, m.down, m.tmp, m.gate_scale, m.up_scale, m.down_scale};
  for (const void* p : p16)
    if (!aligned16(p)) return hipErrorNotSupported;
  f.g.x = static_cast<const uint16_t*>(m.x);
  f.g.w0 = m.gate;
  f.g.s0 = m.gate_scale;
  f.g.w1 = m.up;
  f.g.s1 = m.up_scale;
  f.g.out = static_cast<uint16_t*>(m.tmp);
  f.d.x = static_cast<const uint16_t*>(m.tmp);
  f.d.w0 = f.d.w1 = m.down;
  f.d.s0 = f.d.s1 = m.down_scale;
  f.d.out = static_cast<uint16_t*>(m.out);
  f.g.res = nullptr;
  f.d.res = static_cast<const uint16_t*>(m.residual);
  auto go = [&](auto kern) -> hipError_t {
    if (lds > 64 * 1024 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess) {
      (void)hipGetLastError();
      return hipErrorNotSupported;
    }
    // every workgroup must be resident at once
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kNW * 64, (size_t)lds) != hipSuccess ||
        per_cu < 1) {
      (void)hipGetLastError();
      return hipErrorNotSupported;
    }
    if ((int64_t)per_cu * d.cus < grid) return hipErrorNotSupported;
    kern<<<grid, kNW * 64, (size_t)lds, st>>>(f);
    return hipGetLastError();
  };
  auto pick2 = [&](auto s1_tag, auto xr_tag) -> hipError_t {
    constexpr int S1 = decltype(s1_tag)::value;
    constexpr bool XR = decltype(xr_tag)::value;
    switch (f.d.spu) {
      case 1: return go(fused_kernel<DT, S1, 1, XR>);
      case 2: return go(fused_kernel<DT, S1, 2, XR>);
      case 3: return go(fused_kernel<DT, S1, 3, XR>);
      default: return go(fused_kernel<DT, S1, 4, XR>);
    }
  };
  const bool xreg = DT == kBF16 && f.g.xreg;
  if (f.g.spu <= 1) {
    return xreg ? pick2(std::integral_constant<int, 1>{}, std::true_type{})
                : pick2(std::integral_constant<int, 1>{}, std::false_type{});
  }
  return xreg ? pick2(std::integral_constant<int, 2>{}, std::true_type{})
              : pick2(std::integral_constant<int, 2>{}, std::false_type{});
}

}  // namespace

bool stream_supported(const MlpArgs& a, int stage) {
  const DevCaps d = caps();
  StreamArgs sa;
  int grid = 0;
  int64_t lds = 0;
  const bool bf = a.dtype == kBF16;
  if ((stage & kStageGateUp) && !plan(a.n, a.hidden, a.inter, true, bf, d, sa, grid, lds, 0, a.norm_w != nullptr))
    return false;
  if (a.norm_w && (!aligned16(a.norm_w) || (a.xn && !aligned16(a.xn)))) return false;
  if ((stage & kStageDown) && !plan(a.n, a.inter, a.hidden, false, bf, d, sa, grid, lds)) return false;
  // 16-byte loads of activations, weights and scale rows
  const void* p16[] = {a.x, a.gate, a.up, a.down, a.tmp, a.gate_scale, a.up_scale, a.down_scale};
  for (const void* p : p16)
    if (p && !aligned16(p)) return false;
  return true;
}

hipError_t launch_stream_mlp(const MlpArgs& a, int stage, hipStream_t st) {
  const uint16_t* x = static_cast<const uint16_t*>(a.x);
  uint16_t* h = static_cast<uint16_t*>(a.tmp);
  uint16_t* y = static_cast<uint16_t*>(a.out);
  const bool bf = a.dtype == kBF16;
  if (stage & kStageGateUp) {
    const uint16_t* nw = static_cast<const uint16_t*>(a.norm_w);
    uint16_t* xn = static_cast<uint16_t*>(a.xn);
    const hipError_t e = bf ? run_stage<kBF16, true>(x, a.gate, a.gate_scale, a.up, a.up_scale, a.n, a.hidden,
                                                     a.inter, h, st, nullptr, nw, a.eps, xn)
                            : run_stage<kF16, true>(x, a.gate, a.gate_scale, a.up, a.up_scale, a.n, a.hidden,
                                                    a.inter, h, st, nullptr, nw, a.eps, xn);
    if (e != hipSuccess) return e;
  }
  if (stage & kStageDown) {
    const uint16_t* res = static_cast<const uint16_t*>(a.residual);
    return bf ? run_stage<kBF16, false>(h, a.down, a.down_scale, nullptr, nullptr, a.n, a.inter, a.hidden, y, st, res)
              : run_stage<kF16, false>(h, a.down, a.down_scale, nullptr, nullptr, a.n, a.inter, a.hidden, y, st, res);
  }
  return hipSuccess;
}

hipError_t launch_decode_mlp(const MlpArgs& a, hipStream_t st) {
  if (a.n > 4) return hipErrorNotSupported;
  return a.dtype == kBF16 ? run_fused<kBF16>(a, st) : run_fused<kF16>(a, st);
}

unsigned int decode_barrier_timeouts() {
  unsigned int v = 0;
  if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_fused_timeouts), sizeof(v)) != hipSuccess) return 0xffffffffu;
  return v;
}

hipError_t decode_reset() {
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return e;
  static const uint32_t zeros[kFusedMaxGrid] = {};
  e = hipMemcpyToSymbol(HIP_SYMBOL(g_fused_flags), zeros, sizeof(zeros));
  if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(g_fused_ctl), zeros, 2 * sizeof(uint32_t));
  if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(g_fused_timeouts), zeros, sizeof(uint32_t));
  if (e == hipSuccess) e = hipDeviceSynchronize();
  return e;
}

}  // namespace tinyinfer
