// Fused MXFP4 MLP for decode (M <= 8 tokens): gate_up, SiLU*up and down in
// ONE persistent launch.
//
// Replaces, for small token counts, the reference's two per-token GEMV
// launches mlp_stage1_mxfp4 + mlp_stage2_mxfp4 (tinyinfer/csrc/mlp_fp4.cu:
// 79-142, 365-426, launched back to back at :457-459).  At M = 1 the whole
// MLP is a ~80 MB weight stream; two dependent launches would each pay a
// ramp-up and a tail.  Here one workgroup per CU streams both phases:
//
//   prologue   x (all tokens) and every e8m0 scale the workgroup will use
//              are staged into LDS with coalesced 16-byte loads, issued before
//              any weight load (loads retire in order, so this keeps the first
//              MFMAs from waiting on the weight stream);
//   phase A    gate/up units, a depth-2 software pipeline per wave: while unit
//              k is multiplied, unit k+2's weights are in flight.  The
//              pipeline runs across the phase boundary, so the first down
//              units' weights are already streaming while gate_up finishes;
//   boundary   fixed-order LDS reduction, h = SiLU(g) * u rounded to the
//              activation dtype and stored to `tmp`, grid-wide barrier, h
//              staged into LDS;
//   phase B    down units (weights mostly already in registers), fixed-order
//              reduction, out rounded and stored.
//
// Weight layout in registers ("8 rows x 128 B"): one dwordx4 load instruction
// covers 8 weight rows x 128 contiguous bytes (8 full cache lines).  Lane l
// holds row l&7, 32-element K block l>>3 of a 256-wide K chunk.  In
// v_mfma_f32_16x16x32_bf16 with these weights as A, MFMA row i (lanes i, i+16,
// i+32, i+48) is weight row i&7 over K blocks {2g + (i>>3)}; the B operand in
// lane l carries token (l%16)&7 at lane l's own K block, so C[i][c] is a true
// partial dot product exactly when (i>>3) == (c>>3), and
//      y[row r][token t] = C[r][t] + C[r+8][t+8]      (r, t < 8).
// Half of the MFMA output is discarded; at M <= 8 the MFMA pipe is far from
// busy and the loads are what matter.
//
// Reductions are in a fixed order, so results are bit-reproducible.  The
// grid barrier lives in file-scope device memory: calls of this kernel that
// overlap on one device (several streams) are not supported.
#include <cstdlib>
#include <cstring>

#include "mxfp4_common.hpp"
#include "mxfp4_launch.hpp"

namespace tinyinfer {

namespace {

constexpr int kNL = 8;               // weight loads (8 rows x 128 B) per unit
constexpr int kUnitK = 256 * kNL;    // K elements per unit
constexpr int kMaxTok = 8;
constexpr int kMaxXChunks = 8;       // 16-byte x/h staging chunks per thread
constexpr int kMaxSChunks = 6;       // 16-byte scale staging chunks per thread

// Self-resetting grid barrier state (zero at module load).
struct GridBarrier {
  unsigned int count;
  unsigned int generation;
  unsigned int timeouts;
};
__device__ GridBarrier g_decode_barrier;

// Per-launch geometry, computed on the host.
struct DecodeArgs {
  const uint16_t* x;       // [M, H]
  const uint8_t* wg;       // gate [I, H/2]
  const uint8_t* sg;       // [I, H/32]
  const uint8_t* wu;       // up
  const uint8_t* su;
  const uint8_t* wd;       // down [H, I/2]
  const uint8_t* sd;       // [H, I/32]
  uint16_t* h;             // tmp [M, I]
  uint16_t* out;           // [M, H]
  int M, H, I;
  int rgA, rgB;            // row groups of 8: I/8, H/8
  int ksA, ksB;            // K units per row group: ceil(H/kUnitK), ceil(I/kUnitK)
  int unitsA, unitsB;      // max units per workgroup in each phase
  int nA, nB;              // max row groups per workgroup
  int xs_stride;           // bytes per staged token row (max(H, I) * 2 + 16)
  int lds_x, lds_sa, lds_sb, lds_red;   // LDS byte offsets
  unsigned int spin_limit;
};

// Row groups [lo, hi) of `total` owned by workgroup g of G.
__device__ __forceinline__ void split_range(int total, int g, int G, int& lo, int& hi) {
  lo = (int)((int64_t)total * g / G);
  hi = (int)((int64_t)total * (g + 1) / G);
}

__device__ void grid_barrier(unsigned int nwg, unsigned int spin_limit) {
  // Each wave waits for its own global stores (h) to reach L2 -- a plain
  // counter wait; the cache maintenance is then done once per workgroup.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    // write this XCD's dirty L2 lines back so other XCDs see h
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const unsigned int gen = __hip_atomic_load(&g_decode_barrier.generation, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
    const unsigned int arrived = __hip_atomic_fetch_add(&g_decode_barrier.count, 1u, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT);
    if (arrived == nwg - 1) {
      __hip_atomic_store(&g_decode_barrier.count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&g_decode_barrier.generation, gen + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      unsigned int spins = 0;
      while (__hip_atomic_load(&g_decode_barrier.generation, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             gen) {
        __builtin_amdgcn_s_sleep(1);
        if (++spins >= spin_limit) {   // never expected: every workgroup is resident
          __hip_atomic_fetch_add(&g_decode_barrier.timeouts, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
      }
    }
    // drop this CU's / XCD's stale copies of other workgroups' h
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
}

// A unit of one wave: 8 rows of one matrix x [k_lo, k_lo + kUnitK) of K.
struct Unit {
  const uint8_t* w;       // matrix base
  int K;                  // matrix K (row length in elements)
  int row;                // first global row of the group
  int k_lo;
  int slot;               // partial-result slot
  int srow_lds;           // LDS offset of this group's first scale row
  bool valid;             // false: past the end of the wave's list (loads hit one line, no compute)
};

// Per-wave unit counts.  Wave w owns A units w, w+NWV, ... of the
// workgroup's uA, then the B units continuing the same round robin over the
// concatenated A+B list (so every wave gets nearly the same total).
struct WaveWork {
  int uA, uB, nAw, firstB, nBw;
};

template <int NWV>
__device__ __forceinline__ WaveWork wave_work(const DecodeArgs& a, int wave, int nA_wg, int nB_wg) {
  WaveWork w;
  w.uA = nA_wg * 2 * a.ksA;
  w.uB = nB_wg * a.ksB;
  w.nAw = (w.uA > wave) ? (w.uA - wave + NWV - 1) / NWV : 0;
  w.firstB = ((wave - w.uA) % NWV + NWV) % NWV;   // smallest b with (uA + b) % NWV == wave
  w.nBw = (w.uB > w.firstB) ? (w.uB - w.firstB + NWV - 1) / NWV : 0;
  return w;
}

// The k-th unit of a wave's padded sequence: A units at [0, padA) with
// padA = nAw rounded up to even, then B units; positions past either list
// are invalid placeholders.  Even-length phases keep both pipeline loops
// free of data-dependent branches.
template <int NWV>
__device__ __forceinline__ Unit unit_at(const DecodeArgs& a, const WaveWork& ww, int k, int wave, int rgA0,
                                        int rgB0) {
  Unit u;
  const int padA = (ww.nAw + 1) & ~1;
  const bool isA = k < padA;
  const int j = isA ? k : k - padA;
  u.valid = isA ? (k < ww.nAw) : (j < ww.nBw);
  if (!u.valid) {
    u.w = a.wd;
    u.K = a.I;
    u.row = 0;
    u.k_lo = 0;
    u.slot = 0;
    u.srow_lds = a.lds_sb;
    return u;
  }
  if (isA) {
    const int idx = wave + NWV * k;
    const int s = idx % a.ksA;
    const int lm = idx / a.ksA;          // lrg * 2 + mat
    const int mat = lm & 1, lrg = lm >> 1;
    u.w = mat ? a.wu : a.wg;
    u.K = a.H;
    u.row = (rgA0 + lrg) * 8;
    u.k_lo = s * kUnitK;
    u.slot = idx;
    u.srow_lds = a.lds_sa + (mat * a.nA + lrg) * 8 * (a.H / 32);
    return u;
  }
  const int idx = ww.firstB + NWV * j;
  const int s = idx % a.ksB;
  const int lrg = idx / a.ksB;
  u.w = a.wd;
  u.K = a.I;
  u.row = (rgB0 + lrg) * 8;
  u.k_lo = s * kUnitK;
  u.slot = a.unitsA + idx;
  u.srow_lds = a.lds_sb + lrg * 8 * (a.I / 32);
  return u;
}

// Issue a unit's kNL weight loads.  Always exactly kNL loads with no branch
// around them: the compiler then waits for precisely the loads each MFMA
// needs (a conditional issue makes it wait for everything in flight).
// Addresses past the end of K re-read the row's last block (zeroed at use);
// an invalid unit's loads all hit the matrix's first 16 bytes.
__device__ __forceinline__ void issue_unit(const Unit& u, u32x4_t (&wv)[kNL]) {
  const int lane = threadIdx.x & 63;
  const int r8 = lane & 7, q8 = lane >> 3;
  const int64_t half = u.K / 2;
  const uint8_t* rowp = u.w + (int64_t)(u.row + r8) * half;
#pragma unroll
  for (int j = 0; j < kNL; ++j) {
    int64_t kk = (int64_t)u.k_lo + 256 * j + 32 * q8;
    if (kk >= u.K) kk = u.K - 32;
    const uint8_t* p = u.valid ? rowp + kk / 2 : u.w;
    wv[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  }
}

// Multiply one unit (FAST: all its scale bytes convert exactly in hardware;
// chosen once per unit outside this body so every conversion sits in the
// same basic block as its MFMA).
template <int DT, bool FAST>
__device__ __forceinline__ f32x4_t unit_mfma(const Unit& u, const u32x4_t (&wv)[kNL],
                                             const uint32_t (&sb)[kNL], const uint8_t* xrow) {
  const int lane = threadIdx.x & 63;
  const int q8 = lane >> 3;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < kNL; ++j) {
    const int kk = u.k_lo + 256 * j + 32 * q8;
    if (u.k_lo + 256 * j >= u.K) break;              // wave-uniform: whole chunk past the end
    const bool in = kk < u.K;
    const int kx = in ? kk : u.K - 32;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      u32x4_t wa = FAST ? dq8_bf16_fast(wv[j][t], sb[j]) : dq8_bf16_exact(wv[j][t], sb[j]);
      if (!in) wa = u32x4_t{0u, 0u, 0u, 0u};
      const u32x4_t xb = *reinterpret_cast<const u32x4_t*>(xrow + 2 * (kx + 8 * t));
      if constexpr (DT == kBF16) {
        acc = mfma16x16x32(wa, xb, acc);
      } else {
        u32x4_t hi, lo;
        f16x8_split_bf16(xb, hi, lo);
        acc = mfma16x16x32(wa, hi, acc);
        acc = mfma16x16x32(wa, lo, acc);
      }
    }
  }
  return acc;
}

// Multiply one unit and store its partial (8 rows x 8 tokens fp32) to LDS.
template <int DT>
__device__ __forceinline__ void compute_unit(const DecodeArgs& a, const Unit& u, const u32x4_t (&wv)[kNL],
                                             uint8_t* lds) {
  if (!u.valid) return;
  const int lane = threadIdx.x & 63;
  const int r8 = lane & 7, q8 = lane >> 3;
  const int c = lane & 15;
  const int tok = (c & 7) < a.M ? (c & 7) : a.M - 1;     // columns >= M are discarded
  const int srs = u.K / 32;
  const uint8_t* srow = lds + u.srow_lds + r8 * srs;
  const uint8_t* xrow = lds + a.lds_x + tok * a.xs_stride;
  uint32_t sb[kNL];
  bool ok = true;
#pragma unroll
  for (int j = 0; j < kNL; ++j) {
    const int kk = u.k_lo + 256 * j + 32 * q8;
    const bool in = kk < u.K;
    sb[j] = in ? (uint32_t)srow[(kk < u.K ? kk : u.K - 32) / 32] : 127u;
    ok = ok && e8m0_fast_ok(sb[j]);
  }
  const f32x4_t acc = wave_all(ok) ? unit_mfma<DT, true>(u, wv, sb, xrow) : unit_mfma<DT, false>(u, wv, sb, xrow);
  // y[r][t] = C[r][t] + C[r+8][t+8]: lane l (t = l%16 < 8, g = l/16 < 2) holds
  // rows 4g..4g+3 of column t; lane l + 40 holds the matching rows 8 + 4g.. of
  // column t + 8.
  f32x4_t part;
#pragma unroll
  for (int v = 0; v < 4; ++v) part[v] = acc[v] + __shfl_down(acc[v], 40, 64);
  const int g = lane >> 4;
  if (c < 8 && g < 2 && c < a.M) {
    float* red = reinterpret_cast<float*>(lds + a.lds_red) + u.slot * 64;
    *reinterpret_cast<f32x4_t*>(red + c * 8 + 4 * g) = part;
  }
}

// Stage tokens [0, M) x [0, len) of a row-major [M, ld] activation matrix
// into LDS rows of `stride` bytes: issue (registers) and commit (LDS) halves,
// so the loads can be issued ahead of the weight stream.
template <int NT>
struct ActStager {
  u32x4_t r[kMaxXChunks];
  __device__ __forceinline__ void issue(const uint16_t* src, int M, int len, int ld) {
    const int per_row = len / 8;
#pragma unroll
    for (int i = 0; i < kMaxXChunks; ++i) {
      const int cidx = threadIdx.x + i * NT;
      r[i] = u32x4_t{0u, 0u, 0u, 0u};
      if (cidx < M * per_row) {
        const int t = cidx / per_row, k8 = cidx - t * per_row;
        r[i] = *reinterpret_cast<const u32x4_t*>(src + (int64_t)t * ld + 8 * k8);
      }
    }
  }
  __device__ __forceinline__ void commit(uint8_t* dst, int M, int len, int stride) {
    const int per_row = len / 8;
#pragma unroll
    for (int i = 0; i < kMaxXChunks; ++i) {
      const int cidx = threadIdx.x + i * NT;
      if (cidx < M * per_row) {
        const int t = cidx / per_row, k8 = cidx - t * per_row;
        *reinterpret_cast<u32x4_t*>(dst + t * stride + 16 * k8) = r[i];
      }
    }
  }
};

template <int DT, int NWV>
__global__ __launch_bounds__(NWV * 64, 1) void decode_kernel(DecodeArgs a) {
  constexpr int NT = NWV * 64;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int G = gridDim.x;
  const int g = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int rgA0, rgA1, rgB0, rgB1;
  split_range(a.rgA, g, G, rgA0, rgA1);
  split_range(a.rgB, g, G, rgB0, rgB1);
  const int nA_wg = rgA1 - rgA0, nB_wg = rgB1 - rgB0;

  // ---- prologue: x and scales first, then the first two units' weights ----
  ActStager<NT> xst;
  xst.issue(a.x, a.M, a.H, a.H);
  // scale spans: gate rows, up rows (nA_wg*8 rows of H/32 bytes each) and
  // down rows (nB_wg*8 rows of I/32 bytes) are contiguous in global memory.
  const int spanA = nA_wg * 8 * (a.H / 32), spanB = nB_wg * 8 * (a.I / 32);
  const uint8_t* srcs[3] = {a.sg + (int64_t)rgA0 * 8 * (a.H / 32), a.su + (int64_t)rgA0 * 8 * (a.H / 32),
                            a.sd + (int64_t)rgB0 * 8 * (a.I / 32)};
  const int dsts[3] = {a.lds_sa, a.lds_sa + a.nA * 8 * (a.H / 32), a.lds_sb};
  const int lens[3] = {spanA, spanA, spanB};
  const int c16[3] = {spanA / 16, spanA / 16, spanB / 16};   // spans are multiples of 16 (host-checked)
  u32x4_t sreg[kMaxSChunks];
#pragma unroll
  for (int i = 0; i < kMaxSChunks; ++i) {
    int cidx = threadIdx.x + i * NT;
    sreg[i] = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int s = 0; s < 3; ++s) {
      if (cidx >= 0 && cidx < c16[s]) sreg[i] = *reinterpret_cast<const u32x4_t*>(srcs[s] + 16 * cidx);
      cidx -= c16[s];
    }
  }
  (void)lens;
  const WaveWork ww = wave_work<NWV>(a, wave, nA_wg, nB_wg);
  const int padA = (ww.nAw + 1) & ~1;
  const int endB = padA + ((ww.nBw + 1) & ~1);
  u32x4_t bufA[kNL], bufB[kNL];
  Unit ua = unit_at<NWV>(a, ww, 0, wave, rgA0, rgB0);
  Unit ub = unit_at<NWV>(a, ww, 1, wave, rgA0, rgB0);
  issue_unit(ua, bufA);
  issue_unit(ub, bufB);
  xst.commit(lds + a.lds_x, a.M, a.H, a.xs_stride);
#pragma unroll
  for (int i = 0; i < kMaxSChunks; ++i) {
    int cidx = threadIdx.x + i * NT;
#pragma unroll
    for (int s = 0; s < 3; ++s) {
      if (cidx >= 0 && cidx < c16[s]) *reinterpret_cast<u32x4_t*>(lds + dsts[s] + 16 * cidx) = sreg[i];
      cidx -= c16[s];
    }
  }
  __syncthreads();

  // ---- phase A: depth-2 pipeline; its last iteration prefetches the first B units ----
  for (int k = 0; k < padA; k += 2) {
    compute_unit<DT>(a, ua, bufA, lds);
    ua = unit_at<NWV>(a, ww, k + 2, wave, rgA0, rgB0);
    issue_unit(ua, bufA);
    compute_unit<DT>(a, ub, bufB, lds);
    ub = unit_at<NWV>(a, ww, k + 3, wave, rgA0, rgB0);
    issue_unit(ub, bufB);
  }

  // ---- boundary: h = SiLU(g) * u, grid barrier, stage h ----
  __syncthreads();
  {
    const float* red = reinterpret_cast<const float*>(lds + a.lds_red);
    const int n = nA_wg * 8 * a.M;
    for (int e = threadIdx.x; e < n; e += NT) {
      const int lrg = e / (8 * a.M);
      const int rem = e - lrg * 8 * a.M;
      const int t = rem / 8, r = rem - t * 8;
      float gs = 0.f, us = 0.f;
      for (int s = 0; s < a.ksA; ++s) {
        gs += red[((lrg * 2 + 0) * a.ksA + s) * 64 + t * 8 + r];
        us += red[((lrg * 2 + 1) * a.ksA + s) * 64 + t * 8 + r];
      }
      a.h[(int64_t)t * a.I + (rgA0 + lrg) * 8 + r] = f32_to_act<DT>(silu_f32(gs) * us);
    }
  }
  grid_barrier((unsigned)G, a.spin_limit);
  {
    ActStager<NT> hst;
    hst.issue(a.h, a.M, a.I, a.I);
    hst.commit(lds + a.lds_x, a.M, a.I, a.xs_stride);
  }
  __syncthreads();

  // ---- phase B ----
  for (int k = padA; k < endB; k += 2) {
    compute_unit<DT>(a, ua, bufA, lds);
    ua = unit_at<NWV>(a, ww, k + 2, wave, rgA0, rgB0);
    issue_unit(ua, bufA);
    compute_unit<DT>(a, ub, bufB, lds);
    ub = unit_at<NWV>(a, ww, k + 3, wave, rgA0, rgB0);
    issue_unit(ub, bufB);
  }
  __syncthreads();
  {
    const float* red = reinterpret_cast<const float*>(lds + a.lds_red) + a.unitsA * 64;
    const int n = nB_wg * 8 * a.M;
    for (int e = threadIdx.x; e < n; e += NT) {
      const int lrg = e / (8 * a.M);
      const int rem = e - lrg * 8 * a.M;
      const int t = rem / 8, r = rem - t * 8;
      float ys = 0.f;
      for (int s = 0; s < a.ksB; ++s) ys += red[(lrg * a.ksB + s) * 64 + t * 8 + r];
      a.out[(int64_t)t * a.H + (rgB0 + lrg) * 8 + r] = f32_to_act<DT>(ys);
    }
  }
}

constexpr int kNWV = 12;

struct DevInfo {
  int cus = 0;
  int64_t max_lds = 0;     // dynamic LDS one workgroup may allocate
};

DevInfo dev_info(int dev) {
  static DevInfo cache[64];
  static bool init[64] = {};
  if (dev < 0 || dev >= 64) return DevInfo{};
  if (!init[dev]) {
    hipDeviceProp_t prop;
    DevInfo d;
    if (hipGetDeviceProperties(&prop, dev) == hipSuccess) {
      d.cus = prop.multiProcessorCount;
      d.max_lds = (int64_t)prop.sharedMemPerBlock;
    }
    cache[dev] = d;
    init[dev] = true;
  }
  return cache[dev];
}

bool forced_off() {
  static const bool v = [] {
    const char* e = std::getenv("TINYINFER_DECODE_FUSED");
    return e && std::strcmp(e, "0") == 0;
  }();
  return v;
}

// Geometry for one launch; false when the fused kernel does not apply.
bool plan(const MlpArgs& m, int cus, int64_t max_lds, DecodeArgs& a, int& grid, size_t& lds) {
  if (m.n < 1 || m.n > kMaxTok) return false;
  const int64_t H = m.hidden, I = m.inter;
  if (H % 256 != 0 || I % 256 != 0) return false;           // whole 256-wide K chunks
  if ((H / 32) % 2 != 0 || (I / 32) % 2 != 0) return false; // 16-byte scale spans
  if (H > (1 << 20) || I > (1 << 20)) return false;
  const int rgA = (int)(I / 8), rgB = (int)(H / 8);
  grid = cus < rgB ? cus : rgB;
  if (grid < 1) return false;
  const int nA = (rgA + grid - 1) / grid, nB = (rgB + grid - 1) / grid;
  const int ksA = (int)((H + kUnitK - 1) / kUnitK), ksB = (int)((I + kUnitK - 1) / kUnitK);
  const int unitsA = nA * 2 * ksA, unitsB = nB * ksB;
  const int64_t xs_stride = 2 * (H > I ? H : I) + 16;
  const int64_t lds_x = 0;
  const int64_t lds_sa = lds_x + m.n * xs_stride;
  const int64_t lds_sb = lds_sa + 2 * (int64_t)nA * 8 * (H / 32);
  const int64_t lds_red = (lds_sb + (int64_t)nB * 8 * (I / 32) + 15) & ~int64_t(15);
  const int64_t total = lds_red + (int64_t)(unitsA + unitsB) * 64 * 4;
  if (total > max_lds) return false;
  // staging loop bounds
  if ((int64_t)m.n * (H > I ? H : I) / 8 > (int64_t)kMaxXChunks * kNWV * 64) return false;
  const int64_t s16 = (2 * (int64_t)nA * 8 * (H / 32) + (int64_t)nB * 8 * (I / 32)) / 16;
  if (s16 > (int64_t)kMaxSChunks * kNWV * 64) return false;
  a.M = (int)m.n;
  a.H = (int)H;
  a.I = (int)I;
  a.rgA = rgA;
  a.rgB = rgB;
  a.ksA = ksA;
  a.ksB = ksB;
  a.unitsA = unitsA;
  a.unitsB = unitsB;
  a.nA = nA;
  a.nB = nB;
  a.xs_stride = (int)xs_stride;
  a.lds_x = (int)lds_x;
  a.lds_sa = (int)lds_sa;
  a.lds_sb = (int)lds_sb;
  a.lds_red = (int)lds_red;
  a.spin_limit = 1u << 22;     // ~ seconds of s_sleep polling: a safety net, never reached normally
  lds = (size_t)total;
  return true;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int DT>
hipError_t run(const MlpArgs& m, hipStream_t st, const DevInfo& d) {
  DecodeArgs a;
  int grid = 0;
  size_t lds = 0;
  if (!plan(m, d.cus, d.max_lds, a, grid, lds)) return hipErrorNotSupported;
  const void* ptrs[] = {m.x, m.gate, m.gate_scale, m.up, m.up_scale, m.down, m.down_scale, m.tmp};
  for (const void* p : ptrs)
    if (!aligned16(p)) return hipErrorNotSupported;
  a.x = static_cast<const uint16_t*>(m.x);
  a.wg = m.gate;
  a.sg = m.gate_scale;
  a.wu = m.up;
  a.su = m.up_scale;
  a.wd = m.down;
  a.sd = m.down_scale;
  a.h = static_cast<uint16_t*>(m.tmp);
  a.out = static_cast<uint16_t*>(m.out);
  // every workgroup must be resident at once for the grid barrier
  auto kern = decode_kernel<DT, kNWV>;
  if (lds > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds) != hipSuccess) {
    (void)hipGetLastError();
    return hipErrorNotSupported;
  }
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kNWV * 64, lds) != hipSuccess || per_cu < 1) {
    (void)hipGetLastError();
    return hipErrorNotSupported;
  }
  if ((int64_t)per_cu * d.cus < grid) return hipErrorNotSupported;
  kern<<<grid, kNWV * 64, lds, st>>>(a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_decode_mlp(const MlpArgs& m, hipStream_t stream) {
  if (forced_off()) return hipErrorNotSupported;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return hipErrorNotSupported;
  const DevInfo d = dev_info(dev);
  if (d.cus < 1) return hipErrorNotSupported;
  return m.dtype == kBF16 ? run<kBF16>(m, stream, d) : run<kF16>(m, stream, d);
}

unsigned int decode_barrier_timeouts() {
  GridBarrier host{};
  void* p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_decode_barrier)) != hipSuccess || !p) return 0xffffffffu;
  if (hipMemcpy(&host, p, sizeof(host), hipMemcpyDeviceToHost) != hipSuccess) return 0xffffffffu;
  return host.timeouts;
}

}  // namespace tinyinfer
