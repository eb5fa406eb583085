// Streaming MXFP4 GEMV for decode (M <= 8 tokens): one kernel per MLP stage.
//
// Replaces, for small token counts, the reference's per-token GEMV kernels
// mlp_stage1_mxfp4 / mlp_stage2_mxfp4 (tinyinfer/csrc/mlp_fp4.cu:79-142,
// 365-426): gate_up with the SiLU*up epilogue writes h, down writes out.
//
// Memory order is what decides HBM efficiency here, so the work is laid out
// around the load stream (each choice measured on MI355X with load-only
// probes of the same instruction shapes):
//   * an item is 8 weight rows x 128 contiguous bytes (256 K elements): one
//     dwordx4 load per lane, 8 full cache lines per instruction;
//   * a row group is 8 rows x all of K (x both matrices for gate_up).
//     Workgroup g takes row groups g, g+G, g+2G, ... and each of its waves a
//     contiguous run of the row group's K segments, so the whole chip reads
//     one contiguous band of each matrix at a time;
//   * one 8-wave workgroup per CU, each wave with its next row group's loads
//     in flight while it multiplies the current one (8 waves/CU streaming a
//     few loads each gave the highest bandwidth; more waves gave less);
//   * no workgroup barrier in the stream: a wave stores its partial sums in
//     an LDS slot of the row group and bumps an LDS counter; the last wave to
//     finish a row group sums the slots in a fixed order (bit-reproducible)
//     and runs the epilogue;
//   * a wave fetches the e8m0 scale bytes of its segments with one 8-byte load
//     per (row, segment) ahead of its weights and stages them in its own LDS
//     area (a scale-byte load per weight instruction costs ~20% bandwidth).
// x is staged in LDS once per workgroup, after the first row groups' loads.
//
// MFMA mapping ("8 rows x 128 B"): lane l holds weight row l&7, 32-element K
// block l>>3 of the item.  With these as the A operand of
// v_mfma_f32_16x16x32_bf16, MFMA row i is weight row i&7 over K blocks
// {2g + (i>>3)}; the B operand in lane l carries token (l%16)&7 at lane l's
// own K block, so y[row r][token t] = C[r][t] + C[r+8][t+8] (r, t < 8).
#include "mxfp4_common.hpp"
#include "mxfp4_launch.hpp"

namespace tinyinfer {

namespace {

constexpr int kNW = 8;            // waves per workgroup
constexpr int kItemK = 256;       // K elements per item (one 128-byte segment per row)
constexpr int kMaxSpw = 8;        // max segments per wave per matrix (more would spill)
constexpr int kSclPerWave = 2 * 8 * kMaxSpw * 8;   // wave-private scale bytes (mats x rows x segs x 8)

struct StreamArgs {
  const uint16_t* x;      // [M, K] activations (x for gate_up, h for down)
  const uint8_t* w0;      // [R, K/2] gate (or down)
  const uint8_t* s0;      // [R, K/32]
  const uint8_t* w1;      // [R, K/2] up (gate_up only)
  const uint8_t* s1;
  uint16_t* out;          // [M, R]
  int M, K, R;
  int segs;               // K / kItemK
  int rgroups;            // R / 8
  int nrg_max;            // max row groups per workgroup
  int xs_stride;          // bytes per staged token row
  int lds_scl, lds_red, lds_cnt;   // LDS byte offsets
};

// Wave w's segment run [lo, hi) of a row group (same for both matrices).
__device__ __forceinline__ void seg_run(const StreamArgs& a, int wave, int& lo, int& hi) {
  lo = a.segs * wave / kNW;
  hi = a.segs * (wave + 1) / kNW;
}

// A row group's loads for this wave: scale bytes (8-byte pieces, one per
// (matrix, row, segment), SPL per lane) first, then the weight items
// (matrix-major, then segment).  A fixed instruction count: unused slots read
// the matrices' first bytes and are not used.
template <int SPW, bool GATEUP, int SPL>
__device__ __forceinline__ void issue_rg(const StreamArgs& a, int rg, int wave,
                                         u32x4_t (&wv)[(GATEUP ? 2 : 1) * SPW], u32x2_t (&sc)[SPL]) {
  constexpr int kMats = GATEUP ? 2 : 1;
  const int lane = threadIdx.x & 63;
  const int r8 = lane & 7, q8 = lane >> 3;
  int lo, hi;
  seg_run(a, wave, lo, hi);
  const int n = hi - lo;
  const int nn = n > 0 ? n : 1;
  const bool rg_ok = rg < a.rgroups;
  const int64_t rgc = rg_ok ? rg : 0;
#pragma unroll
  for (int i = 0; i < SPL; ++i) {
    const int p = lane + 64 * i;                 // piece (mat, row, seg): p = (mat * 8 + row) * n + seg
    const bool ok = rg_ok && p < kMats * 8 * n;
    const int pc = ok ? p : 0;
    const int mr = pc / nn, sg = pc - mr * nn;
    const int mat = GATEUP ? mr / 8 : 0;
    const int row = mr - mat * 8;
    const uint8_t* s = mat ? a.s1 : a.s0;
    const uint8_t* sp = ok ? s + (rgc * 8 + row) * (a.K / 32) + (int64_t)(lo + sg) * 8 : a.s0;
    sc[i] = *reinterpret_cast<const u32x2_t*>(sp);
  }
  const int64_t row = rgc * 8 + r8;
#pragma unroll
  for (int k = 0; k < kMats * SPW; ++k) {
    const int mat = GATEUP ? k / SPW : 0;
    const int sg = k - mat * SPW;
    const bool ok = rg_ok && sg < n;
    const uint8_t* w = mat ? a.w1 : a.w0;
    const uint8_t* wp = ok ? w + row * (a.K / 2) + (int64_t)(lo + sg) * (kItemK / 2) + 16 * q8 : a.w0;
    wv[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wp));
  }
}

// Multiply this wave's items of one row group (FAST: every scale byte in the
// hardware-exact range; chosen once outside this body so each conversion
// sits in the same basic block as its MFMA).
template <int DT, int SPW, bool GATEUP, bool FAST>
__device__ __forceinline__ void mma_items(int n, int lo, const u32x4_t (&wv)[(GATEUP ? 2 : 1) * SPW],
                                          const uint32_t (&sb)[(GATEUP ? 2 : 1) * SPW], const uint8_t* xrow,
                                          f32x4_t (&acc)[2]) {
  constexpr int kMats = GATEUP ? 2 : 1;
  const int q8 = (threadIdx.x & 63) >> 3;
#pragma unroll
  for (int mat = 0; mat < kMats; ++mat) {
#pragma unroll
    for (int sg = 0; sg < SPW; ++sg) {
      if (sg >= n) break;                                   // wave-uniform
      const int k = mat * SPW + sg;
      const int kx = (lo + sg) * kItemK + 32 * q8;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const u32x4_t wa = FAST ? dq8_bf16_fast(wv[k][t], sb[k]) : dq8_bf16_exact(wv[k][t], sb[k]);
        const u32x4_t xb = *reinterpret_cast<const u32x4_t*>(xrow + 2 * (kx + 8 * t));
        if constexpr (DT == kBF16) {
          acc[mat] = mfma16x16x32(wa, xb, acc[mat]);
        } else {
          u32x4_t xh, xl;
          f16x8_split_bf16(xb, xh, xl);
          acc[mat] = mfma16x16x32(wa, xl, mfma16x16x32(wa, xh, acc[mat]));
        }
      }
    }
  }
}

template <int DT, int SPW, bool GATEUP, int SPL>
__device__ __forceinline__ void compute_rg(const StreamArgs& a, int wave,
                                           const u32x4_t (&wv)[(GATEUP ? 2 : 1) * SPW],
                                           const u32x2_t (&sc)[SPL], uint8_t* my_scl, const uint8_t* xs,
                                           f32x4_t (&acc)[2]) {
  constexpr int kMats = GATEUP ? 2 : 1;
  const int lane = threadIdx.x & 63;
  const int r8 = lane & 7, q8 = lane >> 3;
  int lo, hi;
  seg_run(a, wave, lo, hi);
  const int n = hi - lo;
  // stage this wave's scale pieces ([mat][row][seg] x 8 bytes) and read back
  // the byte of each of this lane's items
#pragma unroll
  for (int i = 0; i < SPL; ++i) {
    const int p = lane + 64 * i;
    if (p < kMats * 8 * n) *reinterpret_cast<u32x2_t*>(my_scl + 8 * p) = sc[i];
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");   // other lanes' bytes are read back
  uint32_t sb[kMats * SPW];
  bool ok = true;
#pragma unroll
  for (int k = 0; k < kMats * SPW; ++k) {
    const int mat = GATEUP ? k / SPW : 0;
    const int sg = k - mat * SPW;
    sb[k] = sg < n ? (uint32_t)my_scl[8 * ((mat * 8 + r8) * n + sg) + q8] : 127u;
    ok = ok && e8m0_fast_ok(sb[k]);
  }
  const int c = lane & 15;
  const int tok = (c & 7) < a.M ? (c & 7) : a.M - 1;     // columns >= M are discarded
  const uint8_t* xrow = xs + tok * a.xs_stride;
  acc[0] = acc[1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  if (wave_all(ok)) mma_items<DT, SPW, GATEUP, true>(n, lo, wv, sb, xrow, acc);
  else mma_items<DT, SPW, GATEUP, false>(n, lo, wv, sb, xrow, acc);
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

template <int DT, int SPW, bool GATEUP, int SPL>
__global__ __launch_bounds__(kNW * 64, 1) void stream_kernel(StreamArgs a) {
  constexpr int kMats = GATEUP ? 2 : 1;
  constexpr int kItems = kMats * SPW;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int G = gridDim.x;
  const int g = blockIdx.x;
  uint8_t* my_scl = lds + a.lds_scl + wave * kSclPerWave;
  float* red = reinterpret_cast<float*>(lds + a.lds_red);                   // [nrg_max][kNW][kMats][64]
  unsigned int* cnt = reinterpret_cast<unsigned int*>(lds + a.lds_cnt);    // [nrg_max]

  u32x4_t wa[kItems], wb[kItems];
  u32x2_t sca[SPL], scb[SPL];
  issue_rg<SPW, GATEUP, SPL>(a, g, wave, wa, sca);
  issue_rg<SPW, GATEUP, SPL>(a, g + G, wave, wb, scb);

  // stage x [M, K] and clear the row-group counters
  {
    constexpr int kB = 4;
    const int per_row = a.K / 8;
    const int n = a.M * per_row;
    for (int c0 = threadIdx.x; c0 < n; c0 += kB * kNW * 64) {
      u32x4_t v[kB];
#pragma unroll
      for (int b = 0; b < kB; ++b) {
        const int cidx = c0 + b * kNW * 64;
        const int cc = cidx < n ? cidx : n - 1;
        const int t = cc / per_row, k8 = cc - t * per_row;
        v[b] = *reinterpret_cast<const u32x4_t*>(a.x + (int64_t)t * a.K + 8 * k8);
      }
#pragma unroll
      for (int b = 0; b < kB; ++b) {
        const int cidx = c0 + b * kNW * 64;
        if (cidx < n) {
          const int t = cidx / per_row, k8 = cidx - t * per_row;
          *reinterpret_cast<u32x4_t*>(lds + t * a.xs_stride + 16 * k8) = v[b];
        }
      }
    }
    for (int i = threadIdx.x; i < a.nrg_max; i += kNW * 64) cnt[i] = 0u;
  }
  __syncthreads();

  // after a row group: partials into its slot, count, and the last wave of
  // the workgroup to get here runs the epilogue
  auto finish_rg = [&](int rg, int li, const f32x4_t (&acc)[2]) {
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
        a.out[(int64_t)t * a.R + rg * 8 + r] = f32_to_act<DT>(v);
      }
    }
  };

  int li = 0;
  for (int rg = g; rg < a.rgroups; rg += 2 * G, li += 2) {
    f32x4_t acc[2];
    compute_rg<DT, SPW, GATEUP, SPL>(a, wave, wa, sca, my_scl, lds, acc);
    issue_rg<SPW, GATEUP, SPL>(a, rg + 2 * G, wave, wa, sca);
    finish_rg(rg, li, acc);
    if (rg + G >= a.rgroups) break;
    compute_rg<DT, SPW, GATEUP, SPL>(a, wave, wb, scb, my_scl, lds, acc);
    issue_rg<SPW, GATEUP, SPL>(a, rg + 3 * G, wave, wb, scb);
    finish_rg(rg + G, li + 1, acc);
  }
}

struct DevCaps {
  int cus = 0;
  int64_t max_lds = 0;
};

DevCaps caps() {
  static DevCaps cache[64];
  static bool init[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return DevCaps{};
  if (!init[dev]) {
    hipDeviceProp_t prop;
    DevCaps d;
    if (hipGetDeviceProperties(&prop, dev) == hipSuccess) {
      d.cus = prop.multiProcessorCount;
      d.max_lds = (int64_t)prop.sharedMemPerBlock;
    }
    cache[dev] = d;
    init[dev] = true;
  }
  return cache[dev];
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Geometry of one stage; false when the streaming kernel does not apply.
bool plan(int64_t M, int64_t K, int64_t R, bool gateup, const DevCaps& d, StreamArgs& a, int& grid,
          int64_t& lds) {
  if (d.cus < 1 || M < 1 || M > 8 || K % kItemK != 0 || R % 8 != 0) return false;
  if (K > (1 << 20) || R > (1 << 24)) return false;
  const int mats = gateup ? 2 : 1;
  a.M = (int)M;
  a.K = (int)K;
  a.R = (int)R;
  a.segs = (int)(K / kItemK);
  const int spw = (a.segs + kNW - 1) / kNW;
  if (spw > (gateup ? kMaxSpw / 2 : kMaxSpw)) return false;   // double-buffered items fit in VGPRs
  if (mats * 8 * spw > 64) return false;             // scale pieces: one per lane
  a.rgroups = (int)(R / 8);
  grid = d.cus < a.rgroups ? d.cus : a.rgroups;
  a.nrg_max = (a.rgroups + grid - 1) / grid;
  a.xs_stride = (int)(2 * K + 16);
  a.lds_scl = (int)(M * a.xs_stride);
  a.lds_red = a.lds_scl + kNW * kSclPerWave;
  a.lds_cnt = a.lds_red + a.nrg_max * kNW * mats * 64 * 4;
  lds = a.lds_cnt + 4 * ((a.nrg_max + 3) & ~3);
  return lds <= d.max_lds;
}

template <int DT, bool GATEUP>
hipError_t launch(const StreamArgs& a, int64_t lds, int grid, hipStream_t st) {
  const int spw = (a.segs + kNW - 1) / kNW;
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
  if (spw <= 2) return go(stream_kernel<DT, 2, GATEUP, 1>);
  if (GATEUP || spw <= 4) return go(stream_kernel<DT, 4, GATEUP, 1>);
  return go(stream_kernel<DT, 8, false, 1>);
}

template <int DT, bool GATEUP>
hipError_t run_stage(const uint16_t* x, const uint8_t* w0, const uint8_t* s0, const uint8_t* w1,
                     const uint8_t* s1, int64_t M, int64_t K, int64_t R, uint16_t* out, hipStream_t st) {
  StreamArgs a;
  int grid = 0;
  int64_t lds = 0;
  if (!plan(M, K, R, GATEUP, caps(), a, grid, lds)) return hipErrorNotSupported;
  a.x = x;
  a.w0 = w0;
  a.s0 = s0;
  a.w1 = GATEUP ? w1 : w0;
  a.s1 = GATEUP ? s1 : s0;
  a.out = out;
  return launch<DT, GATEUP>(a, lds, grid, st);
}

}  // namespace

bool stream_supported(const MlpArgs& a, int stage) {
  const DevCaps d = caps();
  StreamArgs sa;
  int grid = 0;
  int64_t lds = 0;
  if ((stage & kStageGateUp) && !plan(a.n, a.hidden, a.inter, true, d, sa, grid, lds)) return false;
  if ((stage & kStageDown) && !plan(a.n, a.inter, a.hidden, false, d, sa, grid, lds)) return false;
  // 16-byte loads of activations and weights, 8-byte loads of scale bytes
  const void* p16[] = {a.x, a.gate, a.up, a.down, a.tmp};
  for (const void* p : p16)
    if (p && !aligned16(p)) return false;
  const void* p8[] = {a.gate_scale, a.up_scale, a.down_scale};
  for (const void* p : p8)
    if (p && (reinterpret_cast<uintptr_t>(p) & 7u)) return false;
  return true;
}

hipError_t launch_stream_mlp(const MlpArgs& a, int stage, hipStream_t st) {
  const uint16_t* x = static_cast<const uint16_t*>(a.x);
  uint16_t* h = static_cast<uint16_t*>(a.tmp);
  uint16_t* y = static_cast<uint16_t*>(a.out);
  const bool bf = a.dtype == kBF16;
  if (stage & kStageGateUp) {
    const hipError_t e = bf ? run_stage<kBF16, true>(x, a.gate, a.gate_scale, a.up, a.up_scale, a.n, a.hidden,
                                                     a.inter, h, st)
                            : run_stage<kF16, true>(x, a.gate, a.gate_scale, a.up, a.up_scale, a.n, a.hidden,
                                                    a.inter, h, st);
    if (e != hipSuccess) return e;
  }
  if (stage & kStageDown) {
    return bf ? run_stage<kBF16, false>(h, a.down, a.down_scale, nullptr, nullptr, a.n, a.inter, a.hidden, y, st)
              : run_stage<kF16, false>(h, a.down, a.down_scale, nullptr, nullptr, a.n, a.inter, a.hidden, y, st);
  }
  return hipSuccess;
}

}  // namespace tinyinfer
