// Streaming MXFP4 GEMV for decode (M <= 8 tokens): one kernel per MLP stage.
//
// Replaces, for small token counts, the reference's per-token GEMV kernels
// mlp_stage1_mxfp4 / mlp_stage2_mxfp4 (tinyinfer/csrc/mlp_fp4.cu:79-142,
// 365-426): gate_up with the SiLU*up epilogue writes h, down writes out.
//
// Memory order is what decides HBM efficiency at this size, so the work is
// laid out around the load stream:
//   * an item is 8 weight rows x 128 contiguous bytes (256 K elements): one
//     dwordx4 load per lane, 8 full cache lines per instruction;
//   * a row group is 8 rows x all of K (x both matrices for gate_up); the
//     waves of a workgroup share a row group's items, and workgroup g takes
//     row groups g, g+G, g+2G, ...: at any moment the whole chip reads one
//     contiguous band of each matrix;
//   * each wave keeps the next row group's items in flight (double buffer)
//     while it multiplies the current one; per row group one LDS reduction
//     over the waves, then the epilogue.
// x is staged in LDS once per workgroup (issued after the first row group's
// weight loads, so its latency overlaps them).
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
constexpr int kItemK = 256;       // K elements per item

struct StreamArgs {
  const uint16_t* x;      // [M, K] activations (x for gate_up, h for down)
  const uint8_t* w0;      // [R, K/2] gate (or down)
  const uint8_t* s0;      // [R, K/32]
  const uint8_t* w1;      // [R, K/2] up (gate_up only)
  const uint8_t* s1;
  uint16_t* out;          // [M, R]
  int M, K, R;
  int segs;               // K / kItemK
  int items;              // items per row group: mats * segs
  int ipw;                // items per wave per row group: ceil(items / kNW)
  int rgroups;            // R / 8
  int xs_stride;          // bytes per staged token row
};

// Issue one row group's items for this wave (IPWMAX loads + scale bytes,
// always the same number of instructions: past-the-end items read the
// matrix's first 16 bytes and are not multiplied).
template <int IPWMAX, bool GATEUP>
__device__ __forceinline__ void issue_rg(const StreamArgs& a, int rg, int wave, u32x4_t (&wv)[IPWMAX],
                                         uint32_t (&sb)[IPWMAX]) {
  const int lane = threadIdx.x & 63;
  const int r8 = lane & 7, q8 = lane >> 3;
  const bool rg_ok = rg < a.rgroups;
  const int64_t row = (int64_t)(rg_ok ? rg : 0) * 8 + r8;
#pragma unroll
  for (int k = 0; k < IPWMAX; ++k) {
    const int item = wave + kNW * k;
    const bool ok = rg_ok && k < a.ipw && item < a.items;
    const int mat = GATEUP ? (item >= a.segs) : 0;
    const int seg = item - mat * a.segs;
    const uint8_t* w = mat ? a.w1 : a.w0;
    const uint8_t* s = mat ? a.s1 : a.s0;
    const uint8_t* wp = ok ? w + row * (a.K / 2) + seg * (kItemK / 2) + 16 * q8 : a.w0;
    const uint8_t* sp = ok ? s + row * (a.K / 32) + seg * (kItemK / 32) + q8 : a.s0;
    wv[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wp));
    sb[k] = *sp;
  }
}

// Multiply one row group's items; partial sums per matrix into acc[mat].
// FAST: every scale byte of the items is in the range where the hardware
// conversion is exact.  The choice is made once per row group outside this
// body, so each conversion sits in the same basic block as the MFMA that
// consumes it.
template <int DT, int IPWMAX, bool GATEUP, bool FAST>
__device__ __forceinline__ void compute_body(const StreamArgs& a, int wave, const u32x4_t (&wv)[IPWMAX],
                                             const uint32_t (&sb)[IPWMAX], const uint8_t* xrow,
                                             f32x4_t (&acc)[2]) {
  const int lane = threadIdx.x & 63;
  const int q8 = lane >> 3;
#pragma unroll
  for (int k = 0; k < IPWMAX; ++k) {
    const int item = wave + kNW * k;
    if (k >= a.ipw || item >= a.items) break;            // wave-uniform
    const int mat = GATEUP ? (item >= a.segs) : 0;
    const int seg = item - mat * a.segs;
    const int kx = seg * kItemK + 32 * q8;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const u32x4_t wa = FAST ? dq8_bf16_fast(wv[k][t], sb[k]) : dq8_bf16_exact(wv[k][t], sb[k]);
      const u32x4_t xb = *reinterpret_cast<const u32x4_t*>(xrow + 2 * (kx + 8 * t));
      // uniform branch on the matrix (a runtime index into acc would spill it)
      if (GATEUP && mat) {
        if constexpr (DT == kBF16) {
          acc[1] = mfma16x16x32(wa, xb, acc[1]);
        } else {
          u32x4_t hi, lo;
          f16x8_split_bf16(xb, hi, lo);
          acc[1] = mfma16x16x32(wa, lo, mfma16x16x32(wa, hi, acc[1]));
        }
      } else {
        if constexpr (DT == kBF16) {
          acc[0] = mfma16x16x32(wa, xb, acc[0]);
        } else {
          u32x4_t hi, lo;
          f16x8_split_bf16(xb, hi, lo);
          acc[0] = mfma16x16x32(wa, lo, mfma16x16x32(wa, hi, acc[0]));
        }
      }
    }
  }
}

template <int DT, int IPWMAX, bool GATEUP>
__device__ __forceinline__ void compute_rg(const StreamArgs& a, int wave, const u32x4_t (&wv)[IPWMAX],
                                           const uint32_t (&sb)[IPWMAX], const uint8_t* xs,
                                           f32x4_t (&acc)[2]) {
  const int lane = threadIdx.x & 63;
  const int c = lane & 15;
  const int tok = (c & 7) < a.M ? (c & 7) : a.M - 1;     // columns >= M are discarded
  const uint8_t* xrow = xs + tok * a.xs_stride;
  acc[0] = acc[1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  bool ok = true;
#pragma unroll
  for (int k = 0; k < IPWMAX; ++k) ok = ok && (k >= a.ipw || e8m0_fast_ok(sb[k]));
  if (wave_all(ok)) compute_body<DT, IPWMAX, GATEUP, true>(a, wave, wv, sb, xrow, acc);
  else compute_body<DT, IPWMAX, GATEUP, false>(a, wave, wv, sb, xrow, acc);
}

// Fold C[r][t] + C[r+8][t+8] and store this wave's partial (rows 4g..4g+3,
// token t) for matrix `mat` into LDS.
__device__ __forceinline__ void store_partial(const f32x4_t& acc, float* red, int M) {
  const int lane = threadIdx.x & 63;
  f32x4_t part;
#pragma unroll
  for (int v = 0; v < 4; ++v) part[v] = acc[v] + __shfl_down(acc[v], 40, 64);
  const int c = lane & 15, g = lane >> 4;
  if (c < 8 && g < 2 && c < M) *reinterpret_cast<f32x4_t*>(red + c * 8 + 4 * g) = part;
}

template <int DT, int IPWMAX, bool GATEUP>
__global__ __launch_bounds__(kNW * 64, 2) void stream_kernel(StreamArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int kMats = GATEUP ? 2 : 1;
  // LDS: [x staging M rows][partials 2 parities x kNW waves x kMats x 64 floats]
  float* red = reinterpret_cast<float*>(lds + a.M * a.xs_stride);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = gridDim.x;
  const int g = blockIdx.x;

  u32x4_t wa[IPWMAX], wb[IPWMAX];
  uint32_t sa[IPWMAX], sb2[IPWMAX];
  issue_rg<IPWMAX, GATEUP>(a, g, wave, wa, sa);

  // stage x [M, K] (after the first weight loads: its latency overlaps them),
  // four 16-byte loads in flight per thread per round
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
  }
  __syncthreads();

  int parity = 0;
  auto finish_rg = [&](int rg, const f32x4_t (&acc)[2]) {
    float* slot = red + parity * (kNW * kMats * 64);
#pragma unroll
    for (int m = 0; m < kMats; ++m) store_partial(acc[m], slot + (wave * kMats + m) * 64, a.M);
    __syncthreads();
    // epilogue: 8 rows x M tokens, fixed-order sum over the waves
    const int n = 8 * a.M;
    for (int e = threadIdx.x; e < n; e += kNW * 64) {
      const int t = e >> 3, r = e & 7;
      float y0 = 0.f, y1 = 0.f;
      for (int w = 0; w < kNW; ++w) {
        y0 += slot[(w * kMats + 0) * 64 + t * 8 + r];
        if (GATEUP) y1 += slot[(w * kMats + 1) * 64 + t * 8 + r];
      }
      const float v = GATEUP ? silu_f32(y0) * y1 : y0;
      a.out[(int64_t)t * a.R + rg * 8 + r] = f32_to_act<DT>(v);
    }
    parity ^= 1;
  };

  for (int rg = g; rg < a.rgroups; rg += 2 * G) {
    f32x4_t acc[2];
    issue_rg<IPWMAX, GATEUP>(a, rg + G, wave, wb, sb2);
    compute_rg<DT, IPWMAX, GATEUP>(a, wave, wa, sa, lds, acc);
    finish_rg(rg, acc);
    if (rg + G >= a.rgroups) break;
    issue_rg<IPWMAX, GATEUP>(a, rg + 2 * G, wave, wa, sa);
    compute_rg<DT, IPWMAX, GATEUP>(a, wave, wb, sb2, lds, acc);
    finish_rg(rg + G, acc);
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

// One workgroup per row group up to what is resident at once (a second
// round of workgroups would restart the load stream).
template <int DT, bool GATEUP>
hipError_t launch(StreamArgs a, size_t lds, int cus, hipStream_t st) {
  auto go = [&](auto kern) -> hipError_t {
    if (lds > 64 * 1024 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess) {
      (void)hipGetLastError();
      return hipErrorNotSupported;
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kNW * 64, lds) != hipSuccess) {
      (void)hipGetLastError();
      per_cu = 1;
    }
    if (per_cu < 1) per_cu = 1;
    if (per_cu > 2) per_cu = 2;
    int grid = per_cu * cus;
    if (grid > a.rgroups) grid = a.rgroups;
    kern<<<grid, kNW * 64, lds, st>>>(a);
    return hipGetLastError();
  };
  if (a.ipw <= 2) return go(stream_kernel<DT, 2, GATEUP>);
  if (a.ipw <= 4) return go(stream_kernel<DT, 4, GATEUP>);
  if (a.ipw <= 6) return go(stream_kernel<DT, 6, GATEUP>);
  return go(stream_kernel<DT, 8, GATEUP>);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int DT, bool GATEUP>
hipError_t run_stage(const uint16_t* x, const uint8_t* w0, const uint8_t* s0, const uint8_t* w1,
                     const uint8_t* s1, int64_t M, int64_t K, int64_t R, uint16_t* out, hipStream_t st) {
  const DevCaps d = caps();
  if (d.cus < 1 || M < 1 || M > 8 || K % kItemK != 0 || R % 8 != 0) return hipErrorNotSupported;
  if (K > (1 << 20) || R > (1 << 24)) return hipErrorNotSupported;
  if (!aligned16(x) || !aligned16(w0) || (GATEUP && !aligned16(w1))) return hipErrorNotSupported;
  StreamArgs a;
  a.x = x;
  a.w0 = w0;
  a.s0 = s0;
  a.w1 = GATEUP ? w1 : w0;
  a.s1 = GATEUP ? s1 : s0;
  a.out = out;
  a.M = (int)M;
  a.K = (int)K;
  a.R = (int)R;
  a.segs = (int)(K / kItemK);
  a.items = (GATEUP ? 2 : 1) * a.segs;
  a.ipw = (a.items + kNW - 1) / kNW;
  if (a.ipw > 8) return hipErrorNotSupported;
  a.rgroups = (int)(R / 8);
  a.xs_stride = (int)(2 * K + 16);
  const int64_t lds = M * a.xs_stride + 2 * (int64_t)kNW * (GATEUP ? 2 : 1) * 64 * 4;
  if (lds > d.max_lds) return hipErrorNotSupported;
  return launch<DT, GATEUP>(a, (size_t)lds, d.cus, st);
}

}  // namespace

hipError_t launch_stream_mlp(const MlpArgs& a, int stage, hipStream_t st) {
  const uint16_t* x = static_cast<const uint16_t*>(a.x);
  uint16_t* h = static_cast<uint16_t*>(a.tmp);
  uint16_t* y = static_cast<uint16_t*>(a.out);
  // both stages must be supported before anything is launched
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

bool stream_supported(const MlpArgs& a, int stage) {
  const DevCaps d = caps();
  if (d.cus < 1 || a.n < 1 || a.n > 8) return false;
  auto fits = [&](int64_t K, int mats) {
    if (K % kItemK != 0) return false;
    const int64_t items = mats * (K / kItemK);
    if ((items + kNW - 1) / kNW > 8) return false;
    const int64_t lds = a.n * (2 * K + 16) + 2 * (int64_t)kNW * mats * 64 * 4;
    return lds <= d.max_lds;
  };
  if ((stage & kStageGateUp) && !fits(a.hidden, 2)) return false;
  if ((stage & kStageDown) && !fits(a.inter, 1)) return false;
  const void* ptrs[] = {a.x, a.gate, a.up, a.down, a.tmp};
  for (const void* p : ptrs)
    if (p && !aligned16(p)) return false;
  return true;
}

}  // namespace tinyinfer
