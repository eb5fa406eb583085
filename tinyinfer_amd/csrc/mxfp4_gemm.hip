// Tiled MXFP4 MLP path for prefill / mixed batches (M >= 128 tokens).
//
// Replaces the reference's per-token GEMV kernels mlp_stage1_mxfp4 /
// mlp_stage2_mxfp4 (tinyinfer/csrc/mlp_fp4.cu:79-142, 365-426) in the regime
// where they are compute-bound: each workgroup computes a BN x BM tile of
// C = W X^T (weight rows x tokens) with v_mfma_f32_32x32x16_bf16, fp32
// accumulation, the MXFP4 weights dequantized to bf16 in registers.
//
// Per K step (BK = 64 = two e8m0 blocks) a workgroup stages into LDS:
//   * X  [BM tokens][64] bf16, row stride 144 B (16 B pad: the 32 rows one
//     ds_read_b128 touches start on distinct bank groups);
//   * W  [NMAT*BN rows][32 packed bytes + 2 scale bytes], row stride 48 B.
// Operands use a K permutation shared by A and B: in MFMA k-step s (0..3),
// lane half j (lane / 32) supplies the 8 K elements 32j + 8s .. 32j + 8s + 7
// of the BK slice.  A lane's W bytes for the whole BK slice are then one
// 16-byte run (one scale byte), and its X bytes one 64-byte run.
//
// gate_up (NMAT = 2): the gate and up tiles of the same rows sit in the same
// lanes, so the epilogue computes SiLU(g) * u in registers and stores h.
// down (NMAT = 1): plain rounding to the activation dtype.
//
// Double-buffered: the global loads of step k+1 are issued before the MFMAs
// of step k and written to the other LDS buffer after them; one barrier per
// step.  Tiles are ordered so each XCD (workgroup id mod 8) walks a compact
// band of weight rows and all token tiles of it.
#include "mxfp4_common.hpp"
#include "mxfp4_launch.hpp"

namespace tinyinfer {

namespace {

constexpr int kBK = 64;                  // K per step
constexpr int kThreads = 256;            // 4 waves
constexpr int kXStride = 2 * kBK + 16;   // bytes per staged X row
constexpr int kWStride = 48;             // bytes per staged W row (32 packed + 2 scales + pad)

template <int DT, int NMAT, int BN, int BM>
struct GemmCfg {
  static constexpr int kRowsPerWave = BN / 2;          // weight rows per wave (per matrix)
  static constexpr int kToksPerWave = BM / 2;          // tokens per wave
  static constexpr int TR = kRowsPerWave / 32;         // 32-row MFMA blocks per wave
  static constexpr int TT = kToksPerWave / 32;         // 32-token MFMA blocks per wave
  static constexpr int kXBytes = BM * kXStride;
  static constexpr int kWBytes = NMAT * BN * kWStride;
  static constexpr int kStageBytes = kXBytes + kWBytes;
  // global -> LDS staging work per thread
  static constexpr int kXChunks = BM * (2 * kBK / 16) / kThreads;   // 16-B X chunks
  static constexpr int kWChunks = NMAT * BN * 2 / kThreads;         // 16-B W chunks
  static constexpr int kSRows = NMAT * BN;                          // scale rows (2 bytes each)
  static_assert(kXChunks * kThreads == BM * (2 * kBK / 16), "X staging must divide evenly");
  static_assert(kWChunks * kThreads == NMAT * BN * 2, "W staging must divide evenly");
  static_assert(TR >= 1 && TT >= 1, "tile too small");
};

struct GemmPtrs {
  const uint16_t* x;       // [M, K]
  const uint8_t* w[2];     // [N, K/2]
  const uint8_t* s[2];     // [N, K/32]
  uint16_t* out;           // [M, N]
  int64_t M, N, K;
  const uint16_t* res;     // down only: residual [M, N] added to out, or null
};

// fp16 operand -> exact bf16 hi + lo parts (x = hi + lo)
__device__ __forceinline__ void split_f16(u32x4_t v, u32x4_t& hi, u32x4_t& lo) {
  f16x8_split_bf16(v, hi, lo);
}

template <int DT, int NMAT, int BN, int BM>
__global__ __launch_bounds__(kThreads, 2) void gemm_kernel(GemmPtrs p, int m_tiles, int n_tiles) {
  using C = GemmCfg<DT, NMAT, BN, BM>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  // ---- tile selection (XCD-aware) --------------------------------------
  const int nwg = gridDim.x;
  const int wg = blockIdx.x;
  int logical = wg;
  if ((nwg & 7) == 0) logical = (wg & 7) * (nwg >> 3) + (wg >> 3);
  const int n_tile = logical / m_tiles;
  const int m_tile = logical - n_tile * m_tiles;
  if (n_tile >= n_tiles) return;
  const int64_t row0 = (int64_t)n_tile * BN;   // weight rows (per matrix)
  const int64_t tok0 = (int64_t)m_tile * BM;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int wr = wave & 1;      // row half
  const int wt = wave >> 1;     // token half
  const int l32 = lane & 31;
  const int j = lane >> 5;

  const int64_t M = p.M, N = p.N, K = p.K;
  const int nk = (int)((K + kBK - 1) / kBK);

  // ---- staging registers ----------------------------------------------
  u32x4_t xr[C::kXChunks];
  u32x4_t wreg[C::kWChunks];
  uint32_t sreg[2];   // up to two (row, 2-byte) scale entries per thread

  auto load_tile = [&](int kt) {
    const int64_t k0 = (int64_t)kt * kBK;
#pragma unroll
    for (int i = 0; i < C::kXChunks; ++i) {
      const int c = tid + i * kThreads;
      const int r = c >> 3;            // 8 chunks per row
      const int cc = c & 7;
      const int64_t tok = tok0 + r;
      const int64_t kk = k0 + cc * 8;
      u32x4_t v = {0u, 0u, 0u, 0u};
      if (tok < M && kk < K) v = *reinterpret_cast<const u32x4_t*>(p.x + tok * K + kk);
      xr[i] = v;
    }
#pragma unroll
    for (int i = 0; i < C::kWChunks; ++i) {
      const int c = tid + i * kThreads;
      const int rr = c >> 1;           // staged row (mat * BN + row)
      const int half = c & 1;
      const int mat = rr / BN;
      const int64_t row = row0 + (rr - mat * BN);
      const int64_t kk = k0 + 32 * half;
      u32x4_t v = {0u, 0u, 0u, 0u};
      if (row < N && kk < K) v = *reinterpret_cast<const u32x4_t*>(p.w[mat] + row * (K / 2) + kk / 2);
      wreg[i] = v;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int rr = tid + i * kThreads;
      uint32_t v = 127u | (127u << 8);
      if (rr < C::kSRows) {
        const int mat = rr / BN;
        const int64_t row = row0 + (rr - mat * BN);
        if (row < N) {
          const uint8_t* sp = p.s[mat] + row * (K / 32) + k0 / 32;
          v = sp[0];
          v |= (k0 + 32 < K ? (uint32_t)sp[1] : 127u) << 8;
        }
      }
      sreg[i] = v;
    }
  };

  auto store_tile = [&](int buf) {
    uint8_t* base = smem + buf * C::kStageBytes;
#pragma unroll
    for (int i = 0; i < C::kXChunks; ++i) {
      const int c = tid + i * kThreads;
      const int r = c >> 3;
      const int cc = c & 7;
      *reinterpret_cast<u32x4_t*>(base + r * kXStride + cc * 16) = xr[i];
    }
    uint8_t* wb = base + C::kXBytes;
#pragma unroll
    for (int i = 0; i < C::kWChunks; ++i) {
      const int c = tid + i * kThreads;
      const int rr = c >> 1;
      const int half = c & 1;
      *reinterpret_cast<u32x4_t*>(wb + rr * kWStride + 16 * half) = wreg[i];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int rr = tid + i * kThreads;
      if (rr < C::kSRows) *reinterpret_cast<uint16_t*>(wb + rr * kWStride + 32) = (uint16_t)sreg[i];
    }
  };

  f32x16_t acc[NMAT][C::TR][C::TT];
#pragma unroll
  for (int m = 0; m < NMAT; ++m)
#pragma unroll
    for (int a = 0; a < C::TR; ++a)
#pragma unroll
      for (int b = 0; b < C::TT; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[m][a][b][v] = 0.0f;

  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load_tile(kt + 1);

    const uint8_t* base = smem + buf * C::kStageBytes;
    const uint8_t* wb = base + C::kXBytes;
    // W operands: one 16-byte run + scale byte per (mat, row block)
    u32x4_t wraw[NMAT][C::TR];
    uint32_t wsc[NMAT][C::TR];
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
      for (int a = 0; a < C::TR; ++a) {
        const int rr = m * BN + wr * C::kRowsPerWave + a * 32 + l32;
        wraw[m][a] = *reinterpret_cast<const u32x4_t*>(wb + rr * kWStride + 16 * j);
        wsc[m][a] = wb[rr * kWStride + 32 + j];
      }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4_t xop[C::TT];
#pragma unroll
      for (int b = 0; b < C::TT; ++b) {
        const int r = wt * C::kToksPerWave + b * 32 + l32;
        xop[b] = *reinterpret_cast<const u32x4_t*>(base + r * kXStride + 64 * j + 16 * s);
      }
#pragma unroll
      for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int a = 0; a < C::TR; ++a) {
          const u32x4_t wop = dq8_bf16(wraw[m][a][s], wsc[m][a]);
#pragma unroll
          for (int b = 0; b < C::TT; ++b) {
            if constexpr (DT == kBF16) {
              acc[m][a][b] = mfma32x32x16(wop, xop[b], acc[m][a][b]);
            } else {
              u32x4_t hi, lo;
              split_f16(xop[b], hi, lo);
              acc[m][a][b] = mfma32x32x16(wop, hi, acc[m][a][b]);
              acc[m][a][b] = mfma32x32x16(wop, lo, acc[m][a][b]);
            }
          }
        }
    }

    if (kt + 1 < nk) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue ------------------------------------------------------
  // acc[..][a][b][v]: token tok0 + wt*BM/2 + b*32 + l32,
  //                   row   row0 + wr*BN/2 + a*32 + 8*(v/4) + 4*j + (v%4)
#pragma unroll
  for (int b = 0; b < C::TT; ++b) {
    const int64_t tok = tok0 + wt * C::kToksPerWave + b * 32 + l32;
    if (tok >= M) continue;
#pragma unroll
    for (int a = 0; a < C::TR; ++a) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t row = row0 + wr * C::kRowsPerWave + a * 32 + 8 * g + 4 * j;
        if (row >= N) continue;     // N % 32 == 0, so the 4 rows are all in or all out
        uint32_t lo, hi;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (NMAT == 2) v[e] = silu_f32(acc[0][a][b][4 * g + e]) * acc[1][a][b][4 * g + e];
          else v[e] = acc[0][a][b][4 * g + e];
        }
        lo = (uint32_t)f32_to_act<DT>(v[0]) | ((uint32_t)f32_to_act<DT>(v[1]) << 16);
        hi = (uint32_t)f32_to_act<DT>(v[2]) | ((uint32_t)f32_to_act<DT>(v[3]) << 16);
        *reinterpret_cast<u32x2_t*>(p.out + tok * N + row) = with_residual4<DT>(u32x2_t{lo, hi}, p.res, tok * N + row);
      }
    }
  }
}

template <int DT, int NMAT, int BN, int BM>
hipError_t launch_gemm(const GemmPtrs& p, hipStream_t st) {
  using C = GemmCfg<DT, NMAT, BN, BM>;
  const int64_t m_tiles = (p.M + BM - 1) / BM;
  const int64_t n_tiles = (p.N + BN - 1) / BN;
  const int64_t nwg = m_tiles * n_tiles;
  if (nwg > 0x7fffffff) return hipErrorInvalidValue;
  const size_t lds = 2 * C::kStageBytes;
  gemm_kernel<DT, NMAT, BN, BM><<<(unsigned)nwg, kThreads, lds, st>>>(p, (int)m_tiles, (int)n_tiles);
  return hipGetLastError();
}

template <int DT>
hipError_t run(const MlpArgs& a, int stage, hipStream_t st) {
  if (stage & kStageGateUp) {
    GemmPtrs p{static_cast<const uint16_t*>(a.x), {a.gate, a.up}, {a.gate_scale, a.up_scale},
               static_cast<uint16_t*>(a.tmp), a.n, a.inter, a.hidden, nullptr};
    hipError_t e = launch_gemm<DT, 2, 128, 128>(p, st);
    if (e != hipSuccess) return e;
  }
  if (stage & kStageDown) {
    GemmPtrs p{static_cast<const uint16_t*>(a.tmp), {a.down, a.down}, {a.down_scale, a.down_scale},
               static_cast<uint16_t*>(a.out), a.n, a.hidden, a.inter, static_cast<const uint16_t*>(a.residual)};
    return launch_gemm<DT, 1, 128, 128>(p, st);
  }
  return hipSuccess;
}

}  // namespace

hipError_t launch_gemm_mlp(const MlpArgs& a, int stage, hipStream_t stream) {
  return a.dtype == kBF16 ? run<kBF16>(a, stage, stream) : run<kF16>(a, stage, stream);
}

}  // namespace tinyinfer
