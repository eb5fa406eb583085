// Skinny MXFP4 MLP path (decode / small batch): each weight byte is streamed
// from HBM once per 64 tokens.
//
// Replaces the reference's per-token GEMV kernels mlp_stage1_mxfp4 /
// mlp_stage2_mxfp4 (tinyinfer/csrc/mlp_fp4.cu:79-142, 365-426), which launch
// grid.y = N and re-read every weight once per token with scalar FMAs.
//
// Mapping (per workgroup: one 16-row tile of the weight matrix, all tokens
// of a 16*T token group):
//   * MFMA v_mfma_f32_16x16x32_bf16 with the WEIGHTS as the 16-row A operand
//     and the tokens as the 16-column B operand: C[row][token].
//   * Lane l = 16*q + r loads 16 bytes = one whole 32-element K block of weight
//     row r (one e8m0 byte), at K offset 32*q inside a 128-wide K chunk.
//     The four dwords feed four MFMAs; in MFMA t, lane (r, q) supplies
//     elements 32q + 8t .. 32q + 8t + 7 of row r, and lane (c, q) of the B
//     operand supplies the same K elements of token c. The K order inside an
//     MFMA is a permutation shared by both operands, so the sum is unchanged.
//   * Waves of a workgroup split K (and, for gate_up, the two matrices); an
//     LDS reduction combines them and the epilogue applies SiLU(g)*u (gate_up)
//     or plain rounding (down).
#include "mxfp4_common.hpp"
#include "mxfp4_launch.hpp"

namespace tinyinfer {

namespace {

constexpr int kChunkK = 128;      // K elements per lane-group load (64 lanes x 16 B)

// Chunks in flight per wave: 4 at one token tile, fewer as the per-chunk
// activation registers (T tiles x 4 dwordx4) grow.
template <int T>
constexpr int unroll_for() { return T == 1 ? 4 : (T == 2 ? 2 : 1); }

template <int DT>
__device__ __forceinline__ u32x4_t load_act8(const uint16_t* p, bool ok) {
  u32x4_t v = {0u, 0u, 0u, 0u};
  if (ok) v = *reinterpret_cast<const u32x4_t*>(p);
  return v;
}

// One wave's contribution: rows [row0, row0+16) of W, K chunks [c0, c1).
template <int DT, int T>
__device__ __forceinline__ void wave_skinny(const uint16_t* __restrict__ x, const uint8_t* __restrict__ w,
                                            const uint8_t* __restrict__ ws, int64_t m_base, int64_t M,
                                            int64_t K, int64_t R, int64_t row0, int c0, int c1,
                                            f32x4_t (&acc)[T]) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int q = lane >> 4;
  const int64_t row = row0 + r;
  const bool row_ok = row < R;
  const int64_t rowc = row_ok ? row : 0;
  const uint8_t* wrow = w + rowc * (K / 2);
  const uint8_t* srow = ws + rowc * (K / 32);
  constexpr int kUnroll = unroll_for<T>();
  for (int c = c0; c < c1; c += kUnroll) {
    u32x4_t wv[kUnroll];
    uint32_t sb[kUnroll];
    u32x4_t xv[kUnroll][T][4];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t k0 = (int64_t)(c + u) * kChunkK + 32 * q;
      const bool ok = (c + u < c1) && (k0 < K);
      wv[u] = u32x4_t{0u, 0u, 0u, 0u};
      sb[u] = 127u;
      if (ok && row_ok) {
        wv[u] = *reinterpret_cast<const u32x4_t*>(wrow + k0 / 2);
        sb[u] = srow[k0 / 32];
      }
#pragma unroll
      for (int tt = 0; tt < T; ++tt) {
        const int64_t tok = m_base + tt * 16 + r;
        const bool tok_ok = ok && tok < M;
        const uint16_t* xp = x + (tok_ok ? tok : 0) * K + (ok ? k0 : 0);
#pragma unroll
        for (int t = 0; t < 4; ++t) xv[u][tt][t] = load_act8<DT>(xp + 8 * t, tok_ok);
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const u32x4_t a = dq8_bf16(wv[u][t], sb[u]);
#pragma unroll
        for (int tt = 0; tt < T; ++tt) {
          if constexpr (DT == kBF16) {
            acc[tt] = mfma16x16x32(a, xv[u][tt][t], acc[tt]);
          } else {
            u32x4_t hi, lo;
            f16x8_split_bf16(xv[u][tt][t], hi, lo);
            acc[tt] = mfma16x16x32(a, hi, acc[tt]);
            acc[tt] = mfma16x16x32(a, lo, acc[tt]);
          }
        }
      }
    }
  }
}

// GATEUP: out = h[M, R] = SiLU(x W0^T) * (x W1^T), K = hidden, R = inter.
// else:   out = y[M, R] = x W0^T, K = inter, R = hidden.
template <int DT, int T, bool GATEUP, int NW>
__global__ __launch_bounds__(NW * 64) void skinny_kernel(const uint16_t* __restrict__ x,
                                                         const uint8_t* __restrict__ w0,
                                                         const uint8_t* __restrict__ s0,
                                                         const uint8_t* __restrict__ w1,
                                                         const uint8_t* __restrict__ s1, int64_t M,
                                                         int64_t K, int64_t R,
                                                         uint16_t* __restrict__ out) {
  constexpr int KS = GATEUP ? NW / 2 : NW;   // K slices
  __shared__ f32x4_t red[NW][T][64];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int mat = GATEUP ? (wave & 1) : 0;
  const int ks = GATEUP ? (wave >> 1) : wave;
  const int64_t row0 = (int64_t)blockIdx.x * 16;
  const int64_t m_base = (int64_t)blockIdx.y * 16 * T;
  const int nchunk = (int)((K + kChunkK - 1) / kChunkK);
  const int c0 = (int)((int64_t)nchunk * ks / KS);
  const int c1 = (int)((int64_t)nchunk * (ks + 1) / KS);

  f32x4_t acc[T];
#pragma unroll
  for (int tt = 0; tt < T; ++tt) acc[tt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  wave_skinny<DT, T>(x, mat ? w1 : w0, mat ? s1 : s0, m_base, M, K, R, row0, c0, c1, acc);

#pragma unroll
  for (int tt = 0; tt < T; ++tt) red[wave][tt][lane] = acc[tt];
  __syncthreads();

  // Epilogue: lane owns C rows 4*(lane/16)+v (weight rows), column lane%16 (token).
  // T*64 (token-tile, lane) pairs spread over the first T waves.
  if (wave < T) {
    const int tt = wave;
    f32x4_t g = {0.f, 0.f, 0.f, 0.f}, u = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if constexpr (GATEUP) {
        g += red[2 * s][tt][lane];
        u += red[2 * s + 1][tt][lane];
      } else {
        g += red[s][tt][lane];
      }
    }
    const int64_t tok = m_base + tt * 16 + (lane & 15);
    if (tok < M) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t row = row0 + 4 * (lane >> 4) + v;
        if (row < R) {
          const float val = GATEUP ? silu_f32(g[v]) * u[v] : g[v];
          out[tok * R + row] = f32_to_act<DT>(val);
        }
      }
    }
  }
}

template <int DT, int T, bool GATEUP, int NW>
void launch_one(const uint16_t* x, const uint8_t* w0, const uint8_t* s0, const uint8_t* w1,
                const uint8_t* s1, int64_t M, int64_t K, int64_t R, uint16_t* out, hipStream_t st) {
  dim3 grid((unsigned)((R + 15) / 16), (unsigned)((M + 16 * T - 1) / (16 * T)));
  skinny_kernel<DT, T, GATEUP, NW><<<grid, NW * 64, 0, st>>>(x, w0, s0, w1, s1, M, K, R, out);
}

// Waves per workgroup: enough K slices that the grid holds >= ~8 waves per CU.
template <int DT, int T, bool GATEUP>
void launch_nw(const uint16_t* x, const uint8_t* w0, const uint8_t* s0, const uint8_t* w1,
               const uint8_t* s1, int64_t M, int64_t K, int64_t R, uint16_t* out, hipStream_t st) {
  const int64_t tiles = (R + 15) / 16;
  const int64_t chunks = (K + kChunkK - 1) / kChunkK;
  // target waves in the grid ~ 3072 (256 CUs x 12)
  int64_t nw = (3072 + tiles - 1) / tiles;
  if (GATEUP) nw = (nw + 1) & ~int64_t(1);
  const int64_t max_nw_by_k = GATEUP ? 2 * chunks : chunks;
  if (nw > max_nw_by_k) nw = max_nw_by_k;
  if (nw <= 4) launch_one<DT, T, GATEUP, 4>(x, w0, s0, w1, s1, M, K, R, out, st);
  else if (nw <= 8) launch_one<DT, T, GATEUP, 8>(x, w0, s0, w1, s1, M, K, R, out, st);
  else launch_one<DT, T, GATEUP, 16>(x, w0, s0, w1, s1, M, K, R, out, st);
}

template <int DT, bool GATEUP>
void launch_t(const uint16_t* x, const uint8_t* w0, const uint8_t* s0, const uint8_t* w1,
              const uint8_t* s1, int64_t M, int64_t K, int64_t R, uint16_t* out, hipStream_t st) {
  const int64_t t = M >= 64 ? 4 : (M + 15) / 16;
  switch (t) {
    case 1: launch_nw<DT, 1, GATEUP>(x, w0, s0, w1, s1, M, K, R, out, st); break;
    case 2: launch_nw<DT, 2, GATEUP>(x, w0, s0, w1, s1, M, K, R, out, st); break;
    case 3: launch_nw<DT, 3, GATEUP>(x, w0, s0, w1, s1, M, K, R, out, st); break;
    default: launch_nw<DT, 4, GATEUP>(x, w0, s0, w1, s1, M, K, R, out, st); break;
  }
}

template <int DT>
hipError_t run(const MlpArgs& a, hipStream_t st) {
  const uint16_t* x = static_cast<const uint16_t*>(a.x);
  uint16_t* h = static_cast<uint16_t*>(a.tmp);
  uint16_t* y = static_cast<uint16_t*>(a.out);
  launch_t<DT, true>(x, a.gate, a.gate_scale, a.up, a.up_scale, a.n, a.hidden, a.inter, h, st);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  launch_t<DT, false>(h, a.down, a.down_scale, nullptr, nullptr, a.n, a.inter, a.hidden, y, st);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_skinny_mlp(const MlpArgs& a, hipStream_t stream) {
  return a.dtype == kBF16 ? run<kBF16>(a, stream) : run<kF16>(a, stream);
}

}  // namespace tinyinfer
