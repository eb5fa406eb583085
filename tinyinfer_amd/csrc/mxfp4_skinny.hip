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
//
// Memory pipeline: a wave owns at most NCH chunks and issues every weight and
// scale load of them before its first MFMA, so the whole grid puts (nearly)
// the whole weight matrix in flight at once and pays the HBM latency once;
// activations are fetched one chunk ahead of the MFMAs that use them.
#include <cstdlib>

#include "mxfp4_common.hpp"
#include "mxfp4_launch.hpp"

namespace tinyinfer {

namespace {

constexpr int kChunkK = 128;      // K elements per lane-group load (64 lanes x 16 B)

template <int T>
__device__ __forceinline__ void load_x_chunk(const uint16_t* __restrict__ x, int64_t m_base, int64_t M,
                                             int64_t K, int64_t k0, bool ok, int r, u32x4_t (&dst)[T * 4]) {
#pragma unroll
  for (int tt = 0; tt < T; ++tt) {
    const int64_t tok = m_base + tt * 16 + r;
    const bool tok_ok = ok && tok < M;
    const uint16_t* xp = x + (tok_ok ? tok : 0) * K + (ok ? k0 : 0);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      u32x4_t v = {0u, 0u, 0u, 0u};
      if (tok_ok) v = *reinterpret_cast<const u32x4_t*>(xp + 8 * t);
      dst[tt * 4 + t] = v;
    }
  }
}

// MFMA part of a batch: dequantize chunk u's four dwords and multiply them
// into the token tiles, activations fetched one chunk ahead.
template <int DT, int T, int NCH, bool FAST>
__device__ __forceinline__ void batch_mfma(const uint16_t* __restrict__ x, int64_t m_base, int64_t M,
                                           int64_t K, int c0, int c1, const u32x4_t (&wv)[NCH],
                                           const uint32_t (&sb)[NCH], f32x4_t (&acc)[T]) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int q = lane >> 4;
  auto chunk_ok = [&](int u, int64_t& k0) {
    k0 = (int64_t)(c0 + u) * kChunkK + 32 * q;
    return (c0 + u < c1) && (k0 < K);
  };
  auto compute = [&](int u, const u32x4_t (&xc)[T * 4]) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const u32x4_t a = FAST ? dq8_bf16_fast(wv[u][t], sb[u]) : dq8_bf16_exact(wv[u][t], sb[u]);
#pragma unroll
      for (int tt = 0; tt < T; ++tt) {
        if constexpr (DT == kBF16) {
          acc[tt] = mfma16x16x32(a, xc[tt * 4 + t], acc[tt]);
        } else {
          u32x4_t hi, lo;
          f16x8_split_bf16(xc[tt * 4 + t], hi, lo);
          acc[tt] = mfma16x16x32(a, hi, acc[tt]);
          acc[tt] = mfma16x16x32(a, lo, acc[tt]);
        }
      }
    }
  };
  u32x4_t xa[T * 4], xb[T * 4];
  int64_t kx;
  bool okx = chunk_ok(0, kx);
  load_x_chunk<T>(x, m_base, M, K, kx, okx, r, xa);
#pragma unroll
  for (int u = 0; u < NCH; u += 2) {
    if (u + 1 < NCH) {
      okx = chunk_ok(u + 1, kx);
      load_x_chunk<T>(x, m_base, M, K, kx, okx, r, xb);
    }
    if (c0 + u < c1) compute(u, xa);
    if (u + 2 < NCH) {
      okx = chunk_ok(u + 2, kx);
      load_x_chunk<T>(x, m_base, M, K, kx, okx, r, xa);
    }
    if (u + 1 < NCH && c0 + u + 1 < c1) compute(u + 1, xb);
  }
}

// Whole batch in bounds and the scale rows 16-byte aligned: straight-line
// code, so the compiler can wait for exactly the loads each step needs.
// The batch's scale bytes (16 rows x 4*NCH) are fetched first with one
// coalesced 16-byte load per lane into the wave's private LDS slice `sl`,
// then every weight load is issued, then the slice is read back per lane.
template <int DT, int T, int NCH>
__device__ __forceinline__ void batch_fast(const uint16_t* __restrict__ x, const uint8_t* __restrict__ w,
                                           const uint8_t* __restrict__ ws, int64_t m_base, int64_t M,
                                           int64_t K, int64_t row0, int c0, f32x4_t (&acc)[T],
                                           uint8_t* sl) {
  constexpr int kSRow = 4 * NCH;                 // scale bytes per row per batch
  constexpr int kPieces = kSRow / 16;            // 16-byte pieces per row
  static_assert(kSRow % 16 == 0, "NCH must be a multiple of 4");
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int q = lane >> 4;
  const int s_row = lane / kPieces, s_piece = lane % kPieces;
  u32x4_t sp = {0u, 0u, 0u, 0u};
  if (lane < 16 * kPieces)
    sp = *reinterpret_cast<const u32x4_t*>(ws + (row0 + s_row) * (K / 32) + (int64_t)c0 * 4 + 16 * s_piece);
  // R is a multiple of 32 (checked at the C ABI), so every row of the tile exists.
  const uint8_t* wp = w + (row0 + r) * (K / 2) + 16 * q + (int64_t)c0 * (kChunkK / 2);
  u32x4_t wv[NCH];
#pragma unroll
  for (int u = 0; u < NCH; ++u)
    wv[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wp + u * (kChunkK / 2)));
  if (lane < 16 * kPieces) *reinterpret_cast<u32x4_t*>(sl + s_row * kSRow + 16 * s_piece) = sp;
  // other lanes' bytes are read back: keep the reads after the writes
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  uint32_t sb[NCH];
  bool ok = true;
#pragma unroll
  for (int u = 0; u < NCH; ++u) {
    sb[u] = sl[r * kSRow + 4 * u + q];
    ok = ok && e8m0_fast_ok(sb[u]);
  }
  if (wave_all(ok)) batch_mfma<DT, T, NCH, true>(x, m_base, M, K, c0, c0 + NCH, wv, sb, acc);
  else batch_mfma<DT, T, NCH, false>(x, m_base, M, K, c0, c0 + NCH, wv, sb, acc);
}

// Any batch (partial K tail, unaligned scales): predicated loads, scale bytes
// straight from global memory.
template <int DT, int T, int NCH>
__device__ __forceinline__ void batch_generic(const uint16_t* __restrict__ x, const uint8_t* __restrict__ w,
                                              const uint8_t* __restrict__ ws, int64_t m_base, int64_t M,
                                              int64_t K, int64_t row0, int c0, int c1, f32x4_t (&acc)[T]) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int q = lane >> 4;
  const uint8_t* wrow = w + (row0 + r) * (K / 2) + 16 * q;
  const uint8_t* srow = ws + (row0 + r) * (K / 32) + q;
  u32x4_t wv[NCH];
  uint32_t sb[NCH];
#pragma unroll
  for (int u = 0; u < NCH; ++u) {
    const int64_t k0 = (int64_t)(c0 + u) * kChunkK + 32 * q;
    const bool in = (c0 + u < c1) && (k0 < K);
    wv[u] = u32x4_t{0u, 0u, 0u, 0u};
    sb[u] = 127u;
    if (in) {
      wv[u] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4_t*>(wrow + (int64_t)(c0 + u) * (kChunkK / 2)));
      sb[u] = srow[(int64_t)(c0 + u) * (kChunkK / 32)];
    }
  }
  bool ok = true;
#pragma unroll
  for (int u = 0; u < NCH; ++u) ok = ok && e8m0_fast_ok(sb[u]);
  if (wave_all(ok)) batch_mfma<DT, T, NCH, true>(x, m_base, M, K, c0, c1, wv, sb, acc);
  else batch_mfma<DT, T, NCH, false>(x, m_base, M, K, c0, c1, wv, sb, acc);
}

// A wave's whole K slice [c0, c1), in batches of NCH chunks.
template <int DT, int T, int NCH>
__device__ __forceinline__ void wave_skinny(const uint16_t* __restrict__ x, const uint8_t* __restrict__ w,
                                            const uint8_t* __restrict__ ws, int64_t m_base, int64_t M,
                                            int64_t K, int64_t R, int64_t row0, int c0, int c1,
                                            f32x4_t (&acc)[T], uint8_t* sl) {
  (void)R;
  const bool aligned = ((K / 32) % 16 == 0) && ((reinterpret_cast<uintptr_t>(ws) & 15u) == 0);
  for (int cb = c0; cb < c1; cb += NCH) {
    const int ce = cb + NCH < c1 ? cb + NCH : c1;
    if (aligned && ce - cb == NCH && cb % 4 == 0 && (int64_t)ce * kChunkK <= K)
      batch_fast<DT, T, NCH>(x, w, ws, m_base, M, K, row0, cb, acc, sl);
    else
      batch_generic<DT, T, NCH>(x, w, ws, m_base, M, K, row0, cb, ce, acc);
  }
}

// GATEUP: out = h[M, R] = SiLU(x W0^T) * (x W1^T), K = hidden, R = inter.
// else:   out = y[M, R] = x W0^T, K = inter, R = hidden.
template <int DT, int T, int NCH, bool GATEUP, int NW>
__global__ __launch_bounds__(NW * 64) void skinny_kernel(const uint16_t* __restrict__ x,
                                                         const uint8_t* __restrict__ w0,
                                                         const uint8_t* __restrict__ s0,
                                                         const uint8_t* __restrict__ w1,
                                                         const uint8_t* __restrict__ s1, int64_t M,
                                                         int64_t K, int64_t R,
                                                         uint16_t* out,
                                                         const uint16_t* res) {   // res may alias out
  constexpr int KS = GATEUP ? NW / 2 : NW;   // K slices
  __shared__ f32x4_t red[NW][T][64];
  __shared__ __attribute__((aligned(16))) uint8_t scale_slices[NW][16 * 4 * NCH];
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
  wave_skinny<DT, T, NCH>(x, mat ? w1 : w0, mat ? s1 : s0, m_base, M, K, R, row0, c0, c1, acc,
                          scale_slices[wave]);

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
          out[tok * R + row] = with_residual<DT>(f32_to_act<DT>(val), res, tok * R + row);
        }
      }
    }
  }
}

template <int DT, int T, int NCH, bool GATEUP, int NW>
void launch_one(const uint16_t* x, const uint8_t* w0, const uint8_t* s0, const uint8_t* w1,
                const uint8_t* s1, int64_t M, int64_t K, int64_t R, uint16_t* out, hipStream_t st,
                const uint16_t* res) {
  dim3 grid((unsigned)((R + 15) / 16), (unsigned)((M + 16 * T - 1) / (16 * T)));
  skinny_kernel<DT, T, NCH, GATEUP, NW><<<grid, NW * 64, 0, st>>>(x, w0, s0, w1, s1, M, K, R, out, res);
}

// Test/tuning override: the option TINYINFER_SKINNY_NW=<4|8> forces the
// waves per workgroup (0: chosen below).
int forced_nw() { return option(kOptSkinnyNw); }

// Waves per workgroup (4 or 8; 16 would cap registers at 128 and spill).
// 4 when each wave's K slice fits one NCH batch and the grid still has
// >= 2048 waves (8 per CU); otherwise 8, which halves each slice and doubles
// the waves.  At the Qwen3-8B shapes this puts the whole matrix in flight in
// one round of waves: gate_up 768 tiles x 4 waves x 16 chunks, down 256
// tiles x 8 waves x 12 chunks.
template <int DT, int T, int NCH, bool GATEUP>
void launch_nw(const uint16_t* x, const uint8_t* w0, const uint8_t* s0, const uint8_t* w1,
               const uint8_t* s1, int64_t M, int64_t K, int64_t R, uint16_t* out, hipStream_t st,
               const uint16_t* res) {
  const int64_t tiles = (R + 15) / 16;
  const int64_t chunks = (K + kChunkK - 1) / kChunkK;
  const int64_t mats = GATEUP ? 2 : 1;
  int nw = forced_nw();
  if (nw == 0) {
    const int64_t per_wave4 = (chunks * mats + 3) / 4;
    nw = (per_wave4 <= NCH && tiles * 4 >= 2048) ? 4 : 8;
  }
  if (nw == 4) launch_one<DT, T, NCH, GATEUP, 4>(x, w0, s0, w1, s1, M, K, R, out, st, res);
  else launch_one<DT, T, NCH, GATEUP, 8>(x, w0, s0, w1, s1, M, K, R, out, st, res);
}

// Chunk depth per wave: NCH weight dwordx4 loads in flight per lane; fewer
// as the per-chunk activation registers (T tiles x 2 x 4 dwordx4) grow.
template <int DT, bool GATEUP>
void launch_t(const uint16_t* x, const uint8_t* w0, const uint8_t* s0, const uint8_t* w1,
              const uint8_t* s1, int64_t M, int64_t K, int64_t R, uint16_t* out, hipStream_t st,
              const uint16_t* res = nullptr) {
  const int64_t t = M >= 64 ? 4 : (M + 15) / 16;
  switch (t) {
    case 1: launch_nw<DT, 1, 16, GATEUP>(x, w0, s0, w1, s1, M, K, R, out, st, res); break;
    case 2: launch_nw<DT, 2, 8, GATEUP>(x, w0, s0, w1, s1, M, K, R, out, st, res); break;
    case 3: launch_nw<DT, 3, 4, GATEUP>(x, w0, s0, w1, s1, M, K, R, out, st, res); break;
    default: launch_nw<DT, 4, 4, GATEUP>(x, w0, s0, w1, s1, M, K, R, out, st, res); break;
  }
}

template <int DT>
hipError_t run(const MlpArgs& a, int stage, hipStream_t st) {
  const uint16_t* x = static_cast<const uint16_t*>(a.x);
  uint16_t* h = static_cast<uint16_t*>(a.tmp);
  uint16_t* y = static_cast<uint16_t*>(a.out);
  if (stage & kStageGateUp) {
    launch_t<DT, true>(x, a.gate, a.gate_scale, a.up, a.up_scale, a.n, a.hidden, a.inter, h, st);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (stage & kStageDown) {
    launch_t<DT, false>(h, a.down, a.down_scale, nullptr, nullptr, a.n, a.inter, a.hidden, y, st,
                        static_cast<const uint16_t*>(a.residual));
    return hipGetLastError();
  }
  return hipSuccess;
}

}  // namespace

hipError_t launch_skinny_mlp(const MlpArgs& a, int stage, hipStream_t stream) {
  return a.dtype == kBF16 ? run<kBF16>(a, stage, stream) : run<kF16>(a, stage, stream);
}

}  // namespace tinyinfer
