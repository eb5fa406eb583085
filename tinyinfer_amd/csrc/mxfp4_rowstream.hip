// Row-streaming MXFP4 GEMV for one token (decode at batch 1): one kernel per
// MLP stage, the same contract as the M <= 8 stream kernel (mxfp4_stream.hip)
// for the reference's per-token GEMV kernels mlp_stage1_mxfp4 /
// mlp_stage2_mxfp4 (tinyinfer/csrc/mlp_fp4.cu:79-142, 365-426).
//
// At one token the load pattern decides the speed, so the work is laid out
// for it (each choice measured on MI355X with a read-only kernel of the same
// bytes):
//   * every weight load instruction reads 1 KB of ONE row (lane l: the 16
//     bytes of 32-element block 64c + l of the row's chunk c).  A load whose
//     lanes span 8 rows at a 2 KB stride streams about 10% slower;
//   * a wave owns whole rows (row gw + j * waves of the grid), both matrices
//     for gate_up, so no partial sums cross waves: no LDS slots, counters or
//     last-arriver epilogue inside the stream;
//   * the e8m0 bytes of a chunk are the 64 contiguous bytes of its scale row:
//     one byte load per lane next to the weight load (one cache line), so
//     no scale staging and no workgroup barrier wait on scales;
//   * x (and the RMSNorm weight) are staged once through LDS with one
//     barrier and copied into VGPRs: lane l keeps the 32 activations of its
//     own block of every chunk;
//   * two rows in flight per wave: the loads of row j+2 are issued as soon
//     as row j has been multiplied.
//
// MFMA mapping: with A = the lane's 8 dequantized weights and B = the same
// lane's 8 activations, the diagonal entry C[i][i] of
// v_mfma_f32_16x16x32_bf16 sums the products of lanes i, i+16, i+32, i+48;
// the 16 diagonal entries (lanes 0-3, 20-23, 40-43, 60-63 of the
// accumulator) added over the wave are the row's dot product.  Four MFMAs
// per load, as many as the 8-row layout spends.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "mxfp4_common.hpp"
#include "mxfp4_launch.hpp"

namespace tinyinfer {

namespace {

constexpr int kRW = 8;                 // waves per workgroup
constexpr int kRThreads = kRW * 64;
constexpr int kChunkBlocks = 64;       // 32-element blocks per load (1 KB of fp4)
constexpr int kChunkK = kChunkBlocks * kBlock;
constexpr int kMaxUC = 6;              // chunks per wave (down; gate_up 4)

struct RowArgs {
  const uint16_t* x;       // [K] activations (x for gate_up, h for down)
  const uint8_t* w0;       // [R, K/2] gate (or down)
  const uint8_t* s0;       // [R, K/32]
  const uint8_t* w1;       // [R, K/2] up (gate_up only; else = w0)
  const uint8_t* s1;
  uint16_t* out;           // [R]
  const uint16_t* res;     // down only: residual [R] added to out, or null
  const uint16_t* norm_w;  // gate_up only: RMSNorm weight [K], or null
  float eps;
  uint16_t* xn;            // with norm_w: workgroup 0 writes the normalized x [K]
  int K, R;
  int nc;                  // chunks per row, ceil(K / 2048)
  int nblk;                // K / 32
  int full;                // every chunk has all 64 blocks (K % 2048 == 0)
  int rows_max;            // rows of the busiest wave
  int lds_nw, lds_sum, lds_out;   // LDS byte offsets
};

template <int UC, bool GATEUP>
struct RowBuf {
  static constexpr int kMats = GATEUP ? 2 : 1;
  u32x4_t w[kMats * UC];
  uint32_t s[kMats * UC];   // the aligned dword holding the lane's scale byte (byte lane & 3)
};

// Loads of one row (clamped to the wave's last row past its end: those
// repeat addresses already read and are never used).  Scale bytes first, so
// they have landed whenever the weights they scale have.  Each lane loads the
// aligned dword that holds its scale byte (K % 128 == 0 keeps scale rows
// dword-aligned): a byte load's zero-extension is a VALU op the compiler may
// place right after the issue, where it would wait for the load.
template <int UC, bool GATEUP>
__device__ __forceinline__ void issue_row(const RowArgs& a, int64_t row, int cb, int ncs, RowBuf<UC, GATEUP>& b) {
  constexpr int kMats = GATEUP ? 2 : 1;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int m = 0; m < kMats; ++m) {
    const uint8_t* sp = (m ? a.s1 : a.s0) + row * a.nblk;
#pragma unroll
    for (int q = 0; q < UC; ++q) {
      const int c = cb + (q < ncs ? q : ncs - 1);
      const int blk = c * kChunkBlocks + lane;
      b.s[m * UC + q] = *reinterpret_cast<const uint32_t*>(sp + ((blk < a.nblk ? blk : a.nblk - 1) & ~3));
    }
  }
#pragma unroll
  for (int m = 0; m < kMats; ++m) {
    const uint8_t* wp = (m ? a.w1 : a.w0) + row * (a.K / 2);
#pragma unroll
    for (int q = 0; q < UC; ++q) {
      const int c = cb + (q < ncs ? q : ncs - 1);
      const int blk = c * kChunkBlocks + lane;
      b.w[m * UC + q] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4_t*>(wp + 16 * (int64_t)(blk < a.nblk ? blk : a.nblk - 1)));
    }
  }
  // rows complete in issue order only if their loads are issued in program
  // order: keep the scheduler from interleaving two rows' loads
  __builtin_amdgcn_sched_barrier(0);
}

__device__ __forceinline__ uint32_t scale_byte(uint32_t dw) {
  return (dw >> (8 * (threadIdx.x & 3))) & 0xffu;
}

// The row's dot products (one per matrix and token: T tokens are T MFMA
// passes over the same dequantized operand, each with that token's
// activations) over chunks [cb, cb + ncs) into acc, one accumulator per
// 8-element slice t (one token) or per slice pair (two tokens): independent
// MFMA chains instead of one
// (a chain waits out each MFMA's latency; at one token the multiply is
// otherwise what a wave spends its time on once its rows have landed).  FULL: every lane of
// every slot holds a real block; otherwise slots past the range (they hold a
// repeat of its last chunk) and lanes past K multiply a zero
// weight (scale 1.0) by the zero activation they hold.  bf16: FAST when
// every scale byte is in the hardware bf16 conversion's exact range.  fp16
// (x held as fp16): FAST when every scale byte is e8m0_f16_ok, the weights
// converted to fp16 on fp16 MFMAs; otherwise the exact bf16 weights against
// x's exact bf16 hi and lo parts, two MFMAs.
template <int DT, int UC, bool GATEUP, bool FAST, bool FULL, int T>
__device__ __forceinline__ void mma_row(const RowArgs& a, int cb, int ncs, const RowBuf<UC, GATEUP>& b,
                                        const u32x4_t (&xr)[T][UC][4], const u32x4_t (&xl)[T][UC][4],
                                        f32x4_t (&acc)[2][T][4 / T]) {
  constexpr int kMats = GATEUP ? 2 : 1;
  constexpr int kCh = 4 / T;                  // accumulator chains per (matrix, token)
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int m = 0; m < kMats; ++m) {
#pragma unroll
    for (int q = 0; q < UC; ++q) {
      const bool valid = FULL || (q < ncs && (cb + q) * kChunkBlocks + lane < a.nblk);
      const uint32_t sb = valid ? scale_byte(b.s[m * UC + q]) : 127u;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t wq = valid ? b.w[m * UC + q][t] : 0u;
        const u32x4_t wa = !FAST ? dq8_bf16_exact(wq, sb) : DT == kBF16 ? dq8_bf16_fast(wq, sb) : dq8_f16_fast(wq, sb);
#pragma unroll
        for (int tk = 0; tk < T; ++tk) {
          f32x4_t& c = acc[m][tk][t % kCh];
          if constexpr (DT == kBF16) {
            c = mfma16x16x32(wa, xr[tk][q][t], c);
          } else if constexpr (FAST) {
            c = mfma16x16x32_f16(wa, xr[tk][q][t], c);
          } else {
            u32x4_t xh, xlo;
            f16x8_split_bf16(xr[tk][q][t], xh, xlo);
            c = mfma16x16x32(wa, xlo, mfma16x16x32(wa, xh, c));
          }
        }
      }
    }
  }
}

// Sum of the diagonal of a 16x16 accumulator (lane l holds C[4(l/16)+v][l%16]).
__device__ __forceinline__ float diag_sum(const f32x4_t& c) {
  const int lane = threadIdx.x & 63;
  const int v = lane & 3;
  float d = v == 0 ? c[0] : v == 1 ? c[1] : v == 2 ? c[2] : c[3];
  d = ((lane & 15) >> 2) == (lane >> 4) ? d : 0.f;
  return wave_sum64(d);
}

// S waves share each row (S divides the workgroup's 8 waves): wave s of the
// group multiplies chunks [s nc / S, (s + 1) nc / S) and the S partial sums
// are added in order at the end.  UC is the largest share.
template <int DT, int UC, bool GATEUP, int S, int T>
__global__ __launch_bounds__(kRThreads, 1) void rowstream_kernel(RowArgs a) {
  static_assert(kRW % S == 0, "the waves sharing a row are in one workgroup");
  static_assert(T == 1 || (T == 2 && DT == kBF16), "one token, or two in bf16");
  // 16-byte x chunks per thread: T K / 8 <= 256 UC S T (x is staged whole)
  constexpr int kXPre = (256 * UC * S * T + kRThreads - 1) / kRThreads;
  constexpr int kCh = 4 / T;
  extern __shared__ __align__(16) uint8_t lds[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int nslots = gridDim.x * (kRW / S);
  const int slot = blockIdx.x * (kRW / S) + wave / S;   // row slot: rows slot + j * nslots
  const int sp = wave % S;                               // this wave's part of the row
  const int cb = sp * a.nc / S;
  const int ncs = (sp + 1) * a.nc / S - cb;
  const int rows = slot < a.R ? (a.R - slot + nslots - 1) / nslots : 0;

  // Prologue loads, issued before the first weights (loads complete in
  // issue order): x ([T, K], rows contiguous), and the norm weight when there
  // is one.
  const int nxr = a.K / 8;                   // 16-byte chunks per token row
  const int nxc = T * nxr;
  const bool norm = GATEUP && a.norm_w != nullptr;
  u32x4_t xv[kXPre], nv[kXPre];
#pragma unroll
  for (int p = 0; p < kXPre; ++p) {
    const int c = threadIdx.x + p * kRThreads;
    xv[p] = *reinterpret_cast<const u32x4_t*>(a.x + 8 * (c < nxc ? c : nxc - 1));
  }
  if (norm) {
#pragma unroll
    for (int p = 0; p < kXPre; ++p) {
      const int c = threadIdx.x + p * kRThreads;
      nv[p] = *reinterpret_cast<const u32x4_t*>(a.norm_w + 8 * (c < nxr ? c : nxr - 1));
    }
  }

  // the first two rows in flight (separate named buffers: an array indexed
  // by the pipeline slot would end up in scratch)
  RowBuf<UC, GATEUP> b0, b1;
  // (a wave without rows loads a row it does not use: a conditional issue
  // would make the compiler drain the load queue before the LDS stores)
  auto row_of = [&](int j) {
    return rows > 0 ? (int64_t)slot + (int64_t)(j < rows ? j : rows - 1) * nslots : (int64_t)(slot % a.R);
  };
  issue_row<UC, GATEUP>(a, row_of(0), cb, ncs, b0);
  issue_row<UC, GATEUP>(a, row_of(1), cb, ncs, b1);

  // LDS position of 16-byte x chunk c of a token row (elements 8c .. 8c+7 =
  // slice c % 4 of block c / 4): slice-major, so the copy into registers
  // below, where lane l reads slice t of its block, touches consecutive
  // 16-byte words; token rows 2K bytes apart
  const int plane = a.K / 2;                 // bytes per slice plane
  auto xpos = [&](int c) { return (c & 3) * plane + 16 * (c >> 2); };
  // x (and the norm weight) into LDS; with a norm, each wave's sum of the
  // squares of the chunks it loaded, per token (fixed order: per thread,
  // then the wave)
  float* nsum = reinterpret_cast<float*>(lds + a.lds_sum);   // [kRW][T]
  float sq[T];
#pragma unroll
  for (int tk = 0; tk < T; ++tk) sq[tk] = 0.f;
#pragma unroll
  for (int p = 0; p < kXPre; ++p) {
    const int c = threadIdx.x + p * kRThreads;
    if (c < nxc) {
      const int tk = c / nxr, cc = c - tk * nxr;
      *reinterpret_cast<u32x4_t*>(lds + tk * 2 * a.K + xpos(cc)) = xv[p];
      if (norm) {
        if (c < nxr) *reinterpret_cast<u32x4_t*>(lds + a.lds_nw + xpos(c)) = nv[p];
        float s2 = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float lo = act_to_f32<DT>((uint16_t)(xv[p][j] & 0xffffu));
          const float hi = act_to_f32<DT>((uint16_t)(xv[p][j] >> 16));
          s2 += lo * lo;
          s2 += hi * hi;
        }
#pragma unroll
        for (int t2 = 0; t2 < T; ++t2) sq[t2] += t2 == tk ? s2 : 0.f;
      }
    }
  }
  if (norm) {
#pragma unroll
    for (int tk = 0; tk < T; ++tk) {
      const float w = wave_sum64(sq[tk]);
      if (lane == 0) nsum[wave * T + tk] = w;
    }
  }
  // every wave's LDS stores are done before any wave reads them: wait for
  // LDS only (a full __syncthreads would also wait for the weights in flight)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);    // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // the reference's post_attention_layernorm (tinyinfer/csrc/rmsnorm.cu:10-54):
  // inv = rsqrt(sum / K + eps), the same in every wave and workgroup
  float inv[T];
#pragma unroll
  for (int tk = 0; tk < T; ++tk) {
    inv[tk] = 1.f;
    if (norm) {
      float tot = 0.f;
#pragma unroll
      for (int w = 0; w < kRW; ++w) tot += nsum[w * T + tk];
      inv[tk] = rsqrtf(tot / (float)a.K + a.eps);
    }
  }

  // lane l's activations: block 64c + l of each of its chunks c = cb + q,
  // zero past K; with a norm, x <- round(w * x * inv).
  u32x4_t xr[T][UC][4], xl[T][UC][4];
#pragma unroll
  for (int tk = 0; tk < T; ++tk) {
#pragma unroll
    for (int q = 0; q < UC; ++q) {
      const int blk = (cb + q) * kChunkBlocks + lane;
      const bool valid = q < ncs && blk < a.nblk;
      const int bc = valid ? blk : 0;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        u32x4_t v = *reinterpret_cast<const u32x4_t*>(lds + tk * 2 * a.K + xpos(4 * bc + t));
        if (norm) {
          const u32x4_t g = *reinterpret_cast<const u32x4_t*>(lds + a.lds_nw + xpos(4 * bc + t));
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float lo =
                act_to_f32<DT>((uint16_t)(g[j] & 0xffffu)) * act_to_f32<DT>((uint16_t)(v[j] & 0xffffu)) * inv[tk];
            const float hi = act_to_f32<DT>((uint16_t)(g[j] >> 16)) * act_to_f32<DT>((uint16_t)(v[j] >> 16)) * inv[tk];
            v[j] = (uint32_t)f32_to_act<DT>(lo) | ((uint32_t)f32_to_act<DT>(hi) << 16);
          }
        }
        if (!valid) v = u32x4_t{0u, 0u, 0u, 0u};
        xr[tk][q][t] = v;
        xl[tk][q][t] = v;
      }
    }
  }

  float* outs = reinterpret_cast<float*>(lds + a.lds_out);   // [rows_max][kRW][T][2] partial sums
  // multiply row j from buffer b; with ISSUE, then load row j + 2 into b
  auto step = [&](RowBuf<UC, GATEUP>& b, int j, auto issue_tag) {
    f32x4_t acc[2][T][kCh];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int tk = 0; tk < T; ++tk)
#pragma unroll
        for (int c = 0; c < kCh; ++c) acc[m][tk][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    bool ok = true;
#pragma unroll
    for (int k = 0; k < RowBuf<UC, GATEUP>::kMats * UC; ++k)
      ok = ok && (DT == kBF16 ? e8m0_fast_ok(scale_byte(b.s[k])) : e8m0_f16_ok(scale_byte(b.s[k])));
    if (wave_all(ok)) {
      if (a.full && ncs == UC) mma_row<DT, UC, GATEUP, true, true, T>(a, cb, ncs, b, xr, xl, acc);
      else mma_row<DT, UC, GATEUP, true, false, T>(a, cb, ncs, b, xr, xl, acc);
    } else {
      mma_row<DT, UC, GATEUP, false, false, T>(a, cb, ncs, b, xr, xl, acc);
    }
    if constexpr (decltype(issue_tag)::value) issue_row<UC, GATEUP>(a, row_of(j + 2), cb, ncs, b);
    auto chains = [&](int m, int tk) {
      f32x4_t c = acc[m][tk][0];
#pragma unroll
      for (int i = 1; i < kCh; ++i) c += acc[m][tk][i];
      return c;
    };
#pragma unroll
    for (int tk = 0; tk < T; ++tk) {
      const float y0 = diag_sum(chains(0, tk));
      float y1 = 0.f;
      if constexpr (GATEUP) y1 = diag_sum(chains(1, tk));
      if (lane == 0) *reinterpret_cast<f32x2_t*>(outs + 2 * ((j * kRW + wave) * T + tk)) = f32x2_t{y0, y1};
    }
  };
  constexpr std::true_type kIssue{};
  constexpr std::false_type kLast{};
  // Every load issued is a row the wave multiplies: the loop runs while rows
  // j + 2 and j + 3 exist, and the last two or three rows are peeled off into
  // straight-line tails.  (Loads past the end would cost their bytes and one
  // more memory latency before the wave can end; an issue under a condition
  // inside the loop would make the compiler drain the load queue at every
  // step.  A wave with one row still loads a second, unused one.)
  int j = 0;
  for (; j + 3 < rows; j += 2) {
    step(b0, j, kIssue);
    step(b1, j + 1, kIssue);
  }
  const int left = rows - j;
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

  // the rows' partial sums, staged in LDS (a global store inside the stream
  // would make the load-queue accounting path-dependent): the S parts of a
  // row added in order, then the epilogue; 8 / S consecutive rows per j
  __syncthreads();
  for (int i = threadIdx.x; i < a.rows_max * (kRW / S) * T; i += kRThreads) {
    const int tk = i % T, i2 = i / T;
    const int jj = i2 / (kRW / S), sl = i2 - jj * (kRW / S);
    const int64_t row = (int64_t)blockIdx.x * (kRW / S) + sl + (int64_t)jj * nslots;
    if (row < a.R) {
      float y0 = 0.f, y1 = 0.f;
#pragma unroll
      for (int p = 0; p < S; ++p) {
        const f32x2_t v = *reinterpret_cast<const f32x2_t*>(outs + 2 * ((jj * kRW + sl * S + p) * T + tk));
        y0 += v[0];
        y1 += v[1];
      }
      const float v = GATEUP ? silu_f32(y0) * y1 : y0;
      const int64_t o = (int64_t)tk * a.R + row;
      a.out[o] = with_residual<DT>(f32_to_act<DT>(v), a.res, o);
    }
  }
  if (norm && blockIdx.x == 0 && wave < S && a.xn) {
#pragma unroll
    for (int tk = 0; tk < T; ++tk) {
#pragma unroll
      for (int q = 0; q < UC; ++q) {
        const int blk = (cb + q) * kChunkBlocks + lane;
        if (q < ncs && blk < a.nblk) {
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const u32x4_t v = xr[tk][q][t];
            *reinterpret_cast<u32x4_t*>(a.xn + (int64_t)tk * a.K + 32 * blk + 8 * t) = v;
          }
        }
      }
    }
  }
}

int row_cus() { return device_info().cus; }

bool aligned16_ptr(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }


// Waves per row S and chunks per wave UC for a stage: S in {1, 2, 4} (gate_up
// 1, 2) so that the largest share fits the VGPR budget (gate_up 4 chunks: two
// matrices in flight; down 6; fp16 2 and 3, whose kernels also hold the
// exact hi + lo form)
// and, for down, holds at most 3 chunks where possible; or the S that
// TINYINFER_ROW_SPLIT_GATEUP / _DOWN names, if that fits.
bool row_plan(int64_t M, int64_t K, int64_t R, bool gateup, bool norm, int dtype, RowArgs& a, int& grid,
              int64_t& lds, int& S, int& uc) {
  const int cus = row_cus();
  // K % 128: scale rows start dword-aligned
  if (cus < 1 || K < 128 || K % 128 != 0 || K > (1 << 20) || R < 1 || R > (1 << 24)) return false;
  if (M < 1 || M > 2 || (M == 2 && dtype != kBF16)) return false;
  // two tokens double the multiply per row: gate_up (two matrices) measured
  // 13.06 us on these kernels against 12.82 on the 8-row stream kernel at 8B;
  // down 7.76 against 9.13
  if (M == 2 && gateup) return false;
  const int nc = (int)((K + kChunkK - 1) / kChunkK);
  // chunks per wave: activations of every chunk and token stay in VGPRs
  const int ucmax = dtype != kBF16 ? (gateup ? 2 : 3) : M == 2 ? (gateup ? 2 : 3) : gateup ? 4 : kMaxUC;
  const int smax = gateup ? 2 : 4;
  S = 0;
  const int want = option(gateup ? kOptRowSplitGateUp : kOptRowSplitDown);
  if (want && want <= smax && (nc + want - 1) / want <= ucmax && want <= nc) S = want;
  // down: at most 3 chunks per wave where the split allows it (8B down, 6
  // chunks: 3 + 3 measured 6.36 us against 7.38 us whole and 7.22 us over four
  // waves); gate_up: whole rows (3 + 3 split measured no faster)
  const int ucpref = gateup ? ucmax : std::min(3, ucmax);
  for (int s = 1; S == 0 && s <= smax; s *= 2)
    if ((nc + s - 1) / s <= ucpref) S = s;
  for (int s = 1; S == 0 && s <= smax; s *= 2)
    if ((nc + s - 1) / s <= ucmax) S = s;
  if (S == 0 || S > nc) return false;
  uc = (nc + S - 1) / S;
  if (uc > ucmax) return false;              // no kernel instantiated for it
  grid = (int)std::min<int64_t>(cus, (R * S + kRW - 1) / kRW);
  const int64_t nslots = (int64_t)grid * (kRW / S);
  a.K = (int)K;
  a.R = (int)R;
  a.nc = nc;
  a.nblk = (int)(K / kBlock);
  a.full = K % kChunkK == 0;
  a.rows_max = (int)((R + nslots - 1) / nslots);
  int64_t off = M * K * 2;                   // x
  a.lds_nw = (int)off;
  if (gateup && norm) off += K * 2;          // norm weight
  off = (off + 15) & ~int64_t(15);
  a.lds_sum = (int)off;
  off += 4 * kRW * M;
  a.lds_out = (int)off;
  off += 8 * (int64_t)a.rows_max * kRW * M;  // two fp32 partial sums per (row, wave, token)
  lds = (off + 15) & ~int64_t(15);
  return lds <= 160 * 1024;
}

template <int DT, int UC, bool GATEUP, int S, int T>
hipError_t row_launch(const RowArgs& a, int grid, int64_t lds, hipStream_t st) {
  auto k = rowstream_kernel<DT, UC, GATEUP, S, T>;
  if (lds > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
          hipSuccess)
    return hipErrorNotSupported;
  hipLaunchKernelGGL(k, dim3(grid), dim3(kRThreads), (size_t)lds, st, a);
  return hipGetLastError();
}

// The instantiated (UC, S, T): one token: gate_up S = 1, 2 with UC <= 4, down
// S = 1, 2, 4 with UC <= 6 (fp16: gate_up UC <= 2, down UC <= 3); two tokens
// (bf16): down UC <= 3.
template <int DT, bool GATEUP, int S, int T>
hipError_t row_dispatch_s(const RowArgs& a, int uc, int grid, int64_t lds, hipStream_t st) {
  constexpr int kMax = DT != kBF16 ? (GATEUP ? 2 : 3) : T == 2 ? (GATEUP ? 2 : 3) : GATEUP ? 4 : kMaxUC;
  switch (uc) {
    case 1: if constexpr (S == 1 || GATEUP) return row_launch<DT, 1, GATEUP, S, T>(a, grid, lds, st); break;
    case 2: return row_launch<DT, 2, GATEUP, S, T>(a, grid, lds, st);
    case 3: if constexpr (kMax >= 3) return row_launch<DT, 3, GATEUP, S, T>(a, grid, lds, st); break;
    case 4: if constexpr (kMax >= 4) return row_launch<DT, 4, GATEUP, S, T>(a, grid, lds, st); break;
    case 5: if constexpr (kMax >= 5) return row_launch<DT, 5, GATEUP, S, T>(a, grid, lds, st); break;
    case 6: if constexpr (kMax >= 6) return row_launch<DT, 6, GATEUP, S, T>(a, grid, lds, st); break;
    default: break;
  }
  return hipErrorNotSupported;
}

template <int DT, bool GATEUP, int T>
hipError_t row_dispatch(const RowArgs& a, int S, int uc, int grid, int64_t lds, hipStream_t st) {
  if (S == 1) return row_dispatch_s<DT, GATEUP, 1, T>(a, uc, grid, lds, st);
  if (S == 2) return row_dispatch_s<DT, GATEUP, 2, T>(a, uc, grid, lds, st);
  if constexpr (!GATEUP) {
    if (S == 4) return row_dispatch_s<DT, GATEUP, 4, T>(a, uc, grid, lds, st);
  }
  return hipErrorNotSupported;
}

template <bool GATEUP>
hipError_t row_stage(const MlpArgs& m, hipStream_t st) {
  RowArgs a;
  int grid = 0;
  int64_t lds = 0;
  const int64_t K = GATEUP ? m.hidden : m.inter;
  const int64_t R = GATEUP ? m.inter : m.hidden;
  const bool norm = GATEUP && m.norm_w != nullptr;
  int S = 0, uc = 0;
  if (!row_plan(m.n, K, R, GATEUP, norm, m.dtype, a, grid, lds, S, uc)) return hipErrorNotSupported;
  a.x = static_cast<const uint16_t*>(GATEUP ? m.x : m.tmp);
  a.w0 = GATEUP ? m.gate : m.down;
  a.s0 = GATEUP ? m.gate_scale : m.down_scale;
  a.w1 = GATEUP ? m.up : a.w0;
  a.s1 = GATEUP ? m.up_scale : a.s0;
  a.out = static_cast<uint16_t*>(GATEUP ? m.tmp : m.out);
  a.res = GATEUP ? nullptr : static_cast<const uint16_t*>(m.residual);
  a.norm_w = norm ? static_cast<const uint16_t*>(m.norm_w) : nullptr;
  a.eps = m.eps;
  a.xn = norm ? static_cast<uint16_t*>(m.xn) : nullptr;
  if (m.dtype != kBF16) return row_dispatch<kF16, GATEUP, 1>(a, S, uc, grid, lds, st);
  if constexpr (!GATEUP) {
    if (m.n == 2) return row_dispatch<kBF16, GATEUP, 2>(a, S, uc, grid, lds, st);
  }
  return row_dispatch<kBF16, GATEUP, 1>(a, S, uc, grid, lds, st);
}

}  // namespace

bool rowstream_enabled() { return option(kOptRowstream) != 0; }

bool rowstream_supported(const MlpArgs& m, int stage) {
  if (m.n < 1 || m.n > 2 || (m.dtype != kBF16 && m.dtype != kF16)) return false;
  RowArgs a;
  int grid = 0, S = 0, uc = 0;
  int64_t lds = 0;
  if ((stage & kStageGateUp) &&
      !row_plan(m.n, m.hidden, m.inter, true, m.norm_w != nullptr, m.dtype, a, grid, lds, S, uc))
    return false;
  if ((stage & kStageDown) && !row_plan(m.n, m.inter, m.hidden, false, false, m.dtype, a, grid, lds, S, uc))
    return false;
  // 16-byte loads of activations, weights and the norm weight; 16-byte xn stores
  const void* p16[] = {m.x, m.gate, m.up, m.down, m.tmp, m.norm_w, m.xn};
  for (const void* p : p16)
    if (p && !aligned16_ptr(p)) return false;
  return true;
}

hipError_t launch_rowstream_mlp(const MlpArgs& m, int stage, hipStream_t st) {
  if (stage & kStageGateUp) {
    const hipError_t e = row_stage<true>(m, st);
    if (e != hipSuccess) return e;
  }
  if (stage & kStageDown) return row_stage<false>(m, st);
  return hipSuccess;
}

}  // namespace tinyinfer
