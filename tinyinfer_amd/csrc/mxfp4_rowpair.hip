// Row-pair streaming MXFP4 GEMV for 2..4 tokens: one kernel per MLP
// stage, the same contract as the row-streaming kernel (mxfp4_rowstream.hip)
// and the 8-row stream kernel (mxfp4_stream.hip) for the reference's
// per-token GEMV kernels mlp_stage1_mxfp4 / mlp_stage2_mxfp4
// (tinyinfer/csrc/mlp_fp4.cu:79-142, 365-426).
//
// Load layout: every weight load instruction reads 512 contiguous bytes of
// each of two rows (lane l: row l & 1 of the pair, 32-element block
// 32c + (l >> 1) of the pair's chunk c; a chunk is 1024 K elements).  Loads
// that span one or two rows stream at the speed of a plain read (measured
// 9.4-9.5 us against 9.2-9.3 for one row and 10.2-10.4 for eight, for the
// 8B gate_up bytes), and two rows per load let one MFMA serve two tokens.
//
// MFMA mapping (v_mfma_f32_16x16x32_bf16): A = the lane's 8 dequantized
// weights, B = the same K elements of token (l & 1) (+ 2 in the second pass).
// A row i is weight row i & 1 at block (i >> 1) + 8g, B column n is token
// n & 1 at block (n >> 1) + 8g, so the 2 x 2 diagonal blocks
// C[2b + r][2b + t] (b = 0..7) hold row r x token t over the 32 blocks of the
// chunk, summed over b.  One pass covers two tokens; four tokens take two.
//
// The rest follows the row kernel: a wave owns whole row pairs (or an equal
// share of their chunks, S waves per pair), scale bytes loaded as dwords next
// to the weights, x staged once through LDS and copied into VGPRs, two pairs
// in flight per wave, the last two or three peeled into straight-line tails,
// partial sums added in order in the end-of-kernel epilogue.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "mxfp4_common.hpp"
#include "mxfp4_launch.hpp"

namespace tinyinfer {

namespace {

constexpr int kPW = 8;                 // waves per workgroup
constexpr int kPThreads = kPW * 64;
constexpr int kPairBlocks = 32;        // 32-element blocks per row per load (512 B)
constexpr int kPairChunkK = kPairBlocks * kBlock;

struct PairArgs {
  const uint16_t* x;       // [M, K] activations
  const uint8_t* w0;       // [R, K/2] gate (or down)
  const uint8_t* s0;       // [R, K/32]
  const uint8_t* w1;       // [R, K/2] up (gate_up only; else = w0)
  const uint8_t* s1;
  uint16_t* out;           // [M, R]
  const uint16_t* res;     // down only: residual [M, R] added to out, or null
  const uint16_t* norm_w;  // gate_up only: RMSNorm weight [K], or null
  float eps;
  uint16_t* xn;            // with norm_w: the normalized x [M, K]
  int M, K, R;
  int nc;                  // chunks per row pair, ceil(K / 1024)
  int nblk;                // K / 32
  int full;                // every chunk has all 32 blocks (K % 1024 == 0)
  int rows_max;            // row pairs of the busiest wave
  int lds_nw, lds_sum, lds_out;
};

template <int UC, bool GATEUP>
struct PairBuf {
  static constexpr int kMats = GATEUP ? 2 : 1;
  u32x4_t w[kMats * UC];
  uint32_t s[kMats * UC];   // the aligned dword holding the lane's scale byte
};

__device__ __forceinline__ uint32_t pair_scale_byte(uint32_t dw) {
  // the lane's block is 32c + (lane >> 1): byte (lane >> 1) & 3 of its dword
  return (dw >> (8 * ((threadIdx.x >> 1) & 3))) & 0xffu;
}

// Loads of row pair `pr` (rows 2 pr, 2 pr + 1), chunks cb + q (q < ncs; the
// slots past the range repeat the last chunk and are not used).  Scale
// dwords first.
template <int UC, bool GATEUP>
__device__ __forceinline__ void issue_pair(const PairArgs& a, int64_t pr, int cb, int ncs, PairBuf<UC, GATEUP>& b) {
  constexpr int kMats = GATEUP ? 2 : 1;
  const int lane = threadIdx.x & 63;
  const int64_t row = 2 * pr + (lane & 1);
  const int bl = lane >> 1;
#pragma unroll
  for (int m = 0; m < kMats; ++m) {
    const uint8_t* sp = (m ? a.s1 : a.s0) + row * a.nblk;
#pragma unroll
    for (int q = 0; q < UC; ++q) {
      const int c = cb + (q < ncs ? q : ncs - 1);
      const int blk = c * kPairBlocks + bl;
      b.s[m * UC + q] = *reinterpret_cast<const uint32_t*>(sp + ((blk < a.nblk ? blk : a.nblk - 1) & ~3));
    }
  }
#pragma unroll
  for (int m = 0; m < kMats; ++m) {
    const uint8_t* wp = (m ? a.w1 : a.w0) + row * (a.K / 2);
#pragma unroll
    for (int q = 0; q < UC; ++q) {
      const int c = cb + (q < ncs ? q : ncs - 1);
      const int blk = c * kPairBlocks + bl;
      b.w[m * UC + q] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4_t*>(wp + 16 * (int64_t)(blk < a.nblk ? blk : a.nblk - 1)));
    }
  }
  __builtin_amdgcn_sched_barrier(0);
}

// P passes (tokens 2p + (lane & 1)) over each dequantized operand; 4 / P
// accumulator chains per (matrix, pass).  bf16: FAST when every scale byte is
// in the hardware bf16 conversion's exact range.  fp16 (x held as fp16): FAST
// when every scale byte is e8m0_f16_ok, the weights converted to fp16 on
// fp16 MFMAs; otherwise the exact bf16 weights against x's exact bf16 hi and
// lo parts, two MFMAs.
template <int UC, bool GATEUP, bool FAST, bool FULL, int P, int DT>
__device__ __forceinline__ void mma_pair(const PairArgs& a, int cb, int ncs, const PairBuf<UC, GATEUP>& b,
                                         const u32x4_t (&xr)[P][UC][4], f32x4_t (&acc)[2][P][4 / P]) {
  constexpr int kMats = GATEUP ? 2 : 1;
  constexpr int kCh = 4 / P;
  const int bl = (threadIdx.x & 63) >> 1;
#pragma unroll
  for (int m = 0; m < kMats; ++m) {
#pragma unroll
    for (int q = 0; q < UC; ++q) {
      const bool valid = FULL || (q < ncs && (cb + q) * kPairBlocks + bl < a.nblk);
      const uint32_t sb = valid ? pair_scale_byte(b.s[m * UC + q]) : 127u;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t wq = valid ? b.w[m * UC + q][t] : 0u;
        const u32x4_t wa = !FAST ? dq8_bf16_exact(wq, sb) : DT == kBF16 ? dq8_bf16_fast(wq, sb) : dq8_f16_fast(wq, sb);
#pragma unroll
        for (int p = 0; p < P; ++p) {
          f32x4_t& c = acc[m][p][t % kCh];
          if constexpr (DT == kBF16) {
            c = mfma16x16x32(wa, xr[p][q][t], c);
          } else if constexpr (FAST) {
            c = mfma16x16x32_f16(wa, xr[p][q][t], c);
          } else {
            u32x4_t xh, xl;
            f16x8_split_bf16(xr[p][q][t], xh, xl);
            c = mfma16x16x32(wa, xl, mfma16x16x32(wa, xh, c));
          }
        }
      }
    }
  }
}

// Partial sums of the 2 x 2 diagonal blocks: lane l holds C[4g + v][n]
// (g = l / 16, n = l % 16); C[i][n] is useful when i >> 1 == n >> 1, i.e.
// v = 2d + r with d = (n >> 1) - 2g in {0, 1}, row r, token n & 1.  The
// useful lanes are quad g of row g; one quad DPP add folds d, leaving row r x
// token t of blocks {2g, 2g + 1} (mod 8 per 32-block group) in lane 20g + t.
// Those eight lanes store (r = 0, r = 1) to LDS as [t][g][r]; the epilogue
// adds the four g in order.
__device__ __forceinline__ void pair_partials(const f32x4_t& c, float* blk) {
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const bool d0 = (n & 2) == 0;
  float v0 = d0 ? c[0] : c[2];
  float v1 = d0 ? c[1] : c[3];
  v0 = dpp_add<0x4e>(v0);     // quad_perm [2,3,0,1]: + the lane with the other d
  v1 = dpp_add<0x4e>(v1);
  if ((n >> 2) == g && d0) {
    const int t = n & 1;
    *reinterpret_cast<float2*>(blk + (t * 4 + g) * 2) = make_float2(v0, v1);
  }
}

template <int UC, bool GATEUP, int S, int P, int DT>
__global__ __launch_bounds__(kPThreads, 1) void rowpair_kernel(PairArgs a) {
  static_assert(kPW % S == 0, "the waves sharing a pair are in one workgroup");
  constexpr int kT = 2 * P;                // token slots
  constexpr int kCh = 4 / P;
  // 16-byte x chunks per thread: M K / 8 <= kT * 128 UC S
  constexpr int kXPre = (kT * 128 * UC * S + kPThreads - 1) / kPThreads;
  extern __shared__ __align__(16) uint8_t lds[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int npairs = a.R / 2;
  const int nslots = gridDim.x * (kPW / S);
  const int slot = blockIdx.x * (kPW / S) + wave / S;
  const int sp = wave % S;
  const int cb = sp * a.nc / S;
  const int ncs = (sp + 1) * a.nc / S - cb;
  const int rows = slot < npairs ? (npairs - slot + nslots - 1) / nslots : 0;

  // prologue loads before the first weights: x [M, K], the norm weight
  const int nxr = a.K / 8;
  const int nxc = a.M * nxr;
  const bool norm = GATEUP && a.norm_w != nullptr;
  u32x4_t xv[kXPre], nv[kXPre];
#pragma unroll
  for (int p = 0; p < kXPre; ++p) {
    const int c = threadIdx.x + p * kPThreads;
    xv[p] = *reinterpret_cast<const u32x4_t*>(a.x + 8 * (c < nxc ? c : nxc - 1));
  }
  if (norm) {
#pragma unroll
    for (int p = 0; p < kXPre; ++p) {
      const int c = threadIdx.x + p * kPThreads;
      nv[p] = *reinterpret_cast<const u32x4_t*>(a.norm_w + 8 * (c < nxr ? c : nxr - 1));
    }
  }

  PairBuf<UC, GATEUP> b0, b1;
  auto pair_of = [&](int j) {
    return rows > 0 ? (int64_t)slot + (int64_t)(j < rows ? j : rows - 1) * nslots : (int64_t)(slot % npairs);
  };
  issue_pair<UC, GATEUP>(a, pair_of(0), cb, ncs, b0);
  issue_pair<UC, GATEUP>(a, pair_of(1), cb, ncs, b1);

  // x (and the norm weight) into LDS, slice-major per token row (2K bytes a
  // row); per-token sums of squares for the norm
  const int plane = a.K / 2;
  auto xpos = [&](int c) { return (c & 3) * plane + 16 * (c >> 2); };
  float* nsum = reinterpret_cast<float*>(lds + a.lds_sum);   // [kPW][kT]
  float sq[kT];
#pragma unroll
  for (int tk = 0; tk < kT; ++tk) sq[tk] = 0.f;
#pragma unroll
  for (int p = 0; p < kXPre; ++p) {
    const int c = threadIdx.x + p * kPThreads;
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
        for (int t2 = 0; t2 < kT; ++t2) sq[t2] += t2 == tk ? s2 : 0.f;
      }
    }
  }
  if (norm) {
#pragma unroll
    for (int tk = 0; tk < kT; ++tk) {
      const float w = wave_sum64(sq[tk]);
      if (lane == 0) nsum[wave * kT + tk] = w;
    }
  }
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);    // lgkmcnt(0): LDS only, not the weights in flight
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // the reference's post_attention_layernorm (tinyinfer/csrc/rmsnorm.cu:10-54)
  float inv[kT];
#pragma unroll
  for (int tk = 0; tk < kT; ++tk) {
    inv[tk] = 1.f;
    if (norm) {
      float tot = 0.f;
#pragma unroll
      for (int w = 0; w < kPW; ++w) tot += nsum[w * kT + tk];
      inv[tk] = rsqrtf(tot / (float)a.K + a.eps);
    }
  }

  // lane l's activations: token 2p + (l & 1), block 32c + (l >> 1) of each of
  // its chunks; zero past K and for token slots >= M
  u32x4_t xr[P][UC][4];
#pragma unroll
  for (int p = 0; p < P; ++p) {
#pragma unroll
    for (int q = 0; q < UC; ++q) {
      const int tk = 2 * p + (lane & 1);
      const int blk = (cb + q) * kPairBlocks + (lane >> 1);
      const bool valid = q < ncs && blk < a.nblk && tk < a.M;
      const int bc = valid ? blk : 0;
      const int tr = tk < a.M ? tk : 0;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        u32x4_t v = *reinterpret_cast<const u32x4_t*>(lds + tr * 2 * a.K + xpos(4 * bc + t));
        if (norm) {
          float iv = inv[0];
#pragma unroll
          for (int t2 = 1; t2 < kT; ++t2) iv = tr == t2 ? inv[t2] : iv;
          const u32x4_t g = *reinterpret_cast<const u32x4_t*>(lds + a.lds_nw + xpos(4 * bc + t));
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float lo =
                act_to_f32<DT>((uint16_t)(g[j] & 0xffffu)) * act_to_f32<DT>((uint16_t)(v[j] & 0xffffu)) * iv;
            const float hi = act_to_f32<DT>((uint16_t)(g[j] >> 16)) * act_to_f32<DT>((uint16_t)(v[j] >> 16)) * iv;
            v[j] = (uint32_t)f32_to_act<DT>(lo) | ((uint32_t)f32_to_act<DT>(hi) << 16);
          }
        }
        xr[p][q][t] = valid ? v : u32x4_t{0u, 0u, 0u, 0u};
      }
    }
  }

  float* outs = reinterpret_cast<float*>(lds + a.lds_out);   // [rows_max][kPW][P][2 m][2 t][4 g][2 r]
  auto step = [&](PairBuf<UC, GATEUP>& b, int j, auto issue_tag) {
    f32x4_t acc[2][P][kCh];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int p = 0; p < P; ++p)
#pragma unroll
        for (int c = 0; c < kCh; ++c) acc[m][p][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    bool ok = true;
#pragma unroll
    for (int k = 0; k < PairBuf<UC, GATEUP>::kMats * UC; ++k)
      ok = ok && (DT == kBF16 ? e8m0_fast_ok(pair_scale_byte(b.s[k])) : e8m0_f16_ok(pair_scale_byte(b.s[k])));
    if (wave_all(ok)) {
      if (a.full && ncs == UC) mma_pair<UC, GATEUP, true, true, P, DT>(a, cb, ncs, b, xr, acc);
      else mma_pair<UC, GATEUP, true, false, P, DT>(a, cb, ncs, b, xr, acc);
    } else {
      mma_pair<UC, GATEUP, false, false, P, DT>(a, cb, ncs, b, xr, acc);
    }
    if constexpr (decltype(issue_tag)::value) issue_pair<UC, GATEUP>(a, pair_of(j + 2), cb, ncs, b);
#pragma unroll
    for (int p = 0; p < P; ++p) {
#pragma unroll
      for (int m = 0; m < PairBuf<UC, GATEUP>::kMats; ++m) {
        f32x4_t c = acc[m][p][0];
#pragma unroll
        for (int i = 1; i < kCh; ++i) c += acc[m][p][i];
        pair_partials(c, outs + ((j * kPW + wave) * P + p) * 32 + m * 16);
      }
    }
  };
  constexpr std::true_type kIssue{};
  constexpr std::false_type kLast{};
  // every load issued is a pair the wave multiplies (tails peeled; an issue
  // under a condition inside the loop would drain the load queue each step)
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

  // partial sums of the S waves of a pair in order, then the epilogue
  __syncthreads();
  for (int i = threadIdx.x; i < a.rows_max * (kPW / S) * P * 4; i += kPThreads) {
    const int e = i & 3, i2 = i >> 2;          // e = (row r, token t)
    const int p = i2 % P, i3 = i2 / P;
    const int jj = i3 / (kPW / S), sl = i3 - jj * (kPW / S);
    const int64_t pr = (int64_t)blockIdx.x * (kPW / S) + sl + (int64_t)jj * nslots;
    const int r = e >> 1, t = e & 1;
    const int tk = 2 * p + t;
    if (pr < npairs && tk < a.M) {
      float y0 = 0.f, y1 = 0.f;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const float* o = outs + ((jj * kPW + sl * S + s) * P + p) * 32 + t * 8 + r;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          y0 += o[2 * g];
          if (GATEUP) y1 += o[16 + 2 * g];
        }
      }
      const float v = GATEUP ? silu_f32(y0) * y1 : y0;
      const int64_t idx = (int64_t)tk * a.R + 2 * pr + r;
      a.out[idx] = with_residual<DT>(f32_to_act<DT>(v), a.res, idx);
    }
  }
  if (norm && blockIdx.x == 0 && wave < S && a.xn) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int tk = 2 * p + (lane & 1);
#pragma unroll
      for (int q = 0; q < UC; ++q) {
        const int blk = (cb + q) * kPairBlocks + (lane >> 1);
        if (q < ncs && blk < a.nblk && tk < a.M) {
#pragma unroll
          for (int t = 0; t < 4; ++t)
            *reinterpret_cast<u32x4_t*>(a.xn + (int64_t)tk * a.K + 32 * blk + 8 * t) = xr[p][q][t];
        }
      }
    }
  }
}

int pair_cus() { return device_info().cus; }

// Waves per pair S and chunks per wave UC: gate_up whole pairs where the
// chunks fit (4 at one pass, 3 at two), down at most 3 chunks per wave where
// four waves suffice; more waves per pair when there are too few pairs to
// give every CU a workgroup.
bool pair_plan(int64_t M, int64_t K, int64_t R, bool gateup, bool norm, int dtype, PairArgs& a, int& grid,
               int64_t& lds, int& S, int& uc) {
  const int cus = pair_cus();
  if (cus < 1 || M < 2 || M > 4 || K < 128 || K % 128 != 0 || K > (1 << 20) || R < 2 || R % 2 != 0 ||
      R > (1 << 24))
    return false;
  const int P = (int)((M + 1) / 2);
  const int nc = (int)((K + kPairChunkK - 1) / kPairChunkK);
  // fp16 kernels also hold the exact hi + lo form: fewer chunks per wave
  const int ucmax = dtype != kBF16 ? (gateup ? (P == 1 ? 2 : 1) : (P == 1 ? 3 : 2))
                                   : gateup ? (P == 1 ? 4 : 3) : (P == 1 ? 6 : 4);
  const int ucpref = gateup ? ucmax : std::min(3, ucmax);
  S = 0;
  for (int s = 1; S == 0 && s <= 4; s *= 2)
    if ((nc + s - 1) / s <= ucpref && s <= nc) S = s;
  for (int s = 1; S == 0 && s <= 4; s *= 2)
    if ((nc + s - 1) / s <= ucmax && s <= nc) S = s;
  if (S == 0) return false;
  // two-pass gate_up split over waves for its registers measured slower than
  // the 8-row stream kernel (8B: 12.7-12.9 against 12.6 us at 3-4 tokens)
  if (gateup && P == 2 && S > 1) return false;
  const int64_t npairs = R / 2;
  // too few pairs to give every CU a workgroup: more waves per pair
  while (S < 4 && 2 * S <= nc && (npairs * S + kPW - 1) / kPW < cus) S *= 2;
  uc = (nc + S - 1) / S;
  if (uc > ucmax) return false;              // no kernel instantiated for it
  grid = (int)std::min<int64_t>(cus, (npairs * S + kPW - 1) / kPW);
  const int64_t nslots = (int64_t)grid * (kPW / S);
  a.M = (int)M;
  a.K = (int)K;
  a.R = (int)R;
  a.nc = nc;
  a.nblk = (int)(K / kBlock);
  a.full = K % kPairChunkK == 0;
  a.rows_max = (int)((npairs + nslots - 1) / nslots);
  int64_t off = M * K * 2;                   // x
  a.lds_nw = (int)off;
  if (gateup && norm) off += K * 2;
  off = (off + 15) & ~int64_t(15);
  a.lds_sum = (int)off;
  off += 4 * kPW * 2 * P;
  a.lds_out = (int)off;
  off += 4 * (int64_t)a.rows_max * kPW * P * 32;
  lds = (off + 15) & ~int64_t(15);
  return lds <= 160 * 1024;
}

template <int UC, bool GATEUP, int S, int P, int DT>
hipError_t pair_launch(const PairArgs& a, int grid, int64_t lds, hipStream_t st) {
  auto k = rowpair_kernel<UC, GATEUP, S, P, DT>;
  if (lds > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
          hipSuccess)
    return hipErrorNotSupported;
  hipLaunchKernelGGL(k, dim3(grid), dim3(kPThreads), (size_t)lds, st, a);
  return hipGetLastError();
}

template <bool GATEUP, int S, int P, int DT>
hipError_t pair_dispatch_s(const PairArgs& a, int uc, int grid, int64_t lds, hipStream_t st) {
  constexpr int kMax = DT != kBF16 ? (GATEUP ? (P == 1 ? 2 : 1) : (P == 1 ? 3 : 2))
                                   : GATEUP ? (P == 1 ? 4 : 3) : (P == 1 ? 6 : 4);
  switch (uc) {
    case 1: return pair_launch<1, GATEUP, S, P, DT>(a, grid, lds, st);
    case 2: if constexpr (kMax >= 2) return pair_launch<2, GATEUP, S, P, DT>(a, grid, lds, st); break;
    case 3: if constexpr (kMax >= 3) return pair_launch<3, GATEUP, S, P, DT>(a, grid, lds, st); break;
    case 4: if constexpr (kMax >= 4) return pair_launch<4, GATEUP, S, P, DT>(a, grid, lds, st); break;
    case 5: if constexpr (kMax >= 5) return pair_launch<5, GATEUP, S, P, DT>(a, grid, lds, st); break;
    case 6: if constexpr (kMax >= 6) return pair_launch<6, GATEUP, S, P, DT>(a, grid, lds, st); break;
    default: break;
  }
  return hipErrorNotSupported;
}

template <bool GATEUP, int P, int DT>
hipError_t pair_dispatch(const PairArgs& a, int S, int uc, int grid, int64_t lds, hipStream_t st) {
  if (S == 1) return pair_dispatch_s<GATEUP, 1, P, DT>(a, uc, grid, lds, st);
  if (S == 2) return pair_dispatch_s<GATEUP, 2, P, DT>(a, uc, grid, lds, st);
  if (S == 4) return pair_dispatch_s<GATEUP, 4, P, DT>(a, uc, grid, lds, st);
  return hipErrorNotSupported;
}

template <bool GATEUP>
hipError_t pair_stage(const MlpArgs& m, hipStream_t st) {
  PairArgs a;
  int grid = 0, S = 0, uc = 0;
  int64_t lds = 0;
  const int64_t K = GATEUP ? m.hidden : m.inter;
  const int64_t R = GATEUP ? m.inter : m.hidden;
  const bool norm = GATEUP && m.norm_w != nullptr;
  if ((m.dtype != kBF16 && m.dtype != kF16) || !pair_plan(m.n, K, R, GATEUP, norm, m.dtype, a, grid, lds, S, uc))
    return hipErrorNotSupported;
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
  if (m.dtype == kF16)
    return m.n <= 2 ? pair_dispatch<GATEUP, 1, kF16>(a, S, uc, grid, lds, st)
                    : pair_dispatch<GATEUP, 2, kF16>(a, S, uc, grid, lds, st);
  return m.n <= 2 ? pair_dispatch<GATEUP, 1, kBF16>(a, S, uc, grid, lds, st)
                  : pair_dispatch<GATEUP, 2, kBF16>(a, S, uc, grid, lds, st);
}

bool aligned16_pair(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

bool rowpair_enabled() { return option(kOptRowpair) != 0; }

bool rowpair_supported(const MlpArgs& m, int stage) {
  if (m.dtype != kBF16 && m.dtype != kF16) return false;
  PairArgs a;
  int grid = 0, S = 0, uc = 0;
  int64_t lds = 0;
  if ((stage & kStageGateUp) &&
      !pair_plan(m.n, m.hidden, m.inter, true, m.norm_w != nullptr, m.dtype, a, grid, lds, S, uc))
    return false;
  if ((stage & kStageDown) && !pair_plan(m.n, m.inter, m.hidden, false, false, m.dtype, a, grid, lds, S, uc))
    return false;
  const void* p16[] = {m.x, m.gate, m.up, m.down, m.tmp, m.norm_w, m.xn};
  for (const void* p : p16)
    if (p && !aligned16_pair(p)) return false;
  // dword scale loads
  const void* p4[] = {m.gate_scale, m.up_scale, m.down_scale};
  for (const void* p : p4)
    if (p && (reinterpret_cast<uintptr_t>(p) & 3u) != 0) return false;
  return true;
}

hipError_t launch_rowpair_mlp(const MlpArgs& m, int stage, hipStream_t st) {
  if (stage & kStageGateUp) {
    const hipError_t e = pair_stage<true>(m, st);
    if (e != hipSuccess) return e;
  }
  if (stage & kStageDown) return pair_stage<false>(m, st);
  return hipSuccess;
}

}  // namespace tinyinfer
