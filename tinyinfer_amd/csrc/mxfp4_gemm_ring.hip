// Tiled MXFP4 MLP GEMM for prefill (bf16 or fp16 activations, K a multiple of 512):
// a three-stage LDS ring fed by direct-to-LDS loads.
//
// Replaces the reference's per-token GEMV kernels mlp_stage1_mxfp4 /
// mlp_stage2_mxfp4 (tinyinfer/csrc/mlp_fp4.cu:79-142, 365-426) where they are
// compute-bound.  C = W X^T (weight rows x tokens) on v_mfma_f32_32x32x16_bf16
// with fp32 accumulation; the e2m1 weights are dequantized to bf16 in
// registers right before the MFMAs that use them.
//
// Workgroup: 512 threads (8 waves, 4 row groups x 2 token halves), one per
// CU; a tile is 256 weight rows x BM tokens (gate_up: 128 output rows of gate
// and of up, so the SiLU(g)*u epilogue has both in the same lanes; down: 256
// output rows).  Per K step of 64:
//   X  [BM tokens][64] bf16 = 128 B per token row,
//   W  [256 rows][32 B packed],
// loaded with global_load_lds_dwordx4 (each instruction writes 64 x 16 B
// contiguously in LDS), so no VGPRs hold loads in flight and two stages can
// be in flight while the third is multiplied.  Rows are XOR-swizzled in
// 16-byte units on the global side (the LDS side of the load is fixed), so
// that the MFMA operand reads (32 rows at one K offset) fall in distinct
// banks: X chunk c of token row t sits at slot c ^ ((t >> 1) & 7), W half h of
// row r at slot h ^ ((r >> 3) & 1).
// The e8m0 bytes come 16 per row (8 K steps) with one extra load per wave
// every 8 steps, double-buffered in LDS.
//
// Pipeline: stage k+2 is issued right after the barrier of step k (which
// also proves stage k-1's buffer free), and each wave waits for its own
// loads of stage k before that barrier with an explicit vmcnt.  The barrier
// is a bare s_barrier: a __syncthreads fence would wait for every load in
// flight, which the ring exists to avoid.
//
// Operand K order: in MFMA k-step s (0..3), lane half j (lane / 32) supplies
// the 8 K elements 32j + 8s .. 32j + 8s + 7 of the step, for W and X alike
// (a permutation of K shared by both operands leaves each dot product
// unchanged).  A lane's W bytes for the step are then one 16-byte run under
// one scale byte, and its X bytes one 64-byte run.
#include <mutex>
#include <type_traits>
#include <utility>

#include "mxfp4_common.hpp"
#include "mxfp4_launch.hpp"

namespace tinyinfer {

namespace {

typedef __attribute__((address_space(3))) uint8_t lds_u8_t;

constexpr int kBK = 64;           // K per step
constexpr int kWRows = 256;       // weight rows per tile
constexpr int kWBytes = kWRows * 32;      // packed W per stage
constexpr int kSBlock = kWRows * 16;      // scale bytes per 8-step block
constexpr int kStages = 3;

template <int BM, int NW>
struct RingCfg {
  static constexpr int kXBytes = BM * 2 * kBK;                 // X per stage
  static constexpr int kStage = kXBytes + kWBytes;
  static constexpr int kLds = kStages * kStage + 2 * kSBlock;
  static constexpr int kXInst = BM / 8 / NW;                   // X loads per wave per stage
  static constexpr int kWInst = 8 / NW;                        // W loads per wave per stage
  static constexpr int kSRows = kWRows / NW;                   // scale rows per wave (one per lane)
  static_assert(kXInst >= 1 && kXInst * 8 * NW == BM, "token tile must split over the waves");
  static_assert(kWInst >= 1 && kSRows <= 64, "4 or 8 waves");
};

struct RingArgs {
  const uint16_t* x;        // [M, K]
  const uint8_t* w[2];      // [N, K/2] (gate, up) or (down, down)
  const uint8_t* s[2];      // [N, K/32]
  uint16_t* out;            // [M, N]
  int M, N, K;              // N: output rows
  int m_tiles, n_tiles;
  float* ws;                // split K: fp32 partials [ksplit][M][NMAT * tail_n]
  int ksplit;               // K ranges per split tile (1: no split)
  const uint16_t* res;      // down only: residual [M, N] added to out, or null
  int nfull = 0;            // split kernel: tiles [0, nfull) run whole, the rest split
  int tail_row0 = 0;        // first output row of the split tiles (a band of whole weight tiles)
  int tail_n = 0;           // output rows from tail_row0 to N
};

// 64 lanes x 16 bytes from per-lane global addresses to 1 KB of LDS at l
// (wave-uniform), lane i at l + 16 i.  Written as inline asm: the compiler's
// form of this load makes it assume every such load may overwrite every
// other one's LDS bytes, and it then waits for the whole load queue before
// each of them.  Completion is tracked by the explicit vmcnt waits below.
// M0 (the LDS address of the load) is restored afterwards, so code the
// compiler generates around the statement sees it unchanged.
__device__ __forceinline__ void dma16(const void* g, uint8_t* l) {
  const uint32_t loff = (uint32_t)(uintptr_t)(lds_u8_t*)(l);
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(saved)
               : "v"(g), "s"(__builtin_amdgcn_readfirstlane(loff))
               : "memory");
}

// Weight row (matrix, row) of tile row tr (0..255).
template <int NMAT>
__device__ __forceinline__ void tile_row(int tr, int row0, int N, int& mat, int& row) {
  if constexpr (NMAT == 2) {
    mat = tr >> 7;
    row = row0 + (tr & 127);
  } else {
    mat = 0;
    row = row0 + tr;
  }
  row = row < N ? row : N - 1;     // rows past N load row N-1 and are not stored
}

// SPLIT: the grid also splits K into ksplit ranges of whole 8-step blocks
// (the scale staging's granularity); each workgroup writes its fp32 partial
// tile to the workspace, and ring_reduce sums the ranges in a fixed order and
// applies the epilogue.  Used when the tiles alone would leave CUs idle: for
// every tile (nfull = 0), or for the tiles past the last full round of
// workgroups over the CUs (the first nfull workgroups run tiles [0, nfull)
// whole, with the plain epilogue; the split ones are the band of output rows
// from tail_row0, so their partials take ksplit * M * tail_n floats).
// WR: waves along the weight rows (8 / WR along the tokens).  A wave holds
// WB = 8 / WR blocks of 32 weight rows and kTT = BM / 32 / (8 / WR) blocks of
// 32 tokens; fewer, wider weight blocks per wave read less LDS per MFMA (the
// packed weights are a quarter of the bytes of the activations) at the cost
// of more conversions.
// NW: waves per workgroup.  8 waves run one workgroup per CU; 4 waves with
// 128-token tiles fit two workgroups per CU, whose barriers are independent.
// DT: the activation dtype.  fp16 activations take one of two arithmetics,
// chosen once per workgroup before the K loop from the tile's scale bytes
// (a choice inside the loop, around the MFMAs, would keep two copies of the
// accumulators): every byte in e8m0_f16_ok -> the weights converted to fp16
// by the hardware (exact there) against the fp16 activations on fp16 MFMAs;
// otherwise the exact bf16 weights against the activations' exact bf16 hi
// and lo parts, two bf16 MFMAs per product (exact products either way,
// fp32 sums).
template <int NMAT, int BM, bool SPLIT, int WR, int NW, int DT = kBF16>
__global__ __launch_bounds__(NW * 64, 2) void gemm_ring_kernel(RingArgs a) {
  using C = RingCfg<BM, NW>;
  constexpr int WT = NW / WR;                  // waves along the tokens
  constexpr int WB = 8 / WR;                   // weight blocks per wave
  static_assert(WR * WT == NW, "wave grid");
  constexpr int kTT = BM / 32 / WT;            // token blocks per wave
  constexpr int kRowsW = kWRows / WR;          // tile rows per wave (both matrices)
  static_assert(kTT >= 1 && kTT * 32 * WT == BM, "token tile must split over the waves");
  constexpr int kRowsOut = NMAT == 2 ? 128 : 256;   // output rows per tile
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  // ---- tile (XCD-aware: each XCD walks a contiguous range of tiles, token
  // tiles fastest, so the WGs sharing a weight tile run on one L2) -------
  const int nwg = gridDim.x;
  const int wg = blockIdx.x;
  // whole tiles first (workgroups [0, nfull)), then the split ones; each XCD
  // walks a contiguous range of either
  auto xcd_walk = [](int w, int n) { return (n & 7) == 0 ? (w & 7) * (n >> 3) + (w >> 3) : w; };
  const int nfull = SPLIT ? a.nfull : 0;
  const int logical = wg < nfull ? xcd_walk(wg, nfull) : nfull + xcd_walk(wg - nfull, nwg - nfull);
  const bool part = SPLIT && logical >= nfull;          // this workgroup writes partials
  const int tile = part ? nfull + (logical - nfull) / a.ksplit : logical;
  const int ks = part ? (logical - nfull) - (tile - nfull) * a.ksplit : 0;
  const int n_tile = tile / a.m_tiles;
  const int m_tile = tile - n_tile * a.m_tiles;
  const int row0 = n_tile * kRowsOut;
  const int tok0 = m_tile * BM;
  const int M = a.M, N = a.N, K = a.K;
  // K steps [kbeg, kend) of this workgroup
  const int nblk = K / (8 * kBK);
  const int kbeg = part ? 8 * (ks * nblk / a.ksplit) : 0;
  const int kend = part ? 8 * ((ks + 1) * nblk / a.ksplit) : K / kBK;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wr = wave % WR;         // row group
  const int wt = wave / WR;         // token group
  const int l32 = lane & 31;
  const int j = lane >> 5;

  // ---- loads of one stage (this wave's share) ---------------------------
  // X: instruction q covers token rows 8q .. 8q+7 of the tile.
  auto issue_stage = [&](int k) {
    uint8_t* st = smem + ((k - kbeg) % kStages) * C::kStage;
    const int k0 = k * kBK;
#pragma unroll
    for (int i = 0; i < C::kXInst; ++i) {
      const int q = wave + NW * i;
      const int tr = 8 * q + (lane >> 3);
      const int slot = lane & 7;
      const int c = slot ^ ((tr >> 1) & 7);
      int tok = tok0 + tr;
      tok = tok < M ? tok : M - 1;
      dma16(a.x + (int64_t)tok * K + k0 + 8 * c, st + q * 1024);
    }
#pragma unroll
    for (int i = 0; i < C::kWInst; ++i) {
      // W: instruction qi covers tile rows 32 qi .. 32 qi + 31, two 16-byte halves each
      const int qi = wave * C::kWInst + i;
      const int tr = 32 * qi + (lane >> 1);
      const int h = (lane & 1) ^ ((tr >> 3) & 1);
      int mat, row;
      tile_row<NMAT>(tr, row0, N, mat, row);
      dma16(a.w[mat] + (int64_t)row * (K / 2) + k0 / 2 + 16 * h, st + C::kXBytes + qi * 1024);
    }
    if ((k & 7) == 0) {
      // scale bytes of 8 steps: tile row tr's 16 bytes; lane l of wave w
      // covers row kSRows w + l
      if (lane < C::kSRows) {
        const int tr = C::kSRows * wave + lane;
        int mat, row;
        tile_row<NMAT>(tr, row0, N, mat, row);
        dma16(a.s[mat] + (int64_t)row * (K / 32) + 2 * k,
              smem + kStages * C::kStage + ((k >> 3) & 1) * kSBlock + wave * C::kSRows * 16);
      }
    }
  };
  // loads per wave of a stage (what vmcnt counts): one more every 8 steps
  constexpr int kLoads = C::kXInst + C::kWInst;
  static_assert(kLoads + 1 <= 15, "vmcnt immediate");

  f32x16_t acc[WB][kTT];
#pragma unroll
  for (int b = 0; b < WB; ++b)
#pragma unroll
    for (int t = 0; t < kTT; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[b][t][v] = 0.f;

  // this lane's operand rows
  // tile weight row of block b: gate_up blocks are [gate 0 .. WB/2-1][up ...]
  // over the same output rows, so the epilogue has g and u in one lane
  int wtr[WB];
#pragma unroll
  for (int b = 0; b < WB; ++b) {
    if constexpr (NMAT == 2) wtr[b] = (b / (WB / 2)) * 128 + wr * (kRowsW / 2) + (b % (WB / 2)) * 32 + l32;
    else wtr[b] = wr * kRowsW + b * 32 + l32;
  }
  int xtr[kTT];                   // tile token row of block t
#pragma unroll
  for (int t = 0; t < kTT; ++t) xtr[t] = wt * (BM / WT) + t * 32 + l32;

  issue_stage(kbeg);
  if (kbeg + 1 < kend) issue_stage(kbeg + 1);

  bool f16_fast = true;
  if constexpr (DT == kF16) {
    // the tile rows' scale bytes of steps [kbeg, kend): 2 per step, 16-byte
    // runs (K / 32 and 2 kbeg are multiples of 16); the barrier also lets
    // the two stages issued above land
    const int runs = 2 * (kend - kbeg) / 16;
    bool ok = true;
    for (int i = threadIdx.x; i < kWRows * runs; i += NW * 64) {
      const int tr = i / runs, c = i - tr * runs;
      int mat, row;
      tile_row<NMAT>(tr, row0, N, mat, row);
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(a.s[mat] + (int64_t)row * (K / 32) + 2 * kbeg + 16 * c);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) ok = ok && e8m0_f16_ok((v[j] >> (8 * e)) & 0xffu);
    }
    f16_fast = __syncthreads_and(ok) != 0;
  }

  // MODE 0: bf16 activations; 1: fp16, weights as fp16; 2: fp16, hi + lo
  auto k_loop = [&](auto mode_tag) {
  constexpr int MODE = decltype(mode_tag)::value;
  for (int k = kbeg; k < kend; ++k) {
    // this wave's loads of stage k are done when at most stage k+1's remain
    if (k + 1 < kend) {
      if (((k + 1) & 7) == 0) __builtin_amdgcn_s_waitcnt(0x0F70 | (kLoads + 1));
      else __builtin_amdgcn_s_waitcnt(0x0F70 | kLoads);
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70);       // vmcnt(0)
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();               // all waves: stage k landed, step k-1 done
    asm volatile("" ::: "memory");
    if (k + 2 < kend) issue_stage(k + 2);

    const uint8_t* st = smem + ((k - kbeg) % kStages) * C::kStage;
    const uint8_t* sb = smem + kStages * C::kStage + ((k >> 3) & 1) * kSBlock;
    // W operands (16 B packed per block) and scale bytes
    u32x4_t wraw[WB];
    uint32_t wsc[WB];
    bool ok = true;
#pragma unroll
    for (int b = 0; b < WB; ++b) {
      const int tr = wtr[b];
      wraw[b] = *reinterpret_cast<const u32x4_t*>(st + C::kXBytes + tr * 32 + 16 * (j ^ ((tr >> 3) & 1)));
      wsc[b] = sb[tr * 16 + 2 * (k & 7) + j];
      if constexpr (MODE != 1) ok = ok && e8m0_fast_ok(wsc[b]);
    }
    // X operands of MFMA k-step s, one 16-byte read per token block
    auto load_x = [&](int s, u32x4_t (&xo)[kTT]) {
#pragma unroll
      for (int t = 0; t < kTT; ++t) {
        const int tr = xtr[t];
        xo[t] = *reinterpret_cast<const u32x4_t*>(st + tr * 128 + 16 * ((4 * j + s) ^ ((tr >> 1) & 7)));
      }
    };
    // k-steps in order with the next k-step's X reads in flight; the
    // scheduling barriers keep the compiler from hoisting all four k-steps'
    // reads (64 more live VGPRs at BM = 256).  The exact dequantisation (a
    // scale byte outside [2, 252], wave-uniform and rare) rewrites only the
    // two converted operands: a branch around the MFMAs themselves made the
    // compiler keep two copies of the accumulators.
    const bool fast = MODE == 1 || wave_all(ok);
    u32x4_t xa[kTT], xb[kTT];
    load_x(0, xa);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4_t (&xc)[kTT] = (s & 1) ? xb : xa;
      u32x4_t (&xn)[kTT] = (s & 1) ? xa : xb;
      if (s < 3) load_x(s + 1, xn);
      u32x4_t wop[WB];
      if constexpr (MODE == 1) {
#pragma unroll
        for (int b = 0; b < WB; ++b) wop[b] = dq8_f16_fast(wraw[b][s], wsc[b]);
#pragma unroll
        for (int b = 0; b < WB; ++b)
#pragma unroll
          for (int t = 0; t < kTT; ++t) acc[b][t] = mfma32x32x16_f16(wop[b], xc[t], acc[b][t]);
      } else {
#pragma unroll
        for (int b = 0; b < WB; ++b) wop[b] = dq8_bf16_fast(wraw[b][s], wsc[b]);
        if (!fast) {
#pragma unroll
          for (int b = 0; b < WB; ++b) wop[b] = dq8_bf16_exact(wraw[b][s], wsc[b]);
        }
        if constexpr (MODE == 2) {
#pragma unroll
          for (int t = 0; t < kTT; ++t) {
            u32x4_t xh, xl;
            f16x8_split_bf16(xc[t], xh, xl);
#pragma unroll
            for (int b = 0; b < WB; ++b) acc[b][t] = mfma32x32x16(wop[b], xl, mfma32x32x16(wop[b], xh, acc[b][t]));
          }
        } else {
#pragma unroll
          for (int b = 0; b < WB; ++b)
#pragma unroll
            for (int t = 0; t < kTT; ++t) acc[b][t] = mfma32x32x16(wop[b], xc[t], acc[b][t]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  };
  if constexpr (DT == kBF16) k_loop(std::integral_constant<int, 0>{});
  else if (f16_fast) k_loop(std::integral_constant<int, 1>{});
  else k_loop(std::integral_constant<int, 2>{});

  // ---- epilogue --------------------------------------------------------
  // acc[b][t][v]: token tok0 + xtr[t], tile row block base + 8 (v/4) + 4 j + (v%4)
  if (part) {
    // fp32 partials: [ks][token][mat * tail_n + row - tail_row0], four
    // consecutive rows per store
#pragma unroll
    for (int t = 0; t < kTT; ++t) {
      const int tok = tok0 + xtr[t];
      if (tok >= M) continue;
      float* wrow = a.ws + ((int64_t)ks * M + tok) * (NMAT * a.tail_n);
#pragma unroll
      for (int b = 0; b < WB; ++b) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int orow = row0 + (NMAT == 2 ? wr * (kRowsW / 2) + (b % (WB / 2)) * 32 : wr * kRowsW + b * 32) +
                           8 * g + 4 * j;
          if (orow >= N) continue;
          const int col = (NMAT == 2 ? (b / (WB / 2)) * a.tail_n : 0) + orow - a.tail_row0;
          *reinterpret_cast<f32x4_t*>(wrow + col) =
              f32x4_t{acc[b][t][4 * g], acc[b][t][4 * g + 1], acc[b][t][4 * g + 2], acc[b][t][4 * g + 3]};
        }
      }
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < kTT; ++t) {
    const int tok = tok0 + xtr[t];
    if (tok >= M) continue;
#pragma unroll
    for (int b = 0; b < (NMAT == 2 ? WB / 2 : WB); ++b) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int orow = row0 + (NMAT == 2 ? wr * (kRowsW / 2) : wr * kRowsW) + b * 32 + 8 * g + 4 * j;
        if (orow >= N) continue;   // N % 32 == 0: the 4 rows are all in or all out
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (NMAT == 2) v[e] = silu_f32(acc[b][t][4 * g + e]) * acc[WB / 2 + b][t][4 * g + e];
          else v[e] = acc[b][t][4 * g + e];
        }
        const uint32_t lo = (uint32_t)f32_to_act<DT>(v[0]) | ((uint32_t)f32_to_act<DT>(v[1]) << 16);
        const uint32_t hi = (uint32_t)f32_to_act<DT>(v[2]) | ((uint32_t)f32_to_act<DT>(v[3]) << 16);
        const int64_t o = (int64_t)tok * N + orow;
        *reinterpret_cast<u32x2_t*>(a.out + o) = with_residual4<DT>(u32x2_t{lo, hi}, a.res, o);
      }
    }
  }
}

// out[m][row0 + n] = epilogue(sum over ks of ws[ks][m][n] (and [nt + n] for
// up)), in ks order, for the nt output rows from row0; four outputs per
// thread.
template <int NMAT, int DT>
__global__ __launch_bounds__(256) void ring_reduce(const float* __restrict__ ws, uint16_t* out,
                                                   const uint16_t* res, int M, int N, int ksplit, int row0,
                                                   int nt) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;   // group of 4 outputs
  const int64_t total = (int64_t)M * nt / 4;
  if (q >= total) return;
  const int64_t m = q / (nt / 4);
  const int n = (int)(q - m * (nt / 4)) * 4;
  f32x4_t g = {0.f, 0.f, 0.f, 0.f}, u = {0.f, 0.f, 0.f, 0.f};
  for (int ks = 0; ks < ksplit; ++ks) {
    const float* row = ws + ((int64_t)ks * M + m) * (NMAT * nt);
    g += *reinterpret_cast<const f32x4_t*>(row + n);
    if constexpr (NMAT == 2) u += *reinterpret_cast<const f32x4_t*>(row + nt + n);
  }
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = NMAT == 2 ? silu_f32(g[e]) * u[e] : g[e];
  const uint32_t lo = (uint32_t)f32_to_act<DT>(v[0]) | ((uint32_t)f32_to_act<DT>(v[1]) << 16);
  const uint32_t hi = (uint32_t)f32_to_act<DT>(v[2]) | ((uint32_t)f32_to_act<DT>(v[3]) << 16);
  const int64_t o = m * N + row0 + n;
  *reinterpret_cast<u32x2_t*>(out + o) = with_residual4<DT>(u32x2_t{lo, hi}, res, o);
}

// Number of K ranges per output tile.  Cost model (microseconds): a tile's
// full-K time at ~5 TFLOP/s per CU, times the rounds of workgroups the split
// grid needs on 256 CUs, divided by the split; plus the fp32 partials written
// and read back (mostly from the 256 MB last-level cache) and the reduce
// launch.  The smallest split with the least cost wins; K ranges are whole
// 8-step blocks, and the partials of all ranges fit the workspace limit.
// The option TINYINFER_RING_KSPLIT=<n> forces n (clamped), for tuning.
// whole_per_cu: workgroups of the unsplit kernel that fit one CU at once.
// With two, a CU that runs two tiles together takes ~1.75 tile times (both
// share its matrix cores; Qwen3-8B gate_up, 128-token tiles: 384 tiles in
// 118-128 us against 70.5 us for 192), not two rounds.
int ring_ksplit(const RingArgs& r, int bm, int nmat, int64_t tiles, int per_cu, size_t ws_limit,
                double* cost_out = nullptr, bool* forced = nullptr, int whole_per_cu = 1) {
  const int nblk = r.K / (8 * kBK);
  int cap = nblk < 32 ? nblk : 32;
  const size_t per_split = (size_t)r.M * nmat * r.N * sizeof(float);
  const size_t fit = per_split ? ws_limit / per_split : 0;
  if ((size_t)cap > fit) cap = (int)fit;
  // per_cu workgroups share a CU: each runs at 1 / per_cu of its rate
  const int64_t slots = 256 * per_cu;
  const double t_tile = 2.0 * bm * 256.0 * r.K / 5e6 * per_cu;
  const double ws_us_per_split = 8.0 * r.M * nmat * (double)r.N / 8e6;
  int best = 1;
  double best_cost = t_tile * (double)((tiles + slots - 1) / slots);
  if (per_cu == 1 && whole_per_cu >= 2) {
    const int64_t c = (tiles + 255) / 256;         // tiles per CU
    best_cost = t_tile * (1.75 * (double)(c / 2) + (double)(c % 2));
  }
  if (cost_out) *cost_out = best_cost;
  if (forced) *forced = false;
  if (cap < 2) return 1;
  if (const int v = option(kOptRingKsplit); v >= 1) {
    if (forced) *forced = true;
    return v < cap ? v : cap;
  }
  for (int ks = 2; ks <= cap; ++ks) {
    const double rounds = (double)((tiles * ks + slots - 1) / slots);
    const double cost = t_tile * rounds / ks + ws_us_per_split * ks + 3.0;
    if (cost < best_cost * 0.97) {
      best = ks;
      best_cost = cost;
    }
  }
  if (cost_out) *cost_out = best_cost;
  return best;
}

// Split of the tiles past the last full round only (RingArgs::nfull): the
// first rounds of workgroups over the CUs run whole tiles, and the remaining
// tiles (a band of whole weight-row tiles) are split into s K ranges so that
// they fill one more round.  At Qwen3-8B gate_up and 512 tokens: 384 tiles =
// 256 whole + 128 halves, where the whole-tile grid left half of its second
// round empty.  Same cost model as ring_ksplit; s = 1 when it does not pay.
struct TailSplit {
  int nfull = 0;
  int s = 1;
  int row0 = 0;
  double cost = 0.0;
};
TailSplit ring_tail_split(const RingArgs& r, int bm, int nmat, int rows_out, int64_t tiles, size_t ws_limit) {
  TailSplit t;
  const int64_t slots = 256;
  if (option(kOptRingTail) == 0 || tiles <= slots || tiles % slots == 0 || r.m_tiles < 1) return t;
  const int64_t rounds = tiles / slots;
  const int64_t nfull = rounds * slots / r.m_tiles * r.m_tiles;
  const int64_t ntail = tiles - nfull;
  if (nfull < 1 || ntail < 1) return t;
  const int nblk = r.K / (8 * kBK);
  int64_t s = ((rounds + 1) * slots - nfull) / ntail;
  s = s < nblk ? s : nblk;
  s = s < 32 ? s : 32;
  const int row0 = (int)(nfull / r.m_tiles) * rows_out;
  const int64_t tail_n = (int64_t)r.N - row0;
  if (tail_n <= 0) return t;
  const size_t per_split = (size_t)r.M * nmat * (size_t)tail_n * sizeof(float);
  while (s >= 2 && (size_t)s * per_split > ws_limit) --s;
  if (s < 2) return t;
  const double t_tile = 2.0 * bm * 256.0 * r.K / 5e6;
  // whole rounds, the split round, the partials written and read back, the
  // reduce launch and the extra round's pipeline fill (measured at 8B gate_up:
  // 288 tiles = 255 whole + 33 in 7 ranges 1.40 tile times, 384 = 256 + 128
  // halves 1.78)
  t.cost = t_tile * (double)rounds + t_tile / (double)s + 8.0 * (double)s * r.M * nmat * (double)tail_n / 8e6 +
           3.0 + 0.1 * t_tile;
  t.nfull = (int)nfull;
  t.s = (int)s;
  t.row0 = row0;
  return t;
}

// A caller-provided workspace (fixed != null) of fixed_bytes is used instead
// of the library's per-stream one, and nothing is allocated.
struct FixedWs {
  float* ptr;
  size_t bytes;
};

template <int NMAT, int BM, int WR, int NW = 8, int DT = kBF16>
hipError_t launch_ring(RingArgs r, hipStream_t st, FixedWs fixed) {
  using C = RingCfg<BM, NW>;
  constexpr int kRowsOut = NMAT == 2 ? 128 : 256;
  r.m_tiles = (r.M + BM - 1) / BM;
  r.n_tiles = (r.N + kRowsOut - 1) / kRowsOut;
  const int64_t tiles = (int64_t)r.m_tiles * r.n_tiles;
  if (tiles > 0x7fffffff / 32) return hipErrorInvalidValue;
  const size_t ws_limit = fixed.ptr ? fixed.bytes : workspace_limit();
  // how many unsplit workgroups one CU holds at once (registers and LDS),
  // asked once per kernel
  static std::once_flag occ_once;
  static int whole_per_cu = 1;
  std::call_once(occ_once, [] {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n, reinterpret_cast<const void*>(gemm_ring_kernel<NMAT, BM, false, WR, NW, DT>), NW * 64, C::kLds) ==
            hipSuccess &&
        n > 0)
      whole_per_cu = n;
    else
      (void)hipGetLastError();
  });
  double uniform_cost = 0.0;
  bool forced = false;
  const int ksplit_want =
      ring_ksplit(r, BM, NMAT, tiles, NW == 4 ? 2 : 1, ws_limit, &uniform_cost, &forced, whole_per_cu);
  int ksplit = 1;
  r.ws = nullptr;
  r.nfull = 0;
  r.tail_row0 = 0;
  r.tail_n = r.N;
  // the tail split when the model prefers it to the best split of every tile
  TailSplit t;
  if (NW == 8 && !forced) t = ring_tail_split(r, BM, NMAT, kRowsOut, tiles, ws_limit);
  if (t.s > 1 && t.cost < 0.97 * uniform_cost) {
    const int tail_n = r.N - t.row0;
    r.ws = fixed.ptr ? fixed.ptr : gemm_split_workspace((size_t)t.s * r.M * NMAT * tail_n * sizeof(float), st);
    if (r.ws) {
      ksplit = t.s;
      r.nfull = t.nfull;
      r.tail_row0 = t.row0;
      r.tail_n = tail_n;
    }
  } else if (ksplit_want > 1) {
    r.ws = fixed.ptr ? fixed.ptr
                     : gemm_split_workspace((size_t)ksplit_want * r.M * NMAT * r.N * sizeof(float), st);
    if (r.ws) ksplit = ksplit_want;
  }
  r.ksplit = ksplit;
  auto go = [&](auto kern, int64_t nwg) -> hipError_t {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            C::kLds) != hipSuccess) {
      (void)hipGetLastError();
      return hipErrorNotSupported;
    }
    kern<<<(unsigned)nwg, NW * 64, C::kLds, st>>>(r);
    return hipGetLastError();
  };
  if (ksplit == 1) return go(gemm_ring_kernel<NMAT, BM, false, WR, NW, DT>, tiles);
  const hipError_t e = go(gemm_ring_kernel<NMAT, BM, true, WR, NW, DT>, r.nfull + (tiles - r.nfull) * ksplit);
  if (e != hipSuccess) return e;
  const int64_t groups = (int64_t)r.M * r.tail_n / 4;
  ring_reduce<NMAT, DT><<<(unsigned)((groups + 255) / 256), 256, 0, st>>>(r.ws, r.out, r.res, r.M, r.N, ksplit,
                                                                          r.tail_row0, r.tail_n);
  return hipGetLastError();
}

}  // namespace

bool gemm_ring_supported(const MlpArgs& a, int stage) {
  if (option(kOptGemmRing) == 0 || (a.dtype != kBF16 && a.dtype != kF16)) return false;
  if ((stage & kStageGateUp) && a.hidden % 512 != 0) return false;
  if ((stage & kStageDown) && a.inter % 512 != 0) return false;
  if (a.n > (1 << 24) || a.hidden > (1 << 20) || a.inter > (1 << 22)) return false;
  const void* scales[] = {a.gate_scale, a.up_scale, a.down_scale};
  for (const void* p : scales)
    if (p && (reinterpret_cast<uintptr_t>(p) & 15u)) return false;
  return device_info().lds_per_block >= RingCfg<256, 8>::kLds;
}

// Token tiles of 64 up to this many tokens (a 128-token tile would be mostly
// padding; the tile count is the same).
constexpr int64_t kSmallTile = 64;

hipError_t launch_gemm_ring_mlp(const MlpArgs& a, int stage, hipStream_t st) {
  const FixedWs fx{a.ws, a.ws_bytes};
  if (stage & kStageGateUp) {
    RingArgs r{static_cast<const uint16_t*>(a.x), {a.gate, a.up}, {a.gate_scale, a.up_scale},
               static_cast<uint16_t*>(a.tmp), (int)a.n, (int)a.inter, (int)a.hidden, 0, 0, nullptr, 1, nullptr};
    // 256-token tiles once there are enough of them (more reuse of each
    // weight tile), 128 below
    // wave layout and waves per workgroup (tuning options; 4 x 2 and 8 by default)
    const int wr = option(kOptRingWrGu);
    const int nw = option(kOptRingNwGu);
    hipError_t e;
    if (a.dtype == kF16) {
      // fp16: the default layout only (8 waves, 4 x 2)
      if (a.n > 1024) e = launch_ring<2, 256, 4, 8, kF16>(r, st, fx);
      else if (a.n <= kSmallTile) e = launch_ring<2, 64, 4, 8, kF16>(r, st, fx);
      else e = launch_ring<2, 128, 4, 8, kF16>(r, st, fx);
    } else if (nw == 4) e = wr == 2 ? launch_ring<2, 128, 2, 4>(r, st, fx) : launch_ring<2, 128, 4, 4>(r, st, fx);
    else if (a.n > 1024) e = wr == 2 ? launch_ring<2, 256, 2>(r, st, fx) : launch_ring<2, 256, 4>(r, st, fx);
    else if (a.n <= kSmallTile) e = launch_ring<2, 64, 4>(r, st, fx);
    else e = wr == 2 ? launch_ring<2, 128, 2>(r, st, fx) : launch_ring<2, 128, 4>(r, st, fx);
    if (e != hipSuccess) return e;
  }
  if (stage & kStageDown) {
    RingArgs r{static_cast<const uint16_t*>(a.tmp), {a.down, a.down}, {a.down_scale, a.down_scale},
               static_cast<uint16_t*>(a.out), (int)a.n, (int)a.hidden, (int)a.inter, 0, 0, nullptr, 1,
               static_cast<const uint16_t*>(a.residual)};
    const int wr = option(kOptRingWrDn);
    const int nw = option(kOptRingNwDn);
    if (a.dtype == kF16)
      return a.n <= kSmallTile ? launch_ring<1, 64, 4, 8, kF16>(r, st, fx) : launch_ring<1, 128, 4, 8, kF16>(r, st, fx);
    if (nw == 4) return wr == 2 ? launch_ring<1, 64, 2, 4>(r, st, fx) : launch_ring<1, 64, 4, 4>(r, st, fx);
    if (a.n <= kSmallTile) return launch_ring<1, 64, 4>(r, st, fx);
    return wr == 2 ? launch_ring<1, 128, 2>(r, st, fx) : launch_ring<1, 128, 4>(r, st, fx);
  }
  return hipSuccess;
}

}  // namespace tinyinfer
