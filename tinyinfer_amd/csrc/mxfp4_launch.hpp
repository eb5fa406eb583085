// Internal host-side launchers shared between the kernel translation units and
// the C ABI (mxfp4_capi.hip). Not part of the public interface.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace tinyinfer {

struct MlpArgs {
  const void* x;            // [n, hidden] activation dtype
  const uint8_t* gate;      // [inter, hidden/2]
  const uint8_t* gate_scale;
  const uint8_t* up;        // [inter, hidden/2]
  const uint8_t* up_scale;
  const uint8_t* down;      // [hidden, inter/2]
  const uint8_t* down_scale;
  int64_t n;
  int64_t hidden;
  int64_t inter;
  void* tmp;                // [n, inter] activation dtype
  void* out;                // [n, hidden] activation dtype
  int dtype;                // kF16 / kBF16
  const void* residual;     // [n, hidden] or null: out = residual + down(tmp), rounded like torch's add
  // RMSNorm prologue (the streaming gate_up kernel only): x is normalized in
  // the kernel's LDS copy, xn = round(norm_w * x * rsqrt(mean(x^2) + eps)),
  // and workgroup 0 writes it to xn [n, hidden]; null norm_w: x is used as is
  const void* norm_w = nullptr;   // [hidden] activation dtype
  float eps = 0.f;
  void* xn = nullptr;
  // Caller-provided split-K workspace (the no-alloc entry point): when ws is
  // set, the tile and GEMM launchers use it, up to ws_bytes, and never
  // allocate; null: the per-(device, stream) buffer of gemm_split_workspace.
  float* ws = nullptr;
  size_t ws_bytes = 0;
};

// Properties of the current device, read once per device (thread-safe);
// cus == 0 when they could not be read.
struct DeviceInfo {
  int cus = 0;
  int64_t lds_per_block = 0;
  bool gfx950 = false;
};
DeviceInfo device_info();

// Tuning options.  Each starts from the environment variable of the same
// name (read once, at the first query, by whichever thread gets there) and
// can be changed at any time through set_option (the C ABI's
// tinyinfer_mxfp4_set_option); reads and writes are atomic.
enum Opt : int {
  kOptRowstream,        // TINYINFER_ROWSTREAM      1: row-streaming kernels on (0 off)
  kOptRowpair,          // TINYINFER_ROWPAIR        1: row-pair kernels on
  kOptTile,             // TINYINFER_TILE           1: split-K tile kernels on
  kOptTileGu,           // TINYINFER_TILE_GU        1: one-launch tile gate_up on
  kOptRowSplitGateUp,   // TINYINFER_ROW_SPLIT_GATEUP  waves per gate_up row (0 auto, 1, 2, 4)
  kOptRowSplitDown,     // TINYINFER_ROW_SPLIT_DOWN    waves per down row (0 auto, 1, 2, 4)
  kOptGemmRing,         // TINYINFER_GEMM_RING      1: ring GEMM on (0: register-staged GEMM)
  kOptRingKsplit,       // TINYINFER_RING_KSPLIT    K ranges of the ring GEMM (0 auto)
  kOptRingWrGu,         // TINYINFER_RING_WR_GU     ring wave rows, gate_up (2 or 4)
  kOptRingNwGu,         // TINYINFER_RING_NW_GU     ring waves per workgroup, gate_up (4 or 8)
  kOptRingWrDn,         // TINYINFER_RING_WR_DN
  kOptRingNwDn,         // TINYINFER_RING_NW_DN
  kOptSkinnyNw,         // TINYINFER_SKINNY_NW      skinny waves per workgroup (0 auto, 4, 8)
  kOptStreamSpuGu,      // TINYINFER_STREAM_SPU_GU  stream segments per unit, gate_up (0 auto)
  kOptStreamSpuDn,      // TINYINFER_STREAM_SPU_DN
  kOptStreamXreg,       // TINYINFER_STREAM_XREG    1: gate_up activations in VGPRs
  kOptWorkspaceMB,      // TINYINFER_WORKSPACE_MB   limit of one split-K workspace buffer
  kOptDecodeSpin,       // TINYINFER_DECODE_SPIN    fused decode kernel's wait bound (poll rounds)
  kOptRingTail,         // TINYINFER_RING_TAIL      1: ring GEMM splits only the tiles past the last full round
  kOptCount
};
int option(Opt o);
bool set_option(const char* name, int value);
bool get_option(const char* name, int* value);

// Which part of the MLP a launcher runs: the gate_up stage (tmp = SiLU(x G^T) *
// (x U^T)), the down stage (out = tmp D^T), or both in order.
enum Stage : int { kStageGateUp = 1, kStageDown = 2, kStageBoth = 3 };

// Skinny path: weights streamed once per 64 tokens (MFMA 16x16x32, weights as
// the 16-row operand). Any n >= 1.
hipError_t launch_skinny_mlp(const MlpArgs& a, int stage, hipStream_t stream);

// Tiled MFMA GEMM path (n >= 128 preferred; any n >= 1 is correct).
hipError_t launch_gemm_mlp(const MlpArgs& a, int stage, hipStream_t stream);

// Prefill GEMM with a three-stage direct-to-LDS ring (bf16 or fp16, the
// stage's K a multiple of 512, 16-byte aligned scale rows); launch_gemm_mlp
// serves the other GEMM-path calls.
bool gemm_ring_supported(const MlpArgs& a, int stage);
hipError_t launch_gemm_ring_mlp(const MlpArgs& a, int stage, hipStream_t stream);

// Streaming decode GEMV kernels (n <= 8): one launch per stage, contiguous
// load front across the chip.  stream_supported() says whether the call's
// shape, alignment and LDS needs fit; launch_stream_mlp must only be called
// when it does.
bool stream_supported(const MlpArgs& a, int stage);
hipError_t launch_stream_mlp(const MlpArgs& a, int stage, hipStream_t stream);

// Row-streaming kernels for one token, and for the down stage of two (bf16): each
// load reads 1 KB of one weight row, a wave owns whole rows or a contiguous
// share of them.  rowstream_supported() says whether the call fits (K % 128
// == 0, activations of a wave's chunks in VGPRs, x within the LDS, 16-byte
// alignment); rowstream_enabled() is false when TINYINFER_ROWSTREAM=0 (then
// the n <= 8 stream kernels serve these calls).
bool rowstream_enabled();
bool rowstream_supported(const MlpArgs& a, int stage);
hipError_t launch_rowstream_mlp(const MlpArgs& a, int stage, hipStream_t stream);

// Row-pair kernels for 2..4 tokens: each load reads 512 B of each of
// two weight rows, one MFMA serves two tokens.  rowpair_supported() says
// whether the call fits; rowpair_enabled() is false when TINYINFER_ROWPAIR=0.
bool rowpair_enabled();
bool rowpair_supported(const MlpArgs& a, int stage);
hipError_t launch_rowpair_mlp(const MlpArgs& a, int stage, hipStream_t stream);

// Split-K tile kernels for up to 80 tokens (K % 1024 == 0): a workgroup
// owns one 1024-element K range (its activations staged once in LDS) and
// streams 16-row weight groups through MFMA; a reduce launch adds the K
// ranges in order and applies the epilogue (gate_up in one launch, partials
// added in LDS, when all of x fits).  tile_supported() says whether
// the call fits and its fp32 workspace can be had (not during graph capture
// unless the stream's workspace is already large enough); tile_enabled() is
// false when TINYINFER_TILE=0.
bool tile_enabled();
bool tile_supported(const MlpArgs& a, int stage, hipStream_t stream);
// Workspace bytes the tile kernels need for this call, 0 when they do not
// apply (shape, dtype, alignment).
size_t tile_workspace_need(const MlpArgs& a, int stage);
hipError_t launch_tile_mlp(const MlpArgs& a, int stage, hipStream_t stream);

// The split-K workspace of the GEMM and tile kernels: one fp32 buffer per
// (device, stream), grown on demand up to workspace_limit() bytes; null when
// it cannot grow (over the limit, graph capture, allocation failure).
// Buffers live until release_workspaces(), which synchronizes every device
// that holds one and frees them all.
float* gemm_split_workspace(size_t bytes, hipStream_t stream);
size_t workspace_limit();
size_t workspace_bytes_held();
hipError_t release_workspaces();

// Fused decode kernel (gate_up, cross-workgroup flags, down in one launch)
// for n <= 4 tokens; hipErrorNotSupported when the shape, alignment or the
// device's LDS/occupancy do not allow it.
hipError_t launch_decode_mlp(const MlpArgs& a, hipStream_t stream);

// Spin timeouts of the fused decode kernel's wait since load or the last
// decode_reset() (0 unless a workgroup was not resident); synchronous.  While
// it is nonzero, fused decode launches exit at entry without writing.
unsigned int decode_barrier_timeouts();
// Clears the fused decode kernel's flags, epoch, poison and timeout count on
// the current device after synchronizing it.
hipError_t decode_reset();

// The whole MLP entry (validation, device check, kernel choice, launches) of
// the C ABI, returning a TI_* status; `path` is a TI_PATH_* value.
int run_mlp(const MlpArgs& a, int stage, int path, void* stream);

// RMSNorm of n rows of `hidden` activations (the reference's rmsnorm
// kernel, tinyinfer/csrc/rmsnorm.cu:10-54): out = round(w * x * rsqrt(sum(x^2)
// / hidden + eps)) per row, fp32 inside.  hidden % 8 == 0, 16-byte aligned
// rows.
hipError_t launch_rmsnorm(const void* x, const void* w, float eps, int64_t n, int64_t hidden, void* out,
                          int dtype, hipStream_t stream);

hipError_t launch_dequant(const uint8_t* packed, const uint8_t* scale, int64_t rows, int64_t k,
                          void* out, int out_dtype, hipStream_t stream);

hipError_t launch_quantize(const void* w, int in_dtype, int64_t rows, int64_t k, uint8_t* packed,
                           uint8_t* scale, uint32_t* flags, hipStream_t stream);

}  // namespace tinyinfer
