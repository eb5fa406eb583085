// C ABI of the MXFP4 MLP library (declared in include/tinyinfer_mxfp4.h).
//
// Replaces the reference's extern "C" mlp_forward_mxfp4_cuda
// (tinyinfer/csrc/mlp_fp4.cu:466-518): same arguments plus an explicit
// stream; validation failures and HIP errors come back as status codes
// instead of thrown exceptions, so the boundary is safe for any FFI.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/tinyinfer_mxfp4.h"
#include "mxfp4_common.hpp"
#include "mxfp4_launch.hpp"

namespace {

using tinyinfer::MlpArgs;

// Largest index any kernel forms in 64-bit is fine; grid dimensions and the
// per-row chunk counts are 32-bit, so cap sizes well below that.
constexpr size_t kMaxDim = size_t(1) << 30;
constexpr size_t kMaxTokens = size_t(1) << 24;

int check_device() {
  const tinyinfer::DeviceInfo d = tinyinfer::device_info();
  return d.cus > 0 && d.gfx950 ? TI_OK : TI_ERR_NO_DEVICE;
}

int to_status(hipError_t e) { return e == hipSuccess ? TI_OK : TI_ERR_HIP; }

// Checks shared by every MLP entry point; `stage` says which pointers the
// call reads and writes (the others may be null).
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int validate_mlp(const MlpArgs& a, int stage) {
  if (!a.tmp) return TI_ERR_INVALID_ARG;
  if ((stage & tinyinfer::kStageGateUp) && (!a.x || !a.gate || !a.gate_scale || !a.up || !a.up_scale))
    return TI_ERR_INVALID_ARG;
  if ((stage & tinyinfer::kStageDown) && (!a.down || !a.down_scale || !a.out)) return TI_ERR_INVALID_ARG;
  if (a.n <= 0 || a.hidden <= 0 || a.inter <= 0) return TI_ERR_INVALID_ARG;
  if (a.hidden % 32 != 0 || a.inter % 32 != 0) return TI_ERR_BAD_SHAPE;
  if (a.dtype != TI_DTYPE_F16 && a.dtype != TI_DTYPE_BF16) return TI_ERR_BAD_DTYPE;
  if ((size_t)a.n > kMaxTokens || (size_t)a.hidden > kMaxDim || (size_t)a.inter > kMaxDim)
    return TI_ERR_TOO_LARGE;
  // 16-byte vector loads of activations and packed weights
  if (!aligned16(a.tmp)) return TI_ERR_MISALIGNED;
  if ((stage & tinyinfer::kStageGateUp) && (!aligned16(a.x) || !aligned16(a.gate) || !aligned16(a.up)))
    return TI_ERR_MISALIGNED;
  if ((stage & tinyinfer::kStageDown) && !aligned16(a.down)) return TI_ERR_MISALIGNED;
  if (a.residual && (!(stage & tinyinfer::kStageDown) || !aligned16(a.residual))) return TI_ERR_MISALIGNED;
  return TI_OK;
}

// Token count from which the tiled GEMM beats the skinny path (weights are
// re-streamed once per 64 tokens on the skinny path); for the ring GEMM's
// shapes (K a multiple of 512) it wins from ~16 tokens (8B MLP with
// 64-token tiles: 16 tokens 49.8 against 53.5 us, 64 tokens 56.5 against 152).
constexpr size_t kGemmMinTokens = 96;
constexpr size_t kRingMinTokens = 16;
// Token count up to which the streaming decode kernels are used.
constexpr size_t kStreamMaxTokens = 8;
// split-K tile kernels: up to 80 tokens (five 16-token MFMA column tiles)
constexpr size_t kTileMaxTokens = 80;
// up to this many tokens a caller-provided workspace too small for the tile
// kernels' split is refused (TI_ERR_SCRATCH); from 65 tokens such a call
// takes the ring GEMM, which splits K only as far as the workspace holds
constexpr size_t kTileScratchTokens = 64;

// One stage of a small batch on the best kernel that takes it: 2..4 tokens on
// the row-pair kernels, one or two on the row-streaming kernels, n <= 8 on the
// 8-row item kernels, n <= 80 on the split-K tile kernels, else the
// 16-token-tile skinny kernels.  Chosen per stage: the two stages' K differ
// (at 8B and n = 8 down's activations exceed the LDS the item kernel stages
// them in, while gate_up's fit).
hipError_t small_stage(const MlpArgs& a, int st, hipStream_t s) {
  if (a.n >= 2 && a.n <= 4 && tinyinfer::rowpair_enabled() && tinyinfer::rowpair_supported(a, st))
    return tinyinfer::launch_rowpair_mlp(a, st, s);
  if (a.n <= 2 && tinyinfer::rowstream_enabled() && tinyinfer::rowstream_supported(a, st))
    return tinyinfer::launch_rowstream_mlp(a, st, s);
  if ((size_t)a.n <= kStreamMaxTokens && tinyinfer::stream_supported(a, st))
    return tinyinfer::launch_stream_mlp(a, st, s);
  if ((size_t)a.n <= kTileMaxTokens && tinyinfer::tile_enabled() && tinyinfer::tile_supported(a, st, s))
    return tinyinfer::launch_tile_mlp(a, st, s);
  return tinyinfer::launch_skinny_mlp(a, st, s);
}

int mlp_impl(const MlpArgs& a, int stage, int path, void* stream) {
  // sizes arrive as size_t; anything that wraps negative is rejected here
  int st = validate_mlp(a, stage);
  if (st != TI_OK) return st;
  if (path != TI_PATH_AUTO && path != TI_PATH_SKINNY && path != TI_PATH_GEMM && path != TI_PATH_DECODE)
    return TI_ERR_INVALID_ARG;
  st = check_device();
  if (st != TI_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // a caller-provided workspace (the no-alloc entry point) must hold the
  // whole split of the tile kernels when they would run
  if (a.ws && (path == TI_PATH_AUTO || path == TI_PATH_SKINNY) && (size_t)a.n <= kTileScratchTokens &&
      tinyinfer::tile_enabled()) {
    size_t need = 0;
    for (int sg : {(int)tinyinfer::kStageGateUp, (int)tinyinfer::kStageDown})
      if (stage & sg) need = std::max(need, tinyinfer::tile_workspace_need(a, sg));
    if (need > a.ws_bytes) return TI_ERR_SCRATCH;
  }
  if (path == TI_PATH_DECODE) {
    if (stage != tinyinfer::kStageBoth) return TI_ERR_UNSUPPORTED;
    const hipError_t e = tinyinfer::launch_decode_mlp(a, s);
    if (e == hipErrorNotSupported) return TI_ERR_UNSUPPORTED;
    return to_status(e);
  }
  if (path == TI_PATH_AUTO) {
    const bool tile = (size_t)a.n <= kTileMaxTokens && tinyinfer::tile_enabled() &&
                      tinyinfer::tile_supported(a, stage, s);
    const bool ring = (size_t)a.n >= kRingMinTokens && tinyinfer::gemm_ring_supported(a, stage);
    path = ((size_t)a.n >= kGemmMinTokens || (ring && !tile)) ? TI_PATH_GEMM : TI_PATH_SKINNY;
  }
  if (path == TI_PATH_GEMM) {
    if (tinyinfer::gemm_ring_supported(a, stage)) return to_status(tinyinfer::launch_gemm_ring_mlp(a, stage, s));
    return to_status(tinyinfer::launch_gemm_mlp(a, stage, s));
  }
  if (stage & tinyinfer::kStageGateUp) {
    const hipError_t e = small_stage(a, tinyinfer::kStageGateUp, s);
    if (e != hipSuccess) return to_status(e);
  }
  if (stage & tinyinfer::kStageDown) return to_status(small_stage(a, tinyinfer::kStageDown, s));
  return TI_OK;
}

int64_t as_dim(size_t v) { return v > (size_t)INT64_MAX ? -1 : (int64_t)v; }

}  // namespace

int tinyinfer::run_mlp(const MlpArgs& a, int stage, int path, void* stream) { return mlp_impl(a, stage, path, stream); }

extern "C" {

int tinyinfer_mlp_forward_mxfp4(const void* X, const uint8_t* gate, const uint8_t* gate_scale,
                                const uint8_t* up, const uint8_t* up_scale, const uint8_t* down,
                                const uint8_t* down_scale, size_t N, size_t hidden_dim,
                                size_t intermediate, void* tmp, void* O, int dtype_code,
                                void* stream) {
  MlpArgs a{X, gate, gate_scale, up, up_scale, down, down_scale, as_dim(N), as_dim(hidden_dim),
            as_dim(intermediate), tmp, O, dtype_code};
  return mlp_impl(a, tinyinfer::kStageBoth, TI_PATH_AUTO, stream);
}

int tinyinfer_mlp_forward_mxfp4_path(const void* X, const uint8_t* gate, const uint8_t* gate_scale,
                                     const uint8_t* up, const uint8_t* up_scale,
                                     const uint8_t* down, const uint8_t* down_scale, size_t N,
                                     size_t hidden_dim, size_t intermediate, void* tmp, void* O,
                                     int dtype_code, int path, void* stream) {
  MlpArgs a{X, gate, gate_scale, up, up_scale, down, down_scale, as_dim(N), as_dim(hidden_dim),
            as_dim(intermediate), tmp, O, dtype_code};
  return mlp_impl(a, tinyinfer::kStageBoth, path, stream);
}

int tinyinfer_mlp_gate_up_mxfp4(const void* X, const uint8_t* gate, const uint8_t* gate_scale,
                                const uint8_t* up, const uint8_t* up_scale, size_t N,
                                size_t hidden_dim, size_t intermediate, void* tmp, int dtype_code,
                                int path, void* stream) {
  MlpArgs a{X, gate, gate_scale, up, up_scale, nullptr, nullptr, as_dim(N), as_dim(hidden_dim),
            as_dim(intermediate), tmp, nullptr, dtype_code};
  return mlp_impl(a, tinyinfer::kStageGateUp, path, stream);
}

int tinyinfer_mlp_down_mxfp4(const void* tmp, const uint8_t* down, const uint8_t* down_scale,
                             size_t N, size_t hidden_dim, size_t intermediate, void* O,
                             int dtype_code, int path, void* stream) {
  MlpArgs a{nullptr, nullptr, nullptr, nullptr, nullptr, down, down_scale, as_dim(N),
            as_dim(hidden_dim), as_dim(intermediate), const_cast<void*>(tmp), O, dtype_code};
  return mlp_impl(a, tinyinfer::kStageDown, path, stream);
}

int tinyinfer_mlp_forward_mxfp4_residual(const void* X, const uint8_t* gate, const uint8_t* gate_scale,
                                         const uint8_t* up, const uint8_t* up_scale,
                                         const uint8_t* down, const uint8_t* down_scale, size_t N,
                                         size_t hidden_dim, size_t intermediate, void* tmp,
                                         const void* residual, void* O, int dtype_code, int path,
                                         void* stream) {
  if (!residual) return TI_ERR_INVALID_ARG;
  MlpArgs a{X, gate, gate_scale, up, up_scale, down, down_scale, as_dim(N), as_dim(hidden_dim),
            as_dim(intermediate), tmp, O, dtype_code, residual};
  return mlp_impl(a, tinyinfer::kStageBoth, path, stream);
}

int tinyinfer_mlp_forward_mxfp4_rmsnorm(const void* X, const void* norm_weight, float eps,
                                        const uint8_t* gate, const uint8_t* gate_scale, const uint8_t* up,
                                        const uint8_t* up_scale, const uint8_t* down,
                                        const uint8_t* down_scale, size_t N, size_t hidden_dim,
                                        size_t intermediate, void* xn, void* tmp, void* O, int dtype_code,
                                        int path, void* stream) {
  if (!X || !norm_weight || !xn) return TI_ERR_INVALID_ARG;
  // the hidden state is also the residual
  MlpArgs a{X, gate, gate_scale, up, up_scale, down, down_scale, as_dim(N), as_dim(hidden_dim),
            as_dim(intermediate), tmp, O, dtype_code, X};
  int st = validate_mlp(a, tinyinfer::kStageBoth);
  if (st != TI_OK) return st;
  if (!aligned16(norm_weight) || !aligned16(xn)) return TI_ERR_MISALIGNED;
  if (path != TI_PATH_AUTO && path != TI_PATH_SKINNY && path != TI_PATH_GEMM && path != TI_PATH_DECODE)
    return TI_ERR_INVALID_ARG;
  st = check_device();
  if (st != TI_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // decode sizes on the streaming kernels: the norm in gate_up's prologue
  const bool small = (size_t)a.n <= kStreamMaxTokens;
  if (small && (path == TI_PATH_SKINNY || (path == TI_PATH_AUTO && (size_t)a.n < kGemmMinTokens))) {
    MlpArgs f = a;
    f.norm_w = norm_weight;
    f.eps = eps;
    f.xn = xn;
    hipError_t e = hipErrorNotSupported;
    // the same kernel order as small_stage (the skinny kernels have no norm prologue)
    if (f.n >= 2 && f.n <= 4 && tinyinfer::rowpair_enabled() && tinyinfer::rowpair_supported(f, tinyinfer::kStageGateUp))
      e = tinyinfer::launch_rowpair_mlp(f, tinyinfer::kStageGateUp, s);
    else if (f.n <= 2 && tinyinfer::rowstream_enabled() && tinyinfer::rowstream_supported(f, tinyinfer::kStageGateUp))
      e = tinyinfer::launch_rowstream_mlp(f, tinyinfer::kStageGateUp, s);
    else if (tinyinfer::stream_supported(f, tinyinfer::kStageGateUp))
      e = tinyinfer::launch_stream_mlp(f, tinyinfer::kStageGateUp, s);
    if (e != hipErrorNotSupported) {
      if (e != hipSuccess) return to_status(e);
      return to_status(small_stage(a, tinyinfer::kStageDown, s));   // residual = X
    }
  }
  // elsewhere: the norm kernel writes xn, then the MLP on xn with X as residual
  const hipError_t e = tinyinfer::launch_rmsnorm(X, norm_weight, eps, a.n, a.hidden, xn, dtype_code, s);
  if (e != hipSuccess) return to_status(e);
  a.x = xn;
  return mlp_impl(a, tinyinfer::kStageBoth, path, stream);
}

int tinyinfer_rmsnorm(const void* X, const void* weight, float eps, size_t num_rows, size_t hidden_dim, void* O,
                      int dtype_code, void* stream) {
  if (!X || !weight || !O) return TI_ERR_INVALID_ARG;
  if (num_rows == 0 || hidden_dim == 0) return TI_ERR_INVALID_ARG;
  if (hidden_dim % 8 != 0) return TI_ERR_BAD_SHAPE;
  if (dtype_code != TI_DTYPE_F16 && dtype_code != TI_DTYPE_BF16) return TI_ERR_BAD_DTYPE;
  if (num_rows > kMaxTokens * 64 || hidden_dim > kMaxDim) return TI_ERR_TOO_LARGE;
  if (!aligned16(X) || !aligned16(weight) || !aligned16(O)) return TI_ERR_MISALIGNED;
  const int st = check_device();
  if (st != TI_OK) return st;
  return to_status(tinyinfer::launch_rmsnorm(X, weight, eps, (int64_t)num_rows, (int64_t)hidden_dim, O, dtype_code,
                                             static_cast<hipStream_t>(stream)));
}

int tinyinfer_mxfp4_linear(const void* X, const uint8_t* w, const uint8_t* w_scale, size_t N,
                           size_t in_features, size_t out_features, const void* residual, void* O,
                           int dtype_code, int path, void* stream) {
  if (!X) return TI_ERR_INVALID_ARG;
  // the down stage reads its input from tmp: [N, in_features] -> [N, out_features]
  MlpArgs a{nullptr, nullptr, nullptr, nullptr, nullptr, w, w_scale, as_dim(N), as_dim(out_features),
            as_dim(in_features), const_cast<void*>(X), O, dtype_code, residual};
  return mlp_impl(a, tinyinfer::kStageDown, path, stream);
}

int tinyinfer_mxfp4_dequant(const uint8_t* packed, const uint8_t* scale, size_t rows, size_t k,
                            void* out, int out_dtype, void* stream) {
  if (!packed || !scale || !out) return TI_ERR_INVALID_ARG;
  if (k % 32 != 0) return TI_ERR_BAD_SHAPE;
  if (out_dtype != TI_DTYPE_F32 && out_dtype != TI_DTYPE_BF16) return TI_ERR_BAD_DTYPE;
  if (rows > kMaxDim || k > kMaxDim) return TI_ERR_TOO_LARGE;
  int st = check_device();
  if (st != TI_OK) return st;
  return to_status(tinyinfer::launch_dequant(packed, scale, (int64_t)rows, (int64_t)k, out, out_dtype,
                                             static_cast<hipStream_t>(stream)));
}

int tinyinfer_mxfp4_quantize(const void* w, int in_dtype, size_t rows, size_t k, uint8_t* packed,
                             uint8_t* scale, uint32_t* flags, void* stream) {
  if (!w || !packed || !scale || !flags) return TI_ERR_INVALID_ARG;
  if (k % 32 != 0) return TI_ERR_BAD_SHAPE;
  if (in_dtype != TI_DTYPE_F32 && in_dtype != TI_DTYPE_BF16 && in_dtype != TI_DTYPE_F16)
    return TI_ERR_BAD_DTYPE;
  if (rows > kMaxDim || k > kMaxDim) return TI_ERR_TOO_LARGE;
  int st = check_device();
  if (st != TI_OK) return st;
  return to_status(tinyinfer::launch_quantize(w, in_dtype, (int64_t)rows, (int64_t)k, packed, scale,
                                              flags, static_cast<hipStream_t>(stream)));
}

const char* tinyinfer_mxfp4_status_string(int status) {
  switch (status) {
    case TI_OK: return "ok";
    case TI_ERR_INVALID_ARG: return "invalid argument";
    case TI_ERR_BAD_SHAPE: return "hidden_dim and intermediate must be divisible by 32";
    case TI_ERR_BAD_DTYPE: return "unsupported dtype";
    case TI_ERR_HIP: return "HIP runtime error";
    case TI_ERR_NO_DEVICE: return "no gfx950 (MI355X) device is current";
    case TI_ERR_TOO_LARGE: return "size exceeds kernel limits";
    case TI_ERR_MISALIGNED: return "activation, weight and tmp pointers must be 16-byte aligned";
    case TI_ERR_UNSUPPORTED: return "the requested kernel path does not support this call";
    case TI_ERR_SCRATCH: return "the call needs more scratch memory than the no-alloc entry point's fixed buffer holds";
    default: return "unknown status";
  }
}

int tinyinfer_mxfp4_diagnostics(uint32_t* decode_barrier_timeouts) {
  if (!decode_barrier_timeouts) return TI_ERR_INVALID_ARG;
  const int st = check_device();
  if (st != TI_OK) return st;
  const unsigned int v = tinyinfer::decode_barrier_timeouts();
  if (v == 0xffffffffu) return TI_ERR_HIP;
  *decode_barrier_timeouts = v;
  return TI_OK;
}

int tinyinfer_mxfp4_decode_reset(void) {
  const int st = check_device();
  if (st != TI_OK) return st;
  return to_status(tinyinfer::decode_reset());
}

int tinyinfer_mxfp4_set_option(const char* name, int value) {
  return tinyinfer::set_option(name, value) ? TI_OK : TI_ERR_INVALID_ARG;
}

int tinyinfer_mxfp4_get_option(const char* name, int* value) {
  return tinyinfer::get_option(name, value) ? TI_OK : TI_ERR_INVALID_ARG;
}

int tinyinfer_mxfp4_workspace_info(size_t* bytes_held, size_t* limit_bytes) {
  if (!bytes_held || !limit_bytes) return TI_ERR_INVALID_ARG;
  *bytes_held = tinyinfer::workspace_bytes_held();
  *limit_bytes = tinyinfer::workspace_limit();
  return TI_OK;
}

int tinyinfer_mxfp4_release_workspaces(void) { return to_status(tinyinfer::release_workspaces()); }

int tinyinfer_mxfp4_abi_version(void) { return 7; }

}  // extern "C"
