// The allocation-free MLP entry point (tinyinfer_mlp_forward_mxfp4_noalloc).
//
// For callers that cannot allocate device memory: code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc.  The
// split-K partial sums of the tile and GEMM kernels go to `scratch`, a
// fixed device array of this file (every device the library runs on holds
// its own copy until the process ends), instead of the library's
// per-stream workspace.  No hipMalloc, hipFree or allocating library routine
// is called on this path.
//
// What the kernels keep in scratch: fp32 partial tiles, each written in full
// by the launch that later reads it, so nothing in it must start at zero and
// calls need not clear it.  Every call on a device shares that device's
// array: calls that overlap on one device (other streams, other threads,
// concurrent graph replays) race on it and must not run at the same time.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/tinyinfer_mxfp4.h"
#include "mxfp4_launch.hpp"

namespace {

// 64 MiB: the largest split-K need of the tile kernels on the Qwen3 MLP
// shapes (Qwen3-32B gate_up at 64 tokens: 5 K ranges x 64 tokens x 2 x 25600
// rows x 4 bytes = 62.5 MiB); the GEMM path splits K only as far as it fits.
constexpr size_t kScratchBytes = size_t(64) << 20;
static __device__ __attribute__((aligned(256))) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::once_flag g_once[kMaxDevices];
float* g_ptr[kMaxDevices];       // device address of `scratch` on each device
hipError_t g_err[kMaxDevices];

// The device address of this device's scratch array (looked up once per
// device, with the device current); null on failure.
float* scratch_ptr(int dev) {
  std::call_once(g_once[dev], [dev] {
    void* p = nullptr;
    g_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_ptr[dev] = g_err[dev] == hipSuccess ? static_cast<float*>(p) : nullptr;
    if (g_err[dev] != hipSuccess) (void)hipGetLastError();
  });
  return g_ptr[dev];
}

}  // namespace

extern "C" int tinyinfer_mlp_forward_mxfp4_noalloc(const void* X, const uint8_t* gate, const uint8_t* gate_scale,
                                                   const uint8_t* up, const uint8_t* up_scale, const uint8_t* down,
                                                   const uint8_t* down_scale, size_t N, size_t hidden_dim,
                                                   size_t intermediate, void* tmp, void* O, int dtype_code,
                                                   void* stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return TI_ERR_NO_DEVICE;
  if (N > (size_t)INT64_MAX || hidden_dim > (size_t)INT64_MAX || intermediate > (size_t)INT64_MAX)
    return TI_ERR_TOO_LARGE;
  tinyinfer::MlpArgs a{X, gate, gate_scale, up, up_scale, down, down_scale, (int64_t)N, (int64_t)hidden_dim,
                       (int64_t)intermediate, tmp, O, dtype_code};
  float* p = scratch_ptr(dev);
  if (!p) return TI_ERR_HIP;
  a.ws = p;
  a.ws_bytes = kScratchBytes;
  // run_mlp refuses (TI_ERR_SCRATCH) a call of up to 64 tokens whose tile
  // kernels would need more than kScratchBytes, rather than allocate or
  // change kernels behind the caller (from 65 tokens such a call takes the
  // GEMM path); the GEMM path splits K only as far as scratch holds
  return tinyinfer::run_mlp(a, tinyinfer::kStageBoth, TI_PATH_AUTO, stream);
}
