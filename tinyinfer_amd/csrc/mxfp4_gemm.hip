// Tiled MXFP4 MLP path for prefill / mixed batches: placeholder that routes
// to the skinny kernels until the LDS-tiled MFMA GEMM lands.
#include "mxfp4_common.hpp"
#include "mxfp4_launch.hpp"

namespace tinyinfer {

hipError_t launch_gemm_mlp(const MlpArgs& a, hipStream_t stream) { return launch_skinny_mlp(a, stream); }

}  // namespace tinyinfer
