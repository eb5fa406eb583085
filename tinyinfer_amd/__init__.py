"""MI355X-native (gfx950) MXFP4 weight-only Qwen3 MLP.

Drop-in for tinyInfer's ``--quantization mxfp4`` MLP path:

* ``tinyinfer_amd._C.mlp_forward_mxfp4(X, gate, gate_scale, up, up_scale,
  down, down_scale)`` -- same signature and checks as the reference's
  ``tinyinfer._C.mlp_forward_mxfp4`` (reference tinyinfer/csrc/bind.cpp:656-882).
* ``tinyinfer_amd.extension.load_extension()`` -- same contract as the
  reference's loader (tinyinfer/utils/extension.py:4-14).
* ``tinyinfer_amd.linear.LinearMXFP4`` and ``tinyinfer_amd.mlp.Qwen3MLP`` --
  same parameters and forward dispatch as the reference
  (tinyinfer/layers/linear.py:36-48, tinyinfer/models/qwen3.py:138-177).
* ``tinyinfer_amd.capi`` -- ctypes binding of the C ABI in
  ``include/tinyinfer_mxfp4.h``.

The kernels are hand-written HIP for gfx950; there is no CPU fallback.
"""

__all__ = ["extension", "capi", "linear", "mlp", "quantization", "workloads"]
