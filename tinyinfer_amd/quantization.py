"""Device MXFP4 quantization and the checkpoint format record.

``quantize_chunk`` / ``dequantize_chunk`` have the reference's names,
arguments, return values and ``ValueError`` cases
(tinyinfer/quantization/quantize_mxfp4.py:28-85), but run the HIP kernels on
the GPU: the tensor goes to the current device when it is on the CPU, and the
results come back on the input's device.  The bytes are identical to the
reference's.

``QUANT_CONFIG`` holds the format-describing fields of the
``quantization_config.json`` record that the reference writes
(quantize_mxfp4.py:233-253). Both share one format, so the records match.
"""

from __future__ import annotations

import torch

from .extension import load_extension

QUANT_CONFIG = {
    "format": "tinyinfer_mxfp4_weight_only_v1",
    "quantization": "mxfp4",
    "target_modules": ["mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"],
    "block_size": 32,
    "axis": "input_features_last_dim",
    "value_format": "fp4_e2m1",
    "scale_format": "e8m0",
    "scale_selection": "ceil_log2_amax_over_6",
    "rounding": "nearest_ties_to_even",
    "packed_dtype": "uint8",
    "packed_nibble_order": "first_element_low_nibble",
    "scale_dtype": "uint8_raw_e8m0_exponent",
    "scale_encoding": "stored_byte = unbiased_exponent + 127",
    "weight_key_suffixes": ["weight_packed", "weight_scale"],
}

_QFLAG_NONFINITE = 1
_QFLAG_EXP_RANGE = 2


def _to_device(t: torch.Tensor) -> torch.Tensor:
    if t.is_cuda:
        return t
    if not torch.cuda.is_available():
        raise RuntimeError("tinyinfer_amd quantization needs a gfx950 GPU; no device is visible")
    return t.to("cuda")


def quantize_chunk(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """[rows, K] fp32/bf16/fp16 -> (packed uint8 [rows, K/2], scale uint8 [rows, K/32])."""
    if weight.ndim != 2 or weight.shape[1] % 32:
        raise ValueError(f"expected [rows,K], K multiple of 32; got {tuple(weight.shape)}")
    w = _to_device(weight)
    if w.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        w = w.to(torch.float32)
    packed, scale, flags = load_extension().mxfp4_quantize(w.contiguous())
    f = int(flags.item())  # synchronizes: the reference raises synchronously too
    if f & _QFLAG_NONFINITE:
        raise ValueError("non-finite weights (NaN/Inf) are not supported")
    if f & _QFLAG_EXP_RANGE:
        raise ValueError("E8M0 exponent out of representable range [-127,127]")
    return packed.to(weight.device), scale.to(weight.device)


def dequantize_chunk(packed: torch.Tensor, scale_bits: torch.Tensor, out_dtype=torch.float32) -> torch.Tensor:
    """Decode to ``out_dtype`` (float32 or bfloat16, both exact) [rows, K]."""
    if packed.ndim != 2 or scale_bits.ndim != 2 or packed.shape[0] != scale_bits.shape[0]:
        raise ValueError("packed/scale shape mismatch")
    k = packed.shape[1] * 2
    if k % 32 or scale_bits.shape[1] != k // 32:
        raise ValueError("scale shape mismatch")
    p, s = _to_device(packed).contiguous(), _to_device(scale_bits).contiguous()
    if bool((s == 255).any()):
        raise ValueError("E8M0 NaN scale detected (255)")
    out = load_extension().mxfp4_dequant(p, s, out_dtype)
    return out.to(packed.device)
