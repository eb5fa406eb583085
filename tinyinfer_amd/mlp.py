"""Qwen3 MLP block with the MXFP4 weight-only path.

Mirrors the reference's ``Qwen3MLP`` (tinyinfer/models/qwen3.py:138-177):
``gate_proj``/``up_proj`` are ``LinearMXFP4(hidden, intermediate)``,
``down_proj`` is ``LinearMXFP4(intermediate, hidden)``, and ``forward``
passes the seven tensors to ``mlp_forward_mxfp4`` in the reference's order.
Only ``quantization == "mxfp4"`` is in scope here; the dense path of the
reference (``_C.mlp_forward``) is not part of this package, so other values
raise ``NotImplementedError``.
"""

from types import SimpleNamespace

import torch
from torch import nn

from .extension import load_extension
from .linear import LinearMXFP4


class Qwen3MLP(nn.Module):
    def __init__(self, config, quantization=None):
        super().__init__()
        self.quantization = quantization
        if quantization != "mxfp4":
            raise NotImplementedError("tinyinfer_amd implements only quantization='mxfp4'")
        self.gate_proj = LinearMXFP4(config.hidden_size, config.intermediate_size, bias=False)
        self.up_proj = LinearMXFP4(config.hidden_size, config.intermediate_size, bias=False)
        self.down_proj = LinearMXFP4(config.intermediate_size, config.hidden_size, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # [num_flat_tokens, hidden] -> [num_flat_tokens, hidden]
        return load_extension().mlp_forward_mxfp4(
            x,
            self.gate_proj.weight_packed, self.gate_proj.weight_scale,
            self.up_proj.weight_packed, self.up_proj.weight_scale,
            self.down_proj.weight_packed, self.down_proj.weight_scale,
        )


def qwen3_config(hidden_size: int, intermediate_size: int):
    """Minimal stand-in for the HF config fields Qwen3MLP reads."""
    return SimpleNamespace(hidden_size=hidden_size, intermediate_size=intermediate_size)
