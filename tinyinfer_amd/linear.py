"""MXFP4 linear parameter container.

Same parameters, shapes, dtypes and assertion as the reference's
``LinearMXFP4`` (tinyinfer/layers/linear.py:36-48): ``weight_packed`` uint8
``[out, in/2]`` (two e2m1 codes per byte, first element in the low nibble)
and ``weight_scale`` uint8 ``[out, in/32]`` (e8m0 byte per 32 input
features), both frozen.  The MLP consumes the tensors directly; ``forward``
(which the reference's class lacks) runs the layer as a plain linear on the
MXFP4 kernels.
"""

import torch
from torch import nn


class LinearMXFP4(nn.Module):
    def __init__(self, in_features: int, out_features: int, bias: bool = False, dtype=None, device=None):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        assert in_features % 32 == 0
        self.weight_packed = nn.Parameter(
            torch.empty(out_features, in_features // 2, dtype=torch.uint8, device=device), requires_grad=False)
        self.weight_scale = nn.Parameter(
            torch.empty(out_features, in_features // 32, dtype=torch.uint8, device=device), requires_grad=False)
        if bias:
            self.bias = nn.Parameter(torch.empty(out_features, dtype=dtype, device=device))
        else:
            self.register_parameter("bias", None)

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None) -> torch.Tensor:
        """``x @ dequant(W)^T`` (+ ``bias``, + ``residual``) on the MXFP4
        kernels, for the dense linears the reference runs with ``F.linear``
        (tinyinfer/layers/linear.py:19-21) when their weights are kept in
        MXFP4.  ``x`` is [..., in_features] bf16/fp16 on the GPU."""
        from .extension import load_extension
        shape = x.shape
        y = load_extension().mxfp4_linear(x.reshape(-1, self.in_features).contiguous(), self.weight_packed,
                                          self.weight_scale,
                                          None if residual is None else residual.reshape(-1, self.out_features).contiguous())
        if self.bias is not None:
            y = y + self.bias
        return y.reshape(*shape[:-1], self.out_features)
