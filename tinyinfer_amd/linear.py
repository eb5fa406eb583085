"""MXFP4 linear parameter container.

Same parameters, shapes, dtypes and assertion as the reference's
``LinearMXFP4`` (tinyinfer/layers/linear.py:36-48): ``weight_packed`` uint8
``[out, in/2]`` (two e2m1 codes per byte, first element in the low nibble)
and ``weight_scale`` uint8 ``[out, in/32]`` (e8m0 byte per 32 input
features), both frozen.  Like the reference it has no ``forward``; the MLP
consumes the tensors directly.
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
