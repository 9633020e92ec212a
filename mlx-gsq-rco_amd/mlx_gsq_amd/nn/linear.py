"""Packed mixed-quant linear layer (torch.nn.Module).

Drop-in counterpart of mlx_gsq/nn/linear.py:6-24 ``GSQLinear``: built from a
``PackedWeight``, it keeps the untouched GGUF payload resident on the device and exposes
``packed_weight``, ``in_features``, ``out_features`` and ``qtype``. A single activation
row goes to the fused QMV, more rows to the tiled QMM, as in the reference; the optional
bias is added afterwards.
"""
from __future__ import annotations

import torch

from ..runtime.kernels.qmm import quantized_matmul
from ..runtime.kernels.qmv import quantized_matvec


class GSQLinear(torch.nn.Module):
    def __init__(self, weight, bias=None):
        super().__init__()
        self.packed_weight = weight.data
        self.bias = bias
        self.in_features = weight.logical_shape[1]
        self.out_features = weight.logical_shape[0]
        self.qtype = weight.quantization_type

    def forward(self, x):
        rows = x.numel() // self.in_features
        if rows == 1:
            y = quantized_matvec(x, self.packed_weight, qtype=self.qtype,
                                 out_features=self.out_features, in_features=self.in_features)
        else:
            y = quantized_matmul(x, self.packed_weight, qtype=self.qtype,
                                 out_features=self.out_features, in_features=self.in_features)
        return y if self.bias is None else y + self.bias

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, qtype={self.qtype}"
