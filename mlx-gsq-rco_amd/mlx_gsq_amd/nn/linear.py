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


class GSQFusedLinear(torch.nn.Module):
    """Several packed linears of one quantization type and input width applied to the same
    input in one launch (q/k, gate/up of a decoder layer).

    Packed rows are whole superblocks, row-major, so concatenating the matrices along the
    output dimension is a byte concatenation; it is done once here, on the weights' device.
    ``forward`` returns one output per weight (views of one result), computed exactly as
    ``GSQLinear`` computes the concatenated matrix (one row → QMV, more → QMM). No counterpart
    in the reference, whose model applies each projection on its own.
    """

    def __init__(self, weights, biases=None):
        super().__init__()
        weights = list(weights)
        if not weights:
            raise ValueError("no weights to fuse")
        qtypes = {w.quantization_type for w in weights}
        widths = {w.logical_shape[1] for w in weights}
        if len(qtypes) != 1:
            raise ValueError(f"fused weights must share one quantization type, got {sorted(qtypes)}")
        if len(widths) != 1:
            raise ValueError(f"fused weights must share one input width, got {sorted(widths)}")
        if biases is not None and len(biases) != len(weights):
            raise ValueError("one bias (or None) per weight")
        self.qtype = weights[0].quantization_type
        self.in_features = weights[0].logical_shape[1]
        self.splits = [w.logical_shape[0] for w in weights]
        self.out_features = sum(self.splits)
        self.packed_weight = torch.cat([torch.as_tensor(w.data).reshape(-1) for w in weights])
        self.biases = biases

    def forward(self, x):
        rows = x.numel() // self.in_features
        if rows == 1:
            y = quantized_matvec(x, self.packed_weight, qtype=self.qtype,
                                 out_features=self.out_features, in_features=self.in_features)
        else:
            y = quantized_matmul(x, self.packed_weight, qtype=self.qtype,
                                 out_features=self.out_features, in_features=self.in_features)
        outs = y.split(self.splits, dim=-1)
        if self.biases is None:
            return outs
        return tuple(o if b is None else o + b for o, b in zip(outs, self.biases))

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, splits={self.splits}, qtype={self.qtype}"

