"""Packed mixed-quant linear layer (torch.nn.Module).

Drop-in counterpart of mlx_gsq/nn/linear.py:6-24 ``GSQLinear``: built from a
``PackedWeight``, it keeps the untouched GGUF payload resident on the device and exposes
``packed_weight``, ``in_features``, ``out_features`` and ``qtype``. The reference sends one
activation row to the fused QMV and every larger batch to the tiled QMM; here batches below
the QMM threshold (``QMM_MIN_ROWS`` rows) go through ``quantized_matvec``, whose routing
keeps them on the matrix-vector kernels (one or two rows on the vector kernel, 3-7 fp16 rows on
the quad-row kernel) except the fp16 batches of matrices of 2^26+ weights that the small-batch
QMM computes faster on gfx950 (from 5 rows when K > 8192, from 7 otherwise); from the threshold
on, QMM. The results agree
with the reference's within the operators' tolerances either way. The optional bias is
added afterwards.
"""
from __future__ import annotations

import torch

from ..runtime.kernels.qmm import QMM_MIN_ROWS, quantized_matmul
from ..runtime.kernels.qmv import quantized_matvec, quantized_matvec_group2, quantized_matvec_pre


def _apply(x, packed, qtype, out_features, in_features):
    """One packed product, routed by batch size (see the module docstring)."""
    rows = x.numel() // in_features
    fn = quantized_matvec if rows < QMM_MIN_ROWS else quantized_matmul
    return fn(x, packed, qtype=qtype, out_features=out_features, in_features=in_features)


class GSQLinear(torch.nn.Module):
    def __init__(self, weight, bias=None):
        super().__init__()
        self.packed_weight = weight.data
        self.bias = bias
        self.in_features = weight.logical_shape[1]
        self.out_features = weight.logical_shape[0]
        self.qtype = weight.quantization_type

    def forward(self, x):
        y = _apply(x, self.packed_weight, self.qtype, self.out_features, self.in_features)
        return y if self.bias is None else y + self.bias

    def forward_pre(self, x, pre, **kw):
        """The product of one fp16 row the kernel forms itself from ``x`` (``pre`` =
        "add_rms_norm" or "swiglu", keywords as ``quantized_matvec_pre``)."""
        y = quantized_matvec_pre(x, self.packed_weight, qtype=self.qtype, out_features=self.out_features,
                                 in_features=self.in_features, pre=pre, **kw)
        return y if self.bias is None else y + self.bias

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, qtype={self.qtype}"


class GSQFusedLinear(torch.nn.Module):
    """Several packed linears of one quantization type and input width applied to the same
    input in one launch (q/k, gate/up of a decoder layer).

    Packed rows are whole superblocks, row-major, so concatenating the matrices along the
    output dimension is a byte concatenation; it is done once here, on the weights' device.
    ``forward`` returns one output per weight (views of one result), or with ``concat=True`` the
    one tensor of all outputs side by side, computed exactly as ``GSQLinear`` computes the
    concatenated matrix. No counterpart in the reference, whose model applies each projection
    on its own.
    """

    def __init__(self, weights, biases=None, concat=False):
        super().__init__()
        weights = list(weights)
        if not weights:
            raise ValueError("no weights to fuse")
        self.concat = concat
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
        return self._outputs(_apply(x, self.packed_weight, self.qtype, self.out_features, self.in_features))

    def forward_pre(self, x, pre, **kw):
        """As ``forward``, on one fp16 row the kernel forms itself from ``x`` (``pre`` =
        "add_rms_norm" or "swiglu", keywords as ``quantized_matvec_pre``)."""
        return self._outputs(quantized_matvec_pre(x, self.packed_weight, qtype=self.qtype,
                                                  out_features=self.out_features, in_features=self.in_features,
                                                  pre=pre, **kw))

    def _outputs(self, y):
        if self.concat:  # one tensor of the concatenated outputs
            if self.biases is not None:
                y = y + torch.cat([torch.zeros(n, dtype=y.dtype, device=y.device) if b is None else b
                                   for n, b in zip(self.splits, self.biases)])
            return y
        outs = y.split(self.splits, dim=-1)
        if self.biases is None:
            return outs
        return tuple(o if b is None else o + b for o, b in zip(outs, self.biases))

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, splits={self.splits}, qtype={self.qtype}"


class GSQGroupedLinear(torch.nn.Module):
    """Projections of one input whose weights differ in quantization type (q/k/v of a decoder
    layer: IQ2_XS, IQ2_XS, IQ4_XS), applied as one group: the weights of each type are fused
    (``GSQFusedLinear``), and one fp16 row over two types goes out as one launch
    (``quantized_matvec_group2``), else one launch per type. ``forward`` returns one output per
    weight, in the order given, each within the QMV tolerance of the one ``GSQFusedLinear``
    gives for its type's weights. The launches stay on the current stream: as parallel branches of a
    captured HIP graph (side streams forked from and joined into the current stream) the
    64-layer decode stack ran 16% slower than with the launches in sequence (4.91 against 4.24
    ms per token). No counterpart in the reference, whose model applies each projection on its
    own.
    """

    def __init__(self, weights, biases=None):
        super().__init__()
        weights = list(weights)
        if not weights:
            raise ValueError("no weights to group")
        widths = {w.logical_shape[1] for w in weights}
        if len(widths) != 1:
            raise ValueError(f"grouped weights must share one input width, got {sorted(widths)}")
        if biases is not None and len(biases) != len(weights):
            raise ValueError("one bias (or None) per weight")
        self.in_features = weights[0].logical_shape[1]
        order = []  # quantization types in order of first appearance
        for w in weights:
            if w.quantization_type not in order:
                order.append(w.quantization_type)
        # parts[i] computes the weights slots[i] (indices into the given order)
        self.slots = [[j for j, w in enumerate(weights) if w.quantization_type == q] for q in order]
        self.parts = torch.nn.ModuleList(
            GSQFusedLinear([weights[j] for j in slot],
                           None if biases is None else [biases[j] for j in slot]) for slot in self.slots)
        self.out_features = [w.logical_shape[0] for w in weights]

    def forward(self, x):
        outs = [None] * len(self.out_features)
        if len(self.parts) == 2 and x.numel() == self.in_features and x.dtype == torch.float16:
            # one row, two types: both fused parts in one launch
            p0, p1 = self.parts
            y0, y1 = quantized_matvec_group2(x, p0.packed_weight, p1.packed_weight, qtypes=(p0.qtype, p1.qtype),
                                             out_features=(p0.out_features, p1.out_features),
                                             in_features=self.in_features)
            results = (p0._outputs(y0), p1._outputs(y1))
        else:
            results = tuple(part(x) for part in self.parts)
        for slot, res in zip(self.slots, results):
            for j, r in zip(slot, res):
                outs[j] = r
        return tuple(outs)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, " \
               f"qtypes={[p.qtype for p in self.parts]}"
