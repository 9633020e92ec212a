"""Packed embedding layer (torch.nn.Module).

Drop-in counterpart of mlx_gsq/nn/embedding.py:4-11 ``GSQEmbedding``: built from an IQ2_S
``PackedWeight`` (any other type raises ``NotImplementedError``), it keeps the packed table on
the device and exposes ``packed_weight``, ``num_embeddings``, ``dimensions`` and ``dtype``.
"""
from __future__ import annotations

import torch

from ..runtime.kernels.embedding import iq2_s_embedding


class GSQEmbedding(torch.nn.Module):
    def __init__(self, weight, dtype=None):
        super().__init__()
        if weight.quantization_type != "IQ2_S":
            raise NotImplementedError(weight.quantization_type)
        self.packed_weight = weight.data
        self.num_embeddings = weight.logical_shape[0]
        self.dimensions = weight.logical_shape[1]
        self.dtype = dtype

    def forward(self, ids):
        return iq2_s_embedding(ids, self.packed_weight, vocab_size=self.num_embeddings,
                               dimensions=self.dimensions, dtype=self.dtype)

    def extra_repr(self) -> str:
        return f"num_embeddings={self.num_embeddings}, dimensions={self.dimensions}, qtype=IQ2_S"
