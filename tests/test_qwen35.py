"""Qwen3.5-hybrid decode step around the GEMVs (mlx_gsq/models/qwen35.py:48-152) against
transformers' Qwen3.5 text model on a tiny synthetic checkpoint (tests/qwen35_fixture.py).

CPU: the decoder's structure (GatedDeltaNet with the GGUF head routing, gated attention with
partial RoPE, norms, MLP, caches) in float32 with dense stand-ins for the packed layers: prefill
of a whole prompt and token-by-token decoding against HF's full-sequence logits, rel-L2 <= 1e-4.
GPU: the same model on GSQLinear / GSQEmbedding (the HIP kernels) with fp16 activations,
rel-L2 <= 2e-2 against HF's float32 logits, and the HIP-graph decode step equal to the eager
one on every step.
"""
import numpy as np
import pytest
import torch

from mlx_gsq_amd import tables
from mlx_gsq_amd.models import build_qwen35
from qwen35_fixture import ARGS, TABLES, TinyStore, dense_factories, hf_logits, hf_model, rel_l2

IDS = [17, 301, 5, 77, 402, 9, 256, 130]


@pytest.fixture(scope="module")
def store_and_ref():
    store = TinyStore("cpu", seed=1)
    return store, hf_logits(hf_model(store), IDS)


def test_cpu_prefill_and_decode_match_hf(store_and_ref):
    store, ref = store_and_ref
    linear, embedding = dense_factories(store)
    model = build_qwen35(store, dtype=torch.float32, args=ARGS, linear=linear, embedding=embedding)
    with torch.no_grad():
        cache = model.new_cache(batch=1, max_len=16)
        pre = model(torch.tensor([IDS]), cache)
        assert rel_l2(pre.numpy(), ref.numpy()) <= 1e-4
        cache = model.new_cache(batch=1, max_len=16)
        steps = [model(torch.tensor([[t]]), cache) for t in IDS]
        dec = torch.cat(steps, dim=1)
        assert rel_l2(dec.numpy(), ref.numpy()) <= 1e-4
        # prefill of a prefix, then decoding the rest, continues the same sequence
        cache = model.new_cache(batch=1, max_len=16)
        head = model(torch.tensor([IDS[:5]]), cache)
        tail = [model(torch.tensor([[t]]), cache) for t in IDS[5:]]
        both = torch.cat([head, *tail], dim=1)
        assert rel_l2(both.numpy(), ref.numpy()) <= 1e-4
        assert cache.length == len(IDS) and int(cache.pos) == len(IDS)
        with pytest.raises(ValueError):
            model(torch.tensor([[1] * 9]), cache)  # 8 + 9 > 16 positions


def test_cpu_head_routing_is_cyclic(store_and_ref):
    """With value heads routed by h // 2 (mlx-lm's generic grouping) instead of h % 2 the
    result differs from HF-with-permuted-heads: the check above is sensitive to the routing."""
    store, ref = store_and_ref
    linear, embedding = dense_factories(store)
    model = build_qwen35(store, dtype=torch.float32, args=ARGS, linear=linear, embedding=embedding)
    orig = torch.Tensor.repeat

    def grouped(self, *sizes):
        if self.dim() == 4 and len(sizes) == 4 and sizes[2] > 1:  # (B, S, Hk, d) -> interleaved
            return self.repeat_interleave(sizes[2], dim=2)
        return orig(self, *sizes)
    torch.Tensor.repeat = grouped
    try:
        with torch.no_grad():
            out = model(torch.tensor([IDS]), model.new_cache(batch=1, max_len=16))
    finally:
        torch.Tensor.repeat = orig
    assert rel_l2(out.numpy(), ref.numpy()) > 1e-2


@pytest.mark.gpu
def test_gpu_decode_matches_hf_and_graph_replays(store_and_ref):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from mlx_gsq_amd.models import GraphDecoder
    _, ref = store_and_ref
    tables.set_tables(TABLES)
    dev = torch.device("cuda:0")
    store = TinyStore(dev, seed=1)
    model = build_qwen35(store, dtype=torch.float16, args=ARGS)
    ids = torch.tensor([IDS], device=dev)
    with torch.no_grad():
        pre = model(ids, model.new_cache(batch=1, max_len=16)).float().cpu()
        assert torch.isfinite(pre).all()
        assert rel_l2(pre.numpy(), ref.numpy()) <= 2e-2
        cache = model.new_cache(batch=1, max_len=16)
        eager = torch.cat([model(ids[:, i:i + 1], cache) for i in range(len(IDS))], dim=1).float().cpu()
        assert rel_l2(eager.numpy(), ref.numpy()) <= 2e-2
        cache = model.new_cache(batch=1, max_len=16)
        dec = GraphDecoder(model, cache)
        for i in range(len(IDS)):
            out = dec.step(ids[:, i:i + 1]).float().cpu()
            assert torch.equal(out[0, 0], eager[0, i]), i
        assert cache.length == len(IDS)
