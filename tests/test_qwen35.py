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
    linear, fused, embedding = dense_factories(store)
    model = build_qwen35(store, dtype=torch.float32, args=ARGS, linear=linear, fused=fused, embedding=embedding)
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
    linear, fused, embedding = dense_factories(store)
    model = build_qwen35(store, dtype=torch.float32, args=ARGS, linear=linear, fused=fused, embedding=embedding)
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


@pytest.mark.gpu
def test_gpu_batched_decode_matches_single_sequences():
    """Two sequences decoded together (two-row projections, the step kernels over a batch, one
    HIP graph per step) give each sequence's own single-sequence logits (prefill of 4 tokens,
    then 4 decode steps)."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from mlx_gsq_amd.models import GraphDecoder
    tables.set_tables(TABLES)
    dev = torch.device("cuda:0")
    model = build_qwen35(TinyStore(dev, seed=1), dtype=torch.float16, args=ARGS)
    seqs = [IDS, [3, 14, 15, 92, 65, 35, 89, 79]]
    with torch.no_grad():
        singles = []
        for sq in seqs:
            cache = model.new_cache(batch=1, max_len=16)
            ids = torch.tensor([sq], device=dev)
            outs = [model(ids[:, :4], cache)] + [model(ids[:, i:i + 1], cache) for i in range(4, 8)]
            singles.append(torch.cat(outs, dim=1).float().cpu())
        cache = model.new_cache(batch=2, max_len=16)
        ids = torch.tensor(seqs, device=dev)
        outs = [model(ids[:, :4], cache)]
        dec = GraphDecoder(model, cache, batch=2)
        outs += [dec.step(ids[:, i:i + 1]).clone() for i in range(4, 8)]
        both = torch.cat(outs, dim=1).float().cpu()
    assert torch.isfinite(both).all()
    for b in range(2):
        assert rel_l2(both[b].numpy(), singles[b][0].numpy()) <= 1e-2, b


class _Given(torch.nn.Module):
    """Stands in for a projection: returns the tensor set for the current step."""

    def __init__(self):
        super().__init__()
        self.value = None

    def forward(self, x):
        return self.value


@pytest.mark.gpu
def test_gpu_fused_ops_match_torch_formulation():
    """The fused kernels (add + RMSNorm, SwiGLU, GatedDeltaNet token and sequence) against the
    model's torch formulation run on the CPU in float32, at the 27B head shapes (16 key / 48
    value heads of 128, conv 4): 3 single tokens, then sequences of 5 and 2 tokens, for 2 batch
    rows."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from mlx_gsq_amd.models.qwen35 import GatedDeltaNet, Qwen35Args, Qwen35Cache, rms_norm
    from mlx_gsq_amd.runtime.kernels import model_ops
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(5)
    # add + RMSNorm and SwiGLU
    x = torch.randn(3, 5120, generator=g).half()
    d = torch.randn(3, 5120, generator=g).half()
    w = (1 + 0.1 * torch.randn(5120, generator=g)).half()
    xg = x.to(dev)
    y = model_ops.add_rms_norm(xg, d.to(dev), w.to(dev), 1e-6).cpu()
    xs = x + d
    assert torch.equal(xg.cpu(), xs)
    assert rel_l2(y.float().numpy(), rms_norm(xs.float(), w.float(), 1e-6).numpy()) <= 1e-3
    gu = torch.randn(3, 2, 1024, generator=g).half()
    s = model_ops.swiglu(gu.to(dev)).cpu()
    want = torch.nn.functional.silu(gu[..., :512].float()) * gu[..., 512:].float()
    assert rel_l2(s.float().numpy(), want.numpy()) <= 1e-3
    # GatedDeltaNet token steps
    a = Qwen35Args(num_hidden_layers=1)
    B, C, hv = 2, a.conv_dim, a.linear_num_value_heads
    params = dict(w_a=torch.randn(hv, 64, generator=g) / 8, w_b=torch.randn(hv, 64, generator=g) / 8,
                  conv_w=0.5 * torch.randn(C, 4, generator=g), ssm_a=-torch.rand(hv, generator=g) * 8 - 1,
                  dt_bias=torch.randn(hv, generator=g), norm_w=1 + 0.1 * torch.randn(a.linear_value_head_dim, generator=g))

    def module(device, dtype):
        p = {k: (v.to(device, dtype) if k not in ("ssm_a", "dt_bias") else v.to(device)) for k, v in params.items()}
        m = GatedDeltaNet(a, 0, _Given(), torch.nn.Identity(), p["w_a"], p["w_b"], p["conv_w"], p["ssm_a"],
                          p["dt_bias"], p["norm_w"])
        return m, Qwen35Cache(a, B, 8, device, dtype)
    cpu, ccache = module("cpu", torch.float32)
    gpu, gcache = module(dev, torch.float16)
    for t in range(3):
        qkv = torch.randn(B, 1, C, generator=g).half()
        z = torch.randn(B, 1, a.value_dim, generator=g).half()
        h = torch.randn(B, 1, 64, generator=g).half()
        cpu.in_proj_qkvz.value = torch.cat([qkv, z], dim=-1).float()
        gpu.in_proj_qkvz.value = torch.cat([qkv, z], dim=-1).to(dev)
        want = cpu(h.float(), ccache)
        got = gpu(h.to(dev), gcache).float().cpu()
        assert torch.isfinite(got).all()
        assert rel_l2(got.numpy(), want.numpy()) <= 5e-3, t
        assert rel_l2(gcache.rec[0].cpu().numpy(), ccache.rec[0].numpy()) <= 1e-3, t
        assert torch.equal(gcache.conv[0].cpu().float(), ccache.conv[0])
    # then a 5-token sequence at once (the prefill kernels: a / b by one product, the recurrence
    # over all tokens in one launch), and a 2-token one (shorter than the convolution window)
    for S in (5, 2):
        qkv = torch.randn(B, S, C, generator=g).half()
        z = torch.randn(B, S, a.value_dim, generator=g).half()
        h = torch.randn(B, S, 64, generator=g).half()
        cpu.in_proj_qkvz.value = torch.cat([qkv, z], dim=-1).float()
        gpu.in_proj_qkvz.value = torch.cat([qkv, z], dim=-1).to(dev)
        want = cpu(h.float(), ccache)
        got = gpu(h.to(dev), gcache).float().cpu()
        assert torch.isfinite(got).all()
        assert rel_l2(got.numpy(), want.numpy()) <= 5e-3, S
        assert rel_l2(gcache.rec[0].cpu().numpy(), ccache.rec[0].numpy()) <= 1e-3, S
        assert torch.equal(gcache.conv[0].cpu().float(), ccache.conv[0]), S


@pytest.mark.gpu
def test_gpu_attention_decode_matches_torch_formulation():
    """The fused single-token attention against the torch formulation (CPU, float32) at the 27B
    head shapes (24 query / 4 KV heads of 256, rotary 64) over 5 positions of 2 batch rows,
    caches included."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from mlx_gsq_amd.models.qwen35 import FullAttention, Qwen35Args, Qwen35Cache
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(9)
    a = Qwen35Args(num_hidden_layers=4)
    B, H, Hkv, hd = 2, a.num_attention_heads, a.num_key_value_heads, a.head_dim
    qn, kn = 1 + 0.1 * torch.randn(hd, generator=g), 1 + 0.1 * torch.randn(hd, generator=g)

    def module(device, dtype):
        m = FullAttention(a, 3, _Given(), _Given(), torch.nn.Identity(), qn.to(device, dtype), kn.to(device, dtype))
        return m, Qwen35Cache(a, B, 16, device, dtype)
    cpu, ccache = module("cpu", torch.float32)
    gpu, gcache = module(dev, torch.float16)
    for t in range(5):
        qk = torch.randn(B, 1, H * 2 * hd + Hkv * hd, generator=g).half()
        v = torch.randn(B, 1, Hkv * hd, generator=g).half()
        cpu.qk_proj.value, cpu.v_proj.value = qk.float(), v.float()
        gpu.qk_proj.value, gpu.v_proj.value = qk.to(dev), v.to(dev)
        want = cpu(torch.zeros(B, 1, 8), ccache)
        got = gpu(torch.zeros(B, 1, 8, device=dev, dtype=torch.float16), gcache).float().cpu()
        ccache.pos.add_(1)
        gcache.pos.add_(1)
        assert torch.isfinite(got).all()
        assert rel_l2(got.numpy(), want.numpy()) <= 5e-3, t
        for c in (3,):
            assert rel_l2(gcache.k[c][:, :, :t + 1].float().cpu().numpy(), ccache.k[c][:, :, :t + 1].numpy()) <= 2e-3
            assert torch.equal(gcache.v[c][:, :, :t + 1].float().cpu(), ccache.v[c][:, :, :t + 1])
    # a longer context (three 64-position score passes, the 8-position V blocks and a tail):
    # identical random caches up to position 141, one new token at 141
    for c in (gcache, ccache):
        c.k[3] = c.k[3].new_zeros(B, Hkv, 160, hd)
        c.v[3] = c.v[3].new_zeros(B, Hkv, 160, hd)
    kc = torch.randn(B, Hkv, 141, hd, generator=g).half()
    vc = torch.randn(B, Hkv, 141, hd, generator=g).half()
    gcache.k[3][:, :, :141], gcache.v[3][:, :, :141] = kc.to(dev), vc.to(dev)
    ccache.k[3][:, :, :141], ccache.v[3][:, :, :141] = kc.float(), vc.float()
    gcache.pos.fill_(141)
    ccache.pos.fill_(141)
    qk = torch.randn(B, 1, H * 2 * hd + Hkv * hd, generator=g).half()
    v = torch.randn(B, 1, Hkv * hd, generator=g).half()
    cpu.qk_proj.value, cpu.v_proj.value = qk.float(), v.float()
    gpu.qk_proj.value, gpu.v_proj.value = qk.to(dev), v.to(dev)
    want = cpu(torch.zeros(B, 1, 8), ccache)
    got = gpu(torch.zeros(B, 1, 8, device=dev, dtype=torch.float16), gcache).float().cpu()
    assert rel_l2(got.numpy(), want.numpy()) <= 5e-3
    # the same token with the positions split into chunks of 64 (three chunks hold positions,
    # the last one none) and combined: the long-context form
    from mlx_gsq_amd.runtime.kernels import model_ops
    orig = (model_ops.ATTN_SPLIT_MIN_LEN, model_ops.ATTN_CHUNK)
    model_ops.ATTN_SPLIT_MIN_LEN, model_ops.ATTN_CHUNK = 1, 64
    try:
        kc0, vc0 = gcache.k[3].clone(), gcache.v[3].clone()
        got_split = gpu(torch.zeros(B, 1, 8, device=dev, dtype=torch.float16), gcache).float().cpu()
    finally:
        model_ops.ATTN_SPLIT_MIN_LEN, model_ops.ATTN_CHUNK = orig
    assert rel_l2(got_split.numpy(), want.numpy()) <= 5e-3
    assert rel_l2(got_split.numpy(), got.numpy()) <= 1e-3
    assert torch.equal(gcache.k[3], kc0) and torch.equal(gcache.v[3], vc0)  # same slot, same values


@pytest.mark.gpu
def test_gpu_attention_position_bounds():
    """attn_decode at the last cache slot (pos = max_len - 1) on the single-workgroup and the
    chunked path, and with a position outside the cache (pos = max_len, pos = -1): NaN rows and
    untouched caches instead of writes past the head's cache slab."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from mlx_gsq_amd.runtime.kernels import model_ops
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(21)
    B, H, Hkv, hd, rd, L = 2, 4, 2, 64, 32, 128
    qg = torch.randn(B, H * 2 * hd, generator=g).half().to(dev)
    k = torch.randn(B, Hkv * hd, generator=g).half().to(dev)
    v = torch.randn(B, Hkv * hd, generator=g).half().to(dev)
    qn = (1 + 0.1 * torch.randn(hd, generator=g)).half().to(dev)
    kn = (1 + 0.1 * torch.randn(hd, generator=g)).half().to(dev)
    inv_freq = (1.0 / (10000.0 ** (torch.arange(0, rd, 2, dtype=torch.float64) / rd))).to(dev)
    kc0 = torch.randn(B, Hkv, L, hd, generator=g).half().to(dev)
    vc0 = torch.randn(B, Hkv, L, hd, generator=g).half().to(dev)
    kw = dict(heads=H, kv_heads=Hkv, head_dim=hd, rotary_dim=rd, eps=1e-6)
    outs = []
    for chunk in (0, 64):
        kc, vc = kc0.clone(), vc0.clone()
        pos = torch.tensor([L - 1], dtype=torch.int64, device=dev)
        out = model_ops.attn_decode(qg, k, v, qn, kn, inv_freq, kc, vc, pos, chunk=chunk, **kw)
        torch.cuda.synchronize()
        assert torch.isfinite(out).all(), chunk
        assert torch.equal(kc[:, :, :L - 1], kc0[:, :, :L - 1]) and torch.equal(vc[:, :, L - 1].flatten(1), v), chunk
        outs.append(out.float().cpu())
        for bad in (L, -1):
            kc, vc = kc0.clone(), vc0.clone()
            pos = torch.tensor([bad], dtype=torch.int64, device=dev)
            out = model_ops.attn_decode(qg, k, v, qn, kn, inv_freq, kc, vc, pos, chunk=chunk, **kw)
            torch.cuda.synchronize()
            assert torch.isnan(out).all(), (chunk, bad)
            assert torch.equal(kc, kc0) and torch.equal(vc, vc0), (chunk, bad)
    assert rel_l2(outs[1].numpy(), outs[0].numpy()) <= 1e-3
