"""A tiny Qwen3.5-hybrid checkpoint in GGUF conventions, and its HF transformers counterpart.

The decode step (mlx_gsq_amd/models/qwen35.py) is checked against transformers' own
Qwen3.5 text model (an independent implementation of the architecture, installed in this
image), run in float32 on the CPU on the same weights:

* packed projections are seeded random superblocks whose fp16 scales are rescaled so the
  weights have a std of ~1/sqrt(in_features); both sides use the oracle's exact dequant of the
  very same bytes;
* GGUF conventions the reference relies on (mlx_gsq/models/qwen35.py:40-152) are undone for HF:
  RMSNorm weights hold HF's (1 + w) (llama.cpp adds 1 when converting), ``ssm_a`` is
  -exp(A_log), and value head h of a GatedDeltaNet reads Q/K head h mod n_k (GGUF order) where
  HF reads head h // (n_v / n_k): HF's value heads are the GGUF heads permuted.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from mlx_gsq_amd import synth, tables
from mlx_gsq_amd.formats import BLOCK_BYTES, TYPE_IDS
from mlx_gsq_amd.models.qwen35 import Qwen35Args
from mlx_gsq_amd.runtime.store import PackedWeight
from oracle import gsq_oracle as O

TABLES = tables.synthetic_tables(0)

ARGS = Qwen35Args(hidden_size=256, intermediate_size=512, num_hidden_layers=4, num_attention_heads=4,
                  num_key_value_heads=2, head_dim=64, vocab_size=512, linear_num_value_heads=4,
                  linear_num_key_heads=2, linear_key_head_dim=32, linear_value_head_dim=64)

# quantization type of every packed projection (a checkpoint-like mix)
QTYPES = {"attn_qkv": "IQ2_XS", "attn_gate": "IQ3_S", "ssm_out": "Q4_K", "attn_q": "IQ4_XS", "attn_k": "Q6_K",
          "attn_v": "Q6_K", "attn_output": "IQ3_S", "ffn_gate": "IQ2_S", "ffn_up": "IQ2_S", "ffn_down": "Q4_K",
          "output": "Q6_K", "token_embd": "IQ2_S"}


def _packed(qtype, n, k, seed, std):
    """Seeded packed matrix whose dequantized weights have about the given std."""
    p = synth.make_packed(qtype, n, k, seed=seed)
    w = O.dequantize_reference(p, qtype, TABLES.get(qtype))
    factor = std / max(float(w.std()), 1e-12)
    raw = p.reshape(n * (k // 256), BLOCK_BYTES[qtype]).copy()
    for off in synth._FP16_FIELDS[qtype]:
        d = np.ascontiguousarray(raw[:, off:off + 2]).view(np.float16).astype(np.float32) * factor
        raw[:, off:off + 2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    return raw.reshape(-1)


class TinyStore:
    """The store interface build_qwen35 uses (weight, materialize_plain) over in-memory tensors,
    plus the float32 dequantized value of every packed tensor (``dense``)."""

    def __init__(self, device="cpu", seed=0):
        a = ARGS
        rng = np.random.default_rng(seed)
        self.device = torch.device(device)
        self.packed, self.plain, self.dense, self.shapes = {}, {}, {}, {}
        counter = [seed * 1000]

        def packed(name, kind, n, k, std=None):
            counter[0] += 1
            q = QTYPES[kind]
            p = _packed(q, n, k, counter[0], std if std is not None else 1.0 / math.sqrt(k))
            self.packed[name] = (q, p, n, k)
            self.dense[name] = O.dequantize_reference(p, q, TABLES.get(q)).reshape(n, k)

        def plain(name, value):
            self.plain[name] = np.asarray(value, dtype=np.float32)

        H = a.hidden_size
        packed("token_embd.weight", "token_embd", a.vocab_size, H, std=1.0)
        packed("output.weight", "output", a.vocab_size, H)
        plain("output_norm.weight", 1.0 + 0.1 * rng.standard_normal(H))
        hv, dv, dk = a.linear_num_value_heads, a.linear_value_head_dim, a.linear_key_head_dim
        for i in range(a.num_hidden_layers):
            p = f"blk.{i}."
            plain(p + "attn_norm.weight", 1.0 + 0.1 * rng.standard_normal(H))
            plain(p + "post_attention_norm.weight", 1.0 + 0.1 * rng.standard_normal(H))
            packed(p + "ffn_gate.weight", "ffn_gate", a.intermediate_size, H)
            packed(p + "ffn_up.weight", "ffn_up", a.intermediate_size, H)
            packed(p + "ffn_down.weight", "ffn_down", H, a.intermediate_size)
            if a.is_linear(i):
                packed(p + "attn_qkv.weight", "attn_qkv", a.conv_dim, H)
                packed(p + "attn_gate.weight", "attn_gate", a.value_dim, H)
                packed(p + "ssm_out.weight", "ssm_out", H, a.value_dim)
                plain(p + "ssm_alpha.weight", rng.standard_normal((hv, H)) / math.sqrt(H))
                plain(p + "ssm_beta.weight", rng.standard_normal((hv, H)) / math.sqrt(H))
                plain(p + "ssm_conv1d.weight", 0.5 * rng.standard_normal((a.conv_dim, a.linear_conv_kernel_dim)))
                plain(p + "ssm_a", -np.exp(np.log(rng.uniform(1, 16, hv))))
                plain(p + "ssm_dt.bias", rng.standard_normal(hv))
                plain(p + "ssm_norm.weight", 1.0 + 0.1 * rng.standard_normal(dv))
            else:
                packed(p + "attn_q.weight", "attn_q", a.num_attention_heads * a.head_dim * 2, H)
                packed(p + "attn_k.weight", "attn_k", a.num_key_value_heads * a.head_dim, H)
                packed(p + "attn_v.weight", "attn_v", a.num_key_value_heads * a.head_dim, H)
                packed(p + "attn_output.weight", "attn_output", H, a.num_attention_heads * a.head_dim)
                plain(p + "attn_q_norm.weight", 1.0 + 0.1 * rng.standard_normal(a.head_dim))
                plain(p + "attn_k_norm.weight", 1.0 + 0.1 * rng.standard_normal(a.head_dim))

    def weight(self, name):
        q, p, n, k = self.packed[name]
        data = torch.from_numpy(p).to(self.device)
        return PackedWeight(name=name, data=data, gguf_shape=(k, n), logical_shape=(n, k), quantization_type=q,
                            quantization_type_id=TYPE_IDS[q], num_elements=n * k, num_bytes=p.size)

    def materialize_plain(self, name):
        return torch.from_numpy(self.plain[name]).to(self.device)


class DenseLinear(torch.nn.Module):
    """x @ W^T with W the oracle's dequant of a packed weight (test stand-in on the CPU)."""

    def __init__(self, w):
        super().__init__()
        self.w = torch.from_numpy(np.ascontiguousarray(w))

    def forward(self, x):
        return (x.float() @ self.w.T).to(x.dtype)


def dense_factories(store):
    """(linear, fused, embedding) factories of build_qwen35 over the dense dequantized weights."""
    def linear(weight):
        return DenseLinear(store.dense[weight.name])

    def fused(weights):
        return DenseLinear(np.concatenate([store.dense[w.name] for w in weights]))

    def embedding(weight, dtype):
        table = torch.from_numpy(store.dense[weight.name])
        return lambda ids: table[ids].to(dtype)
    return linear, fused, embedding


def hf_model(store):
    """transformers' Qwen3.5 causal LM (float32, eager attention) with the store's weights."""
    from transformers import Qwen3_5ForCausalLM, Qwen3_5TextConfig
    a = ARGS
    cfg = Qwen3_5TextConfig(
        vocab_size=a.vocab_size, hidden_size=a.hidden_size, intermediate_size=a.intermediate_size,
        num_hidden_layers=a.num_hidden_layers, num_attention_heads=a.num_attention_heads,
        num_key_value_heads=a.num_key_value_heads, head_dim=a.head_dim, rms_norm_eps=a.rms_norm_eps,
        linear_conv_kernel_dim=a.linear_conv_kernel_dim, linear_key_head_dim=a.linear_key_head_dim,
        linear_value_head_dim=a.linear_value_head_dim, linear_num_key_heads=a.linear_num_key_heads,
        linear_num_value_heads=a.linear_num_value_heads, tie_word_embeddings=False,
        rope_parameters={"rope_type": "default", "rope_theta": a.rope_theta,
                         "partial_rotary_factor": a.partial_rotary_factor, "mrope_section": [3, 3, 2]})
    cfg._attn_implementation = "eager"
    torch.manual_seed(0)
    model = Qwen3_5ForCausalLM(cfg).float().eval()
    hk, hv, dv = a.linear_num_key_heads, a.linear_num_value_heads, a.linear_value_head_dim
    r = hv // hk
    # HF value head h' = GGUF value head perm[h'] (GGUF head h reads Q/K head h % hk, HF head
    # h' reads head h' // r)
    perm = np.empty(hv, dtype=np.int64)
    for h in range(hv):
        perm[(h % hk) * r + h // hk] = h
    rows_v = np.concatenate([np.arange(p * dv, (p + 1) * dv) for p in perm])
    d, pl = store.dense, store.plain
    sd = {"model.embed_tokens.weight": d["token_embd.weight"], "lm_head.weight": d["output.weight"],
          "model.norm.weight": pl["output_norm.weight"] - 1.0}
    for i in range(a.num_hidden_layers):
        p, m = f"blk.{i}.", f"model.layers.{i}."
        sd[m + "input_layernorm.weight"] = pl[p + "attn_norm.weight"] - 1.0
        sd[m + "post_attention_layernorm.weight"] = pl[p + "post_attention_norm.weight"] - 1.0
        sd[m + "mlp.gate_proj.weight"] = d[p + "ffn_gate.weight"]
        sd[m + "mlp.up_proj.weight"] = d[p + "ffn_up.weight"]
        sd[m + "mlp.down_proj.weight"] = d[p + "ffn_down.weight"]
        if a.is_linear(i):
            la = m + "linear_attn."
            qkv = d[p + "attn_qkv.weight"]
            sd[la + "in_proj_qkv.weight"] = np.concatenate([qkv[:2 * a.key_dim], qkv[2 * a.key_dim:][rows_v]])
            conv = pl[p + "ssm_conv1d.weight"]
            conv = np.concatenate([conv[:2 * a.key_dim], conv[2 * a.key_dim:][rows_v]])
            sd[la + "conv1d.weight"] = conv[:, None, :]
            sd[la + "in_proj_z.weight"] = d[p + "attn_gate.weight"][rows_v]
            sd[la + "in_proj_a.weight"] = pl[p + "ssm_alpha.weight"][perm]
            sd[la + "in_proj_b.weight"] = pl[p + "ssm_beta.weight"][perm]
            sd[la + "A_log"] = np.log(-pl[p + "ssm_a"])[perm]
            sd[la + "dt_bias"] = pl[p + "ssm_dt.bias"][perm]
            sd[la + "norm.weight"] = pl[p + "ssm_norm.weight"]
            sd[la + "out_proj.weight"] = d[p + "ssm_out.weight"][:, rows_v]
        else:
            sa = m + "self_attn."
            sd[sa + "q_proj.weight"] = d[p + "attn_q.weight"]
            sd[sa + "k_proj.weight"] = d[p + "attn_k.weight"]
            sd[sa + "v_proj.weight"] = d[p + "attn_v.weight"]
            sd[sa + "o_proj.weight"] = d[p + "attn_output.weight"]
            sd[sa + "q_norm.weight"] = pl[p + "attn_q_norm.weight"] - 1.0
            sd[sa + "k_norm.weight"] = pl[p + "attn_k_norm.weight"] - 1.0
    state = {k: torch.from_numpy(np.ascontiguousarray(v, dtype=np.float32)) for k, v in sd.items()}
    missing, unexpected = model.load_state_dict(state, strict=False)
    assert not unexpected, unexpected
    assert not [k for k in missing if "rotary" not in k], missing
    return model


def hf_logits(model, ids):
    """float32 logits of every position of one sequence (1, S, vocab)."""
    with torch.no_grad():
        return model(input_ids=torch.as_tensor(ids).reshape(1, -1), use_cache=False).logits.float()


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
