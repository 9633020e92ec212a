"""Fused element-wise operations of the model decode step, on libgsq.so.

Residual add + RMSNorm, SwiGLU and one GatedDeltaNet token (include/gsq.h: gsq_add_rms_norm,
gsq_swiglu, gsq_gdn_step). They replace mlx / mlx-lm operations of the reference's model
(mlx_gsq/models/qwen35.py:48-111 and the layers it builds on) and compute what the torch
formulation in mlx_gsq_amd/models/qwen35.py computes, in one launch each. Tensors must be on a
GPU (there is no CPU path here) and share one dtype: float32, float16 or bfloat16.
"""
from __future__ import annotations

import torch

from ... import _lib


def _dt(t):
    if t.dtype not in _lib.DTYPE_CODES:
        raise TypeError(f"unsupported dtype {t.dtype}")
    return _lib.DTYPE_CODES[t.dtype]


def _on_gpu(*ts):
    dev = ts[0].device
    if dev.type != "cuda" or any(t.device != dev for t in ts):
        raise ValueError("tensors must be on one GPU device")
    return dev


def add_rms_norm(x, delta, w, eps: float):
    """If ``delta`` is given, ``x += delta`` in place (rounded to x's dtype); returns
    ``x / sqrt(mean(x^2) + eps) * w`` over the last axis. x, delta contiguous."""
    dim = x.shape[-1]
    ts = (x, w) if delta is None else (x, delta, w)
    dev = _on_gpu(*ts)
    if any(t.dtype != x.dtype for t in ts) or w.numel() != dim:
        raise ValueError("x, delta and w must share the dtype and the last dimension")
    if not x.is_contiguous() or (delta is not None and (not delta.is_contiguous() or delta.shape != x.shape)):
        raise ValueError("x and delta must be contiguous and of one shape")
    y = torch.empty_like(x)
    rows = x.numel() // dim
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().gsq_add_rms_norm(x.data_ptr(), None if delta is None else delta.data_ptr(),
                                               w.contiguous().data_ptr(), y.data_ptr(), rows, dim, float(eps), _dt(x),
                                               _lib.stream_handle(dev)), "add_rms_norm")
    return y


def swiglu(gate_up):
    """``silu(gate) * up`` for rows of [gate | up] (last axis 2n) -> last axis n."""
    dev = _on_gpu(gate_up)
    if not gate_up.is_contiguous() or gate_up.shape[-1] % 2:
        raise ValueError("gate_up must be contiguous with an even last dimension")
    n = gate_up.shape[-1] // 2
    out = torch.empty(*gate_up.shape[:-1], n, dtype=gate_up.dtype, device=dev)
    rows = gate_up.numel() // (2 * n)
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().gsq_swiglu(gate_up.data_ptr(), out.data_ptr(), rows, n, _dt(gate_up),
                                         _lib.stream_handle(dev)), "swiglu")
    return out


def gdn_step(qkv, z, x, w_ab, conv_state, conv_w, ssm_a, dt_bias, rec_state, norm_w, *, key_heads: int,
             value_heads: int, head_k_dim: int, head_v_dim: int, eps: float, conv_out=None):
    """One GatedDeltaNet token for B rows: qkv (B, conv_dim), z (B, Hv*dv) and the layer input x
    (B, hidden) as rows with unit stride along the last axis; w_ab (2 Hv, hidden) the a and b
    projections; conv_state (B, K-1, conv_dim) and rec_state (B, Hv, dk, dv, float32) are
    updated in place. ``conv_out`` (B, conv_dim, float32): the convolution has run already (in
    the input projection's epilogue, ``quantized_matvec_pre(..., conv=...)``) and these are its
    outputs; conv_state is then left alone. Returns (B, Hv*dv)."""
    dev = _on_gpu(qkv, z, x, w_ab, conv_state, conv_w, ssm_a, dt_bias, rec_state, norm_w)
    B = qkv.shape[0]
    for t in (qkv, z, x):
        if t.dim() != 2 or t.shape[0] != B or t.stride(1) != 1 or t.dtype != qkv.dtype:
            raise ValueError("qkv, z and x must be (B, n) rows of one dtype with unit inner stride")
    for t in (w_ab, conv_state, conv_w, norm_w):
        if t.dtype != qkv.dtype or not t.is_contiguous():
            raise ValueError("w_ab, conv_state, conv_w and norm_w must be contiguous in the activation dtype")
    for t in (ssm_a, dt_bias, rec_state):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError("ssm_a, dt_bias and rec_state must be contiguous float32")
    conv_dim = 2 * key_heads * head_k_dim + value_heads * head_v_dim
    K = conv_w.shape[-1]
    hidden = x.shape[1]
    if (qkv.shape[1] != conv_dim or z.shape[1] != value_heads * head_v_dim
            or tuple(w_ab.shape) != (2 * value_heads, hidden)
            or tuple(conv_state.shape) != (B, K - 1, conv_dim) or conv_w.numel() != conv_dim * K
            or tuple(rec_state.shape) != (B, value_heads, head_k_dim, head_v_dim) or norm_w.numel() != head_v_dim
            or ssm_a.numel() != value_heads or dt_bias.numel() != value_heads):
        raise ValueError("GatedDeltaNet tensor shapes do not match the head configuration")
    out = torch.empty(B, value_heads * head_v_dim, dtype=qkv.dtype, device=dev)
    if conv_out is None:
        work = torch.empty(B, conv_dim, dtype=torch.float32, device=dev)
    else:
        if (conv_out.dtype != torch.float32 or not conv_out.is_contiguous() or conv_out.numel() != B * conv_dim
                or conv_out.device != dev):
            raise ValueError("conv_out must be contiguous float32 (B, conv_dim) on the same device")
        work = conv_out
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().gsq_gdn_step(
            qkv.data_ptr(), qkv.stride(0), z.data_ptr(), z.stride(0), x.data_ptr(), x.stride(0), w_ab.data_ptr(),
            hidden, None if conv_out is not None else conv_state.data_ptr(), conv_w.data_ptr(), ssm_a.data_ptr(),
            dt_bias.data_ptr(),
            rec_state.data_ptr(), norm_w.data_ptr(), out.data_ptr(), out.stride(0), work.data_ptr(), B, key_heads,
            value_heads, head_k_dim, head_v_dim, K, float(eps), _dt(qkv), _lib.stream_handle(dev)), "gdn_step")
    return out


def gdn_seq(qkv, z, ab, conv_state, conv_w, ssm_a, dt_bias, rec_state, norm_w, *, key_heads: int, value_heads: int,
            head_k_dim: int, head_v_dim: int, eps: float):
    """``gdn_step`` over S tokens of B rows (prefill): qkv (B, S, conv_dim), z (B, S, Hv*dv) and ab
    (B, S, 2 Hv: the a and b projections, a then b) with unit stride along the last axis and the
    (B, S) rows at one stride each. The states advance over all S tokens. Returns (B, S, Hv*dv)."""
    dev = _on_gpu(qkv, z, ab, conv_state, conv_w, ssm_a, dt_bias, rec_state, norm_w)
    B, S = qkv.shape[0], qkv.shape[1]
    rows = []
    for t in (qkv, z, ab):
        if (t.dim() != 3 or tuple(t.shape[:2]) != (B, S) or t.stride(2) != 1 or t.dtype != qkv.dtype
                or (S > 1 and t.stride(0) != S * t.stride(1))):
            raise ValueError("qkv, z and ab must be (B, S, n) of one dtype, unit inner stride, rows at one stride")
        rows.append(t.stride(1))
    for t in (conv_state, conv_w, norm_w):
        if t.dtype != qkv.dtype or not t.is_contiguous():
            raise ValueError("conv_state, conv_w and norm_w must be contiguous in the activation dtype")
    for t in (ssm_a, dt_bias, rec_state):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError("ssm_a, dt_bias and rec_state must be contiguous float32")
    conv_dim = 2 * key_heads * head_k_dim + value_heads * head_v_dim
    K = conv_w.shape[-1]
    if (qkv.shape[2] != conv_dim or z.shape[2] != value_heads * head_v_dim or ab.shape[2] != 2 * value_heads
            or tuple(conv_state.shape) != (B, K - 1, conv_dim) or conv_w.numel() != conv_dim * K
            or tuple(rec_state.shape) != (B, value_heads, head_k_dim, head_v_dim) or norm_w.numel() != head_v_dim
            or ssm_a.numel() != value_heads or dt_bias.numel() != value_heads):
        raise ValueError("GatedDeltaNet tensor shapes do not match the head configuration")
    out = torch.empty(B, S, value_heads * head_v_dim, dtype=qkv.dtype, device=dev)
    work = torch.empty(B * S, conv_dim, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().gsq_gdn_seq(
            qkv.data_ptr(), rows[0], z.data_ptr(), rows[1], ab.data_ptr(), rows[2], conv_state.data_ptr(),
            conv_w.data_ptr(), ssm_a.data_ptr(), dt_bias.data_ptr(), rec_state.data_ptr(), norm_w.data_ptr(),
            out.data_ptr(), out.stride(1), work.data_ptr(), B, S, key_heads, value_heads, head_k_dim, head_v_dim, K,
            float(eps), _dt(qkv), _lib.stream_handle(dev)), "gdn_seq")
    return out


# caches at least this long split the positions into chunks (one workgroup each, then a combine)
ATTN_SPLIT_MIN_LEN = 2048
ATTN_CHUNK = 256


def attn_decode(qg, k, v, q_norm_w, k_norm_w, inv_freq, k_cache, v_cache, pos, *, heads: int, kv_heads: int,
                head_dim: int, rotary_dim: int, eps: float, chunk=None):
    """One new token of gated grouped-query attention for B rows: qg (B, heads * 2 head_dim) with
    [q | gate] per head, k and v (B, kv_heads * head_dim), rows with unit inner stride; the caches
    (B, kv_heads, max_len, head_dim) get k and v at position ``pos`` (a one-element int64 device
    tensor); inv_freq (rotary_dim / 2,) float64. ``chunk``: positions per workgroup (a multiple of
    64 up to 1024; 0 = one workgroup per head over all positions; default: ``ATTN_CHUNK`` for
    caches of ``ATTN_SPLIT_MIN_LEN`` positions or more, else 0). Returns (B, heads * head_dim)."""
    dev = _on_gpu(qg, k, v, q_norm_w, k_norm_w, inv_freq, k_cache, v_cache, pos)
    B = qg.shape[0]
    for t in (qg, k, v):
        if t.dim() != 2 or t.shape[0] != B or t.stride(1) != 1 or t.dtype != qg.dtype:
            raise ValueError("qg, k and v must be (B, n) rows of one dtype with unit inner stride")
    if (qg.shape[1] != heads * 2 * head_dim or k.shape[1] != kv_heads * head_dim or v.shape[1] != kv_heads * head_dim
            or q_norm_w.numel() != head_dim or k_norm_w.numel() != head_dim or inv_freq.numel() != rotary_dim // 2
            or k_cache.shape != v_cache.shape or tuple(k_cache.shape[:2]) != (B, kv_heads)
            or k_cache.shape[3] != head_dim):
        raise ValueError("attention tensor shapes do not match the head configuration")
    if inv_freq.dtype != torch.float64 or pos.dtype != torch.int64 or pos.numel() != 1:
        raise ValueError("inv_freq must be float64 and pos one int64")
    for t in (q_norm_w, k_norm_w, k_cache, v_cache):
        if t.dtype != qg.dtype or not t.is_contiguous():
            raise ValueError("norm weights and caches must be contiguous in the activation dtype")
    out = torch.empty(B, heads * head_dim, dtype=qg.dtype, device=dev)
    L = k_cache.shape[2]
    if chunk is None:
        chunk = ATTN_CHUNK if L >= ATTN_SPLIT_MIN_LEN else 0
    work = None
    if chunk:
        work = torch.empty(B * heads * (-(-L // chunk)) * (head_dim + 2), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().gsq_attn_decode(
            qg.data_ptr(), qg.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0), q_norm_w.data_ptr(),
            k_norm_w.data_ptr(), inv_freq.contiguous().data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
            pos.data_ptr(), out.data_ptr(), out.stride(0), B, heads, kv_heads, head_dim, rotary_dim,
            L, float(eps), None if work is None else work.data_ptr(), int(chunk), _dt(qg),
            _lib.stream_handle(dev)), "attn_decode")
    return out
