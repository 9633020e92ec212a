"""Qwen3.5-hybrid decoder on packed GGUF weights (torch, one GPU).

Stands in for mlx_gsq/models/qwen35.py:11-152: ``build_qwen35(store, dtype)`` builds the 27B
hybrid text model (``_args`` :11-36) from a ``PackedModelStore`` with ``GSQEmbedding`` for the
token table, ``GSQLinear`` for every packed projection and the plain tensors for norms,
convolution and recurrence coefficients (:114-152), and runs the GatedDeltaNet layers with
llama.cpp's cyclic Q/K-to-value-head routing (:48-111). The reference attaches those modules
to mlx-lm's Qwen3.5 model; that package is not part of this build, so the decoder around the
projections is written here on torch ops, following the same layer structure:

* 64 layers; layer i is full attention when (i + 1) % 4 == 0, else a GatedDeltaNet
  (linear attention); each is pre-norm + residual, followed by a pre-norm SwiGLU MLP.
* Norms: RMSNorm, y = x / rms(x) * w, with the GGUF weights as stored (llama.cpp's converter
  bakes HF's (1 + w) scaling into them, and the reference loads them into plain RMSNorms).
* GatedDeltaNet: in_proj_qkv -> depthwise causal conv (kernel 4, state of the last 3 inputs) ->
  SiLU -> q, k, v; q and k RMS-normalized per head (eps 1e-6) and scaled by d^-1 and d^-1/2;
  value head h reads Q/K head h mod 16 (the GGUF layout; mlx-lm's generic helper would group
  three consecutive value heads instead, hence the reference's patch); beta = sigmoid(b),
  decay = exp(ssm_a * softplus(a + dt_bias)) with ssm_a = -exp(A_log) as GGUF stores it;
  recurrence S <- decay S; S <- S + k (beta (v - S^T k))^T; out = S^T q (fp32 state);
  gated RMSNorm out / rms(out) * w * silu(z); out_proj.
* Full attention: q_proj gives per head [q | gate]; q and k RMS-normalized per head with their
  weights; rotary embedding on the first 64 of 256 dims (rotate-half form, base 1e7, the text
  positions of the interleaved multimodal RoPE, whose three sections coincide for text);
  24 query heads over 4 KV heads (head h reads KV head h // 6), softmax(q k^T / 16) v in fp32,
  times sigmoid(gate), o_proj.
* Output: final RMSNorm, lm_head.

Decoding keeps a cache per layer in fixed device buffers (convolution and fp32 recurrent
state; K/V up to ``max_len`` positions, masked by a device-side position), so a whole
single-token step can be captured once in a HIP graph and replayed (``GraphDecoder``).

On a GPU the residual adds + RMSNorms, the SwiGLU, each GatedDeltaNet token and each
single-token attention run as fused libgsq.so kernels (runtime/kernels/model_ops.py); gate and
up, qkv and z, q and k are one packed launch each where they share a quantization type. For
one token of one sequence the norms and the SwiGLU go further, into the prologue of the packed
projection that consumes them (``forward_pre``, libgsq ``gsq_qmv_pre``). The torch
formulation below computes the same values and is what CPU tensors run (the structure test
runs the model on the CPU with dense stand-ins for the packed layers).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F


@dataclass(frozen=True)
class Qwen35Args:
    """Model shape; the defaults are the 27B checkpoint's (reference qwen35.py:11-36)."""
    hidden_size: int = 5120
    intermediate_size: int = 17408
    num_hidden_layers: int = 64
    num_attention_heads: int = 24
    num_key_value_heads: int = 4
    head_dim: int = 256
    vocab_size: int = 248320
    rms_norm_eps: float = 1e-6
    linear_num_value_heads: int = 48
    linear_num_key_heads: int = 16
    linear_key_head_dim: int = 128
    linear_value_head_dim: int = 128
    linear_conv_kernel_dim: int = 4
    full_attention_interval: int = 4
    rope_theta: float = 10_000_000.0
    partial_rotary_factor: float = 0.25

    def is_linear(self, layer: int) -> bool:
        return (layer + 1) % self.full_attention_interval != 0

    @property
    def key_dim(self) -> int:
        return self.linear_num_key_heads * self.linear_key_head_dim

    @property
    def value_dim(self) -> int:
        return self.linear_num_value_heads * self.linear_value_head_dim

    @property
    def conv_dim(self) -> int:
        return 2 * self.key_dim + self.value_dim

    @property
    def rotary_dim(self) -> int:
        return int(self.head_dim * self.partial_rotary_factor)


def rms_norm(x, weight, eps):
    """x / sqrt(mean(x^2) + eps) (* weight) over the last axis, in fp32, back to x's dtype."""
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    if weight is not None:
        y = y * weight.float()
    return y.to(x.dtype)


def add_rms_norm(x, delta, weight, eps):
    """x += delta in place (when given); returns rms_norm(x, weight, eps)."""
    if x.is_cuda:
        from ..runtime.kernels import model_ops
        return model_ops.add_rms_norm(x, delta, weight, eps)
    if delta is not None:
        x.add_(delta)
    return rms_norm(x, weight, eps)


class Qwen35Cache:
    """Per-layer decode state in fixed device buffers, and the position of the next token.

    ``pos`` is a one-element int64 device tensor (read by the captured graph); ``length`` is the
    host's count of cached tokens, which guards ``max_len``.
    """

    def __init__(self, args: Qwen35Args, batch: int, max_len: int, device, dtype):
        self.max_len = max_len
        self.length = 0
        self.pos = torch.zeros(1, dtype=torch.int64, device=device)
        self.conv, self.rec, self.k, self.v = {}, {}, {}, {}
        for i in range(args.num_hidden_layers):
            if args.is_linear(i):
                self.conv[i] = torch.zeros(batch, args.linear_conv_kernel_dim - 1, args.conv_dim, device=device,
                                           dtype=dtype)
                self.rec[i] = torch.zeros(batch, args.linear_num_value_heads, args.linear_key_head_dim,
                                          args.linear_value_head_dim, device=device, dtype=torch.float32)
            else:
                shape = (batch, args.num_key_value_heads, max_len, args.head_dim)
                self.k[i] = torch.zeros(shape, device=device, dtype=dtype)
                self.v[i] = torch.zeros(shape, device=device, dtype=dtype)

    def reset(self):
        self.length = 0
        self.pos.zero_()
        for t in (*self.conv.values(), *self.rec.values()):
            t.zero_()


class GatedDeltaNet(torch.nn.Module):
    """Linear-attention layer with the GGUF (cyclic) value-to-Q/K head routing
    (reference qwen35.py:48-111)."""

    def __init__(self, args: Qwen35Args, layer: int, in_proj_qkvz, out_proj, w_a, w_b, conv_w, ssm_a, dt_bias,
                 norm_w):
        super().__init__()
        self.args, self.layer = args, layer
        self.in_proj_qkvz, self.out_proj = in_proj_qkvz, out_proj  # in_proj_qkvz: [qkv | z]
        self.register_buffer("w_ab", torch.cat([w_a, w_b]))  # (2 Hv, hidden): a then b
        self.register_buffer("conv_w", conv_w)  # (conv_dim, kernel)
        self.register_buffer("ssm_a", ssm_a.float())    # (Hv,) = -exp(A_log)
        self.register_buffer("dt_bias", dt_bias.float())  # (Hv,)
        self.register_buffer("norm_w", norm_w)  # (head_v_dim,)

    @property
    def first_proj(self):
        """The projection of the layer input (its input norm can be fused into it)."""
        return self.in_proj_qkvz

    def first_pre(self, x, cache: Qwen35Cache, **kw):
        """in_proj_qkvz of the row its prologue forms from x (``forward_pre`` keywords), with the
        convolution of the qkv rows in its epilogue: returns (qkvz, convolution outputs), the
        ``first`` of ``forward``."""
        work = torch.empty(1, self.args.conv_dim, dtype=torch.float32, device=x.device)
        qkvz = self.in_proj_qkvz.forward_pre(x, "add_rms_norm", conv=(cache.conv[self.layer], self.conv_w, work),
                                             **kw)
        return qkvz, work

    def forward(self, x, cache: Qwen35Cache, first=None):
        """``first``: ``in_proj_qkvz(x)`` when the caller has computed it already, or
        ``first_pre``'s (qkvz, convolution outputs)."""
        a_ = self.args
        B, S, _ = x.shape
        hk, hv = a_.linear_num_key_heads, a_.linear_num_value_heads
        dk, dv = a_.linear_key_head_dim, a_.linear_value_head_dim
        kw = a_.linear_conv_kernel_dim
        conv_out = None
        if isinstance(first, tuple):
            first, conv_out = first
        qkvz = self.in_proj_qkvz(x) if first is None else first
        qkv, z = qkvz[..., :a_.conv_dim], qkvz[..., a_.conv_dim:]   # (B, S, conv_dim), (B, S, Hv * dv)
        if x.is_cuda:
            from ..runtime.kernels import model_ops
            if S == 1:  # the a / b projections happen inside the fused step
                out = model_ops.gdn_step(qkv[:, 0], z[:, 0], x[:, 0], self.w_ab, cache.conv[self.layer], self.conv_w,
                                         self.ssm_a, self.dt_bias, cache.rec[self.layer], self.norm_w,
                                         key_heads=hk, value_heads=hv, head_k_dim=dk, head_v_dim=dv,
                                         eps=a_.rms_norm_eps, conv_out=conv_out)[:, None]
            else:  # a sequence: a / b of all tokens in one product, then one recurrence launch
                out = model_ops.gdn_seq(qkv, z, F.linear(x, self.w_ab), cache.conv[self.layer], self.conv_w,
                                        self.ssm_a, self.dt_bias, cache.rec[self.layer], self.norm_w,
                                        key_heads=hk, value_heads=hv, head_k_dim=dk, head_v_dim=dv,
                                        eps=a_.rms_norm_eps)
            return self.out_proj(out)
        z = z.view(B, S, hv, dv)
        a, b = F.linear(x, self.w_ab).float().split(hv, dim=-1)  # (B, S, Hv) each
        # depthwise causal convolution over [3 cached inputs, S new ones]
        conv_in = torch.cat([cache.conv[self.layer], qkv.to(cache.conv[self.layer].dtype)], dim=1)
        cache.conv[self.layer].copy_(conv_in[:, S:])
        w = self.conv_w.float()
        acc = conv_in[:, 0:S].float() * w[:, 0]
        for j in range(1, kw):
            acc = acc + conv_in[:, j:j + S].float() * w[:, j]
        conv_out = F.silu(acc)                           # (B, S, conv_dim), fp32
        q, k, v = conv_out.split([a_.key_dim, a_.key_dim, a_.value_dim], dim=-1)
        q = rms_norm(q.reshape(B, S, hk, dk), None, 1e-6) * (1.0 / dk)
        k = rms_norm(k.reshape(B, S, hk, dk), None, 1e-6) * (dk ** -0.5)
        v = v.reshape(B, S, hv, dv)
        # value head h reads Q/K head h % hk (tile, not repeat-interleave)
        if hv != hk:
            q = q.repeat(1, 1, hv // hk, 1)
            k = k.repeat(1, 1, hv // hk, 1)
        beta = torch.sigmoid(b)
        decay = torch.exp(self.ssm_a * F.softplus(a + self.dt_bias))   # (B, S, Hv)
        st = cache.rec[self.layer]
        outs = []
        for t in range(S):
            st = st * decay[:, t, :, None, None]
            kv_mem = (st * k[:, t, :, :, None]).sum(-2)                # (B, Hv, dv)
            delta = (v[:, t] - kv_mem) * beta[:, t, :, None]
            st = st + k[:, t, :, :, None] * delta[:, :, None, :]
            outs.append((st * q[:, t, :, :, None]).sum(-2))
        cache.rec[self.layer].copy_(st)
        out = torch.stack(outs, dim=1)                                  # (B, S, Hv, dv), fp32
        out = rms_norm(out, self.norm_w, a_.rms_norm_eps) * F.silu(z.float())
        return self.out_proj(out.to(x.dtype).reshape(B, S, hv * dv))


def _rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], dim=-1)


class FullAttention(torch.nn.Module):
    """Gated grouped-query attention with partial rotary embedding over the cached K/V."""

    def __init__(self, args: Qwen35Args, layer: int, qk_proj, v_proj, o_proj, q_norm_w, k_norm_w):
        super().__init__()
        self.args, self.layer = args, layer
        self.qk_proj, self.v_proj, self.o_proj = qk_proj, v_proj, o_proj  # qk_proj: [q_proj | k_proj]
        self.register_buffer("q_norm_w", q_norm_w)
        self.register_buffer("k_norm_w", k_norm_w)
        rd = args.rotary_dim
        steps = torch.arange(0, rd, 2, dtype=torch.float64, device=q_norm_w.device)
        self.register_buffer("inv_freq", 1.0 / (args.rope_theta ** (steps / rd)))

    def _rope(self, x, pos):
        """x (B, S, H, hd); pos (S,) int64 positions."""
        rd = self.args.rotary_dim
        ang = pos.to(torch.float64)[:, None] * self.inv_freq[None, :]   # (S, rd/2)
        ang = torch.cat([ang, ang], dim=-1)
        cos = ang.cos().float()[None, :, None, :]
        sin = ang.sin().float()[None, :, None, :]
        xr = x[..., :rd].float()
        xr = xr * cos + _rotate_half(xr) * sin
        return torch.cat([xr.to(x.dtype), x[..., rd:]], dim=-1)

    @property
    def first_proj(self):
        """The projection of the layer input (its input norm can be fused into it)."""
        return self.qk_proj

    def first_pre(self, x, cache: Qwen35Cache, **kw):
        """qk_proj of the row its prologue forms from x (``forward_pre`` keywords)."""
        return self.qk_proj.forward_pre(x, "add_rms_norm", **kw)

    def forward(self, x, cache: Qwen35Cache, first=None):
        """``first``: ``qk_proj(x)`` when the caller has computed it already."""
        a_ = self.args
        B, S, _ = x.shape
        H, Hkv, hd = a_.num_attention_heads, a_.num_key_value_heads, a_.head_dim
        qk = self.qk_proj(x) if first is None else first
        v = self.v_proj(x)
        if x.is_cuda and S == 1:
            from ..runtime.kernels import model_ops
            out = model_ops.attn_decode(qk[:, 0, :H * 2 * hd], qk[:, 0, H * 2 * hd:], v[:, 0], self.q_norm_w,
                                        self.k_norm_w, self.inv_freq, cache.k[self.layer], cache.v[self.layer],
                                        cache.pos, heads=H, kv_heads=Hkv, head_dim=hd, rotary_dim=a_.rotary_dim,
                                        eps=a_.rms_norm_eps)
            return self.o_proj(out.view(B, 1, H * hd))
        qg = qk[..., :H * 2 * hd].reshape(B, S, H, 2 * hd)
        q, gate = qg[..., :hd], qg[..., hd:].reshape(B, S, H * hd)
        q = rms_norm(q, self.q_norm_w, a_.rms_norm_eps)
        k = rms_norm(qk[..., H * 2 * hd:].reshape(B, S, Hkv, hd), self.k_norm_w, a_.rms_norm_eps)
        v = v.view(B, S, Hkv, hd)
        pos = cache.pos + torch.arange(S, device=x.device)             # (S,)
        q = self._rope(q, pos)
        k = self._rope(k, pos)
        kc, vc = cache.k[self.layer], cache.v[self.layer]              # (B, Hkv, L, hd)
        kc.index_copy_(2, pos, k.transpose(1, 2).to(kc.dtype))
        vc.index_copy_(2, pos, v.transpose(1, 2).to(vc.dtype))
        L = kc.shape[2]
        rep = H // Hkv
        qf = q.float().transpose(1, 2).reshape(B, Hkv, rep * S, hd)   # query head h -> KV head h // rep
        scores = torch.matmul(qf, kc.float().transpose(2, 3).contiguous()) * (hd ** -0.5)  # (B, Hkv, rep*S, L)
        qpos = pos.repeat(rep)                                          # (rep*S,) position of each query row
        mask = torch.arange(L, device=x.device)[None, :] > qpos[:, None]
        scores = scores.masked_fill(mask, float("-inf"))
        att = torch.matmul(torch.softmax(scores, dim=-1), vc.float())  # (B, Hkv, rep*S, hd)
        att = att.reshape(B, H, S, hd).transpose(1, 2).reshape(B, S, H * hd)
        out = att * torch.sigmoid(gate.float())
        return self.o_proj(out.to(x.dtype))


def _can_pre(m) -> bool:
    """Whether module m can form its input row itself (``forward_pre``)."""
    return hasattr(m, "forward_pre") and getattr(m, "pre_ok", True)


def _fused_row(x, *mods) -> bool:
    """One fp16 row on a GPU, through modules that can form their input row themselves."""
    return x.is_cuda and x.dtype == torch.float16 and x.shape[0] * x.shape[1] == 1 and all(map(_can_pre, mods))


class Qwen35Layer(torch.nn.Module):
    """Pre-norm mixer and SwiGLU MLP. ``forward(x, delta, cache)`` first adds the previous
    layer's pending MLP output ``delta`` into the residual stream ``x`` (fused with this layer's
    input norm) and returns ``(x, m)``: the residual stream and this layer's MLP output, to be
    added the same way by the next layer or the final norm. The residual stream is ``x`` itself,
    updated in place, except for one fp16 row on a GPU with packed projections: there the norms
    and the SwiGLU run inside the projections that consume them (``forward_pre``), which write
    the updated stream to a new buffer (other workgroups of the launch still read ``x``)."""

    def __init__(self, args, mixer, input_norm_w, post_norm_w, gate_up, down):
        super().__init__()
        self.args, self.mixer = args, mixer
        self.register_buffer("input_norm_w", input_norm_w)
        self.register_buffer("post_norm_w", post_norm_w)
        self.gate_up, self.down = gate_up, down  # gate_up: [gate | up] of the MLP in one product

    def forward(self, x, delta, cache):
        eps = self.args.rms_norm_eps
        if _fused_row(x, self.mixer.first_proj, self.gate_up, self.down):
            h = torch.empty_like(x)                 # the normalized layer input
            x1 = x if delta is None else torch.empty_like(x)
            first = self.mixer.first_pre(x, cache, pre_a=delta, pre_w=self.input_norm_w, eps=eps,
                                         res_out=None if delta is None else x1, x_out=h)
            m = self.mixer(h, cache, first=first)
            x2 = torch.empty_like(x)
            gu = self.gate_up.forward_pre(x1, "add_rms_norm", pre_a=m, pre_w=self.post_norm_w, eps=eps, res_out=x2)
            return x2, self.down.forward_pre(gu, "swiglu")
        m = self.mixer(add_rms_norm(x, delta, self.input_norm_w, eps), cache)
        gu = self.gate_up(add_rms_norm(x, m, self.post_norm_w, eps))
        if gu.is_cuda:
            from ..runtime.kernels import model_ops
            act = model_ops.swiglu(gu)
        else:
            g, u = gu.split(gu.shape[-1] // 2, dim=-1)
            act = (F.silu(g.float()) * u.float()).to(gu.dtype)
        return x, self.down(act)


class Qwen35Model(torch.nn.Module):
    """Token ids (B, S) -> logits (B, S, vocab) of the next tokens, advancing ``cache``."""

    def __init__(self, args: Qwen35Args, embed, layers, norm_w, lm_head, dtype):
        super().__init__()
        self.args, self.embed, self.lm_head, self.dtype = args, embed, lm_head, dtype
        self.layers = torch.nn.ModuleList(layers)
        self.register_buffer("norm_w", norm_w)

    def new_cache(self, batch: int = 1, max_len: int = 4096, device=None) -> Qwen35Cache:
        device = device if device is not None else self.norm_w.device
        return Qwen35Cache(self.args, batch, max_len, device, self.dtype)

    def forward(self, ids, cache: Qwen35Cache):
        B, S = ids.shape
        if cache.length + S > cache.max_len:
            raise ValueError(f"cache holds {cache.max_len} positions; {cache.length} used, {S} more asked")
        x = self.embed(ids).to(self.dtype).reshape(B, S, -1).contiguous()
        delta = None
        for layer in self.layers:
            x, delta = layer(x, delta, cache)
        eps = self.args.rms_norm_eps
        if _fused_row(x, self.lm_head):
            logits = self.lm_head.forward_pre(x, "add_rms_norm", pre_a=delta, pre_w=self.norm_w, eps=eps)
        else:
            logits = self.lm_head(add_rms_norm(x, delta, self.norm_w, eps))
        cache.pos.add_(S)
        cache.length += S
        return logits


class _SideBySide(torch.nn.Module):
    """Several projections of one input, outputs concatenated on the last axis."""

    def __init__(self, mods):
        super().__init__()
        self.mods = torch.nn.ModuleList(mods)

    def forward(self, x):
        return torch.cat([m(x) for m in self.mods], dim=-1)

    @property
    def pre_ok(self) -> bool:
        return all(map(_can_pre, self.mods))

    def forward_pre(self, x, pre, x_out=None, **kw):
        """The first projection forms the row (and writes it to ``x_out``); the others read it."""
        h = x.new_empty(x.shape[:-1] + (self.mods[0].in_features,)) if x_out is None else x_out
        first = self.mods[0].forward_pre(x, pre, x_out=h, **kw)
        return torch.cat([first] + [m(h) for m in self.mods[1:]], dim=-1)


def build_qwen35(store, dtype=torch.float16, args: Qwen35Args | None = None, linear=None, embedding=None,
                 fused=None):
    """The model of ``store`` (a ``PackedModelStore`` with the reference's GGUF tensor names,
    qwen35.py:114-152) on the store's device. ``linear(weight)``, ``fused(weights)`` (the
    outputs of several weights side by side) and ``embedding(weight, dtype)`` build the packed
    modules (``GSQLinear``, ``GSQFusedLinear(..., concat=True)``, ``GSQEmbedding`` by default)."""
    from ..nn import GSQEmbedding, GSQFusedLinear, GSQLinear
    args = args or Qwen35Args()
    linear = linear or GSQLinear
    fused = fused or (lambda ws: GSQFusedLinear(ws, concat=True))
    embedding = embedding or (lambda w, dt: GSQEmbedding(w, dtype=dt))

    def plain(name, dt=dtype):
        return store.materialize_plain(name).to(dt)

    def joint(names):
        """One module whose output is the named projections' outputs side by side: one packed
        launch when they share a quantization type."""
        ws = [store.weight(n) for n in names]
        if len({w.quantization_type for w in ws}) == 1:
            return fused(ws)
        return _SideBySide([linear(w) for w in ws])

    layers = []
    for i in range(args.num_hidden_layers):
        p = f"blk.{i}."
        if args.is_linear(i):
            conv = plain(p + "ssm_conv1d.weight")
            mixer = GatedDeltaNet(
                args, i, joint([p + "attn_qkv.weight", p + "attn_gate.weight"]),
                linear(store.weight(p + "ssm_out.weight")), plain(p + "ssm_alpha.weight"),
                plain(p + "ssm_beta.weight"), conv.reshape(conv.shape[0], conv.shape[-1]),
                # dt_bias rounded to the activation dtype, as the reference loads it
                # (qwen35.py:142 ``.astype(dtype)``); the kernels add it to a in float32
                plain(p + "ssm_a", torch.float32), plain(p + "ssm_dt.bias"),
                plain(p + "ssm_norm.weight"))
        else:
            mixer = FullAttention(
                args, i, joint([p + "attn_q.weight", p + "attn_k.weight"]),
                linear(store.weight(p + "attn_v.weight")), linear(store.weight(p + "attn_output.weight")),
                plain(p + "attn_q_norm.weight"), plain(p + "attn_k_norm.weight"))
        layers.append(Qwen35Layer(args, mixer, plain(p + "attn_norm.weight"), plain(p + "post_attention_norm.weight"),
                                  fused([store.weight(p + "ffn_gate.weight"), store.weight(p + "ffn_up.weight")]),
                                  linear(store.weight(p + "ffn_down.weight"))))
    return Qwen35Model(args, embedding(store.weight("token_embd.weight"), dtype), layers,
                       plain("output_norm.weight"), linear(store.weight("output.weight")), dtype)


class GraphDecoder:
    """Single-token decode steps of ``model`` captured once in a HIP graph and replayed.

    The captured step reads the token ids from a fixed buffer and the position from the cache's
    device tensor, so every replay decodes the next token; ``step(ids)`` returns the (B, 1,
    vocab) logits buffer, overwritten by the next step.
    """

    def __init__(self, model: Qwen35Model, cache: Qwen35Cache, batch: int = 1):
        self.model, self.cache = model, cache
        device = cache.pos.device
        self.ids = torch.zeros(batch, 1, dtype=torch.int64, device=device)
        # one eager step on the side stream first: libraries allocate their tables and
        # workspaces outside the capture; the cache is then restored to its state before it
        snap = self._snapshot()
        side = torch.cuda.Stream(device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            model(self.ids, cache)
            torch.cuda.synchronize(device)
            self._restore(snap)
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph, stream=side):
                self.logits = model(self.ids, cache)
        torch.cuda.current_stream(device).wait_stream(side)
        torch.cuda.synchronize(device)
        # the graph's QMM launches use the capture stream's workspace (libgsq keys workspaces
        # by stream): the stream is kept with the graph
        self.capture_stream = side
        # the capture traced one step without running it: undo its host-side bookkeeping
        self._restore(snap)

    def _snapshot(self):
        c = self.cache
        return (c.length, c.pos.clone(), {k: t.clone() for k, t in c.conv.items()},
                {k: t.clone() for k, t in c.rec.items()})

    def _restore(self, snap):
        c = self.cache
        c.length = snap[0]
        c.pos.copy_(snap[1])
        for k, t in snap[2].items():
            c.conv[k].copy_(t)
        for k, t in snap[3].items():
            c.rec[k].copy_(t)

    def step(self, ids):
        if self.cache.length + 1 > self.cache.max_len:
            raise ValueError("cache is full")
        self.ids.copy_(ids.reshape(self.ids.shape))
        self.graph.replay()
        self.cache.length += 1
        return self.logits
