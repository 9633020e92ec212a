"""Fused dequant + matrix-vector product on packed GGUF weights (decode path).

Drop-in counterpart of mlx_gsq/runtime/kernels/qmv.py:537-576 ``quantized_matvec`` on
torch tensors: same name, keyword arguments, validation order and exceptions. Inputs
with at least ``QMM_MIN_ROWS`` rows are routed to the tiled QMM, as in the reference
(qmv.py:548-549). The work runs in libgsq.so's gfx950 QMV kernel on the tensors' device
and current stream.
"""
from __future__ import annotations

import torch

from ... import _lib
from ...formats import QTYPES, TYPE_IDS
from ...gguf.parser import GGMLQuantizationType, QUANT_BLOCK_SIZES
from .qmm import QMM_MIN_ROWS, quantized_matmul


def _validate_width(packed, qtype, out_features, in_features):
    type_id = int(GGMLQuantizationType[qtype])  # KeyError for unknown names, as qmv.py:540
    block_elements, block_bytes = QUANT_BLOCK_SIZES[type_id]
    if block_elements != 256 or in_features % 256:
        raise ValueError(f"invalid {qtype} matrix width")
    expected = out_features * (in_features // 256) * block_bytes
    if packed.numel() != expected:
        raise ValueError(f"packed size {packed.numel()} != expected {expected}")


def _validate(x, packed, qtype, out_features, in_features):
    _validate_width(packed, qtype, out_features, in_features)
    if x.shape[-1] != in_features:
        raise ValueError("input feature size mismatch")


def _check_tensors(x, packed):
    if packed.dtype != torch.uint8:
        raise TypeError("packed input must be uint8")
    if x.dtype not in _lib.DTYPE_CODES:
        raise TypeError(f"unsupported activation dtype {x.dtype}")
    if x.device.type != "cuda" or packed.device != x.device:
        raise ValueError("x and packed must be on the same GPU device")


# Rows below the reference's QMM threshold stay on gsq_qmv (the quad-row kernel takes 3-8 fp16
# rows) except on matrices of at least 2^26 weights: there gsq_qmm's small-batch kernel is faster
# from 5 rows when K is wider than the quad-row kernel stages in LDS (K > 8192) and from 7 rows
# otherwise. Measured per 27B projection at 4 / 5 / 6 / 7 rows (us, gsq_qmv against gsq_qmm):
# down Q4_K 5120x17408 20.7 / 24.3 / 25.1 / 26.0 against 23.3-23.8; gate/up IQ2_S 17408x5120
# 15.1 / 21.6 / 21.3 / 23.8 against 22.3-22.6; the 5120x5120 and 1024x5120 products faster on
# gsq_qmv up to 8 rows (q IQ2_XS 9.1-10.3 against 12.1-12.5, k 5.6-6.4 against 7.5).
SMALL_BATCH_MIN_WEIGHTS = 1 << 26
SMALL_BATCH_WIDE_K = 8192


def _small_batch_faster(rows, dtype, out_features, in_features):
    if dtype != torch.float16 or out_features * in_features < SMALL_BATCH_MIN_WEIGHTS:
        return False
    return rows >= (5 if in_features > SMALL_BATCH_WIDE_K else 7)


def routes_to_qmm(rows, dtype, out_features, in_features):
    """True if ``quantized_matvec`` sends ``rows`` activation rows of ``dtype`` to the QMM
    kernels: the reference's row threshold (qmv.py:548-549), rows wider than the vector
    kernel's activation registers hold (K <= 65536 for fp16 activations, K <= 32768 for
    fp32/bf16, split into two fp16 parts), and the small batches where the small-batch QMM is
    faster."""
    max_k = 65536 if dtype == torch.float16 else 32768
    return (rows >= QMM_MIN_ROWS or in_features > max_k
            or _small_batch_faster(rows, dtype, out_features, in_features))


def quantized_matvec(x, packed, *, qtype: str, out_features: int, in_features: int, out_dtype=None):
    """y = x @ W.T for packed ``W`` of shape ``(out_features, in_features)``.

    ``x`` has shape ``(..., in_features)``; the result has shape ``(..., out_features)`` and
    dtype ``out_dtype`` (default: ``x.dtype``, as the reference).
    """
    _validate(x, packed, qtype, out_features, in_features)
    original = x.shape[:-1]
    rows = x.numel() // in_features
    flat = x.reshape(rows, in_features)
    if routes_to_qmm(rows, x.dtype, out_features, in_features):
        return quantized_matmul(flat, packed, qtype=qtype, out_features=out_features,
                                in_features=in_features, out_dtype=out_dtype).reshape(*original, out_features)
    if qtype not in QTYPES:
        raise KeyError(qtype)
    _check_tensors(x, packed)
    odt = out_dtype or x.dtype
    flat = flat.contiguous()
    packed = packed.contiguous()
    y = torch.empty((rows, out_features), dtype=odt, device=x.device)
    if rows:
        _lib.ensure_tables(qtype, x.device)
        with torch.cuda.device(x.device):
            _lib.check(_lib.lib().gsq_qmv(TYPE_IDS[qtype], packed.data_ptr(), flat.data_ptr(),
                                          _lib.DTYPE_CODES[flat.dtype], y.data_ptr(), _lib.DTYPE_CODES[odt],
                                          rows, out_features, in_features, _lib.stream_handle(x.device)),
                       "quantized_matvec")
    return y.reshape(*original, out_features)


def quantized_matvec_group2(x, packed0, packed1, *, qtypes, out_features, in_features: int, out_dtype=None):
    """``(x @ W0.T, x @ W1.T)`` for one activation row ``x`` (``in_features`` values) and two
    packed matrices of any two quantization types (``qtypes``, ``out_features``: one per
    matrix) in one launch (``gsq_qmv_group2``). No counterpart in the reference, whose model
    applies each projection on its own; validation and exceptions as ``quantized_matvec``.
    Not one fp16 row: the two products through ``quantized_matvec``."""
    (q0, q1), (n0, n1) = qtypes, out_features
    _validate(x, packed0, q0, n0, in_features)
    _validate(x, packed1, q1, n1, in_features)
    if x.numel() != in_features or x.dtype != torch.float16:
        return (quantized_matvec(x, packed0, qtype=q0, out_features=n0, in_features=in_features, out_dtype=out_dtype),
                quantized_matvec(x, packed1, qtype=q1, out_features=n1, in_features=in_features, out_dtype=out_dtype))
    for q in (q0, q1):
        if q not in QTYPES:
            raise KeyError(q)
    _check_tensors(x, packed0)
    _check_tensors(x, packed1)
    odt = out_dtype or x.dtype
    flat = x.reshape(in_features).contiguous()
    packed0, packed1 = packed0.contiguous(), packed1.contiguous()
    y0 = torch.empty(x.shape[:-1] + (n0,), dtype=odt, device=x.device)
    y1 = torch.empty(x.shape[:-1] + (n1,), dtype=odt, device=x.device)
    _lib.ensure_tables(q0, x.device)
    _lib.ensure_tables(q1, x.device)
    with torch.cuda.device(x.device):
        _lib.check(_lib.lib().gsq_qmv_group2(TYPE_IDS[q0], packed0.data_ptr(), n0, y0.data_ptr(), TYPE_IDS[q1],
                                             packed1.data_ptr(), n1, y1.data_ptr(), flat.data_ptr(),
                                             _lib.DTYPE_CODES[odt], in_features, _lib.stream_handle(x.device)),
                   "quantized_matvec_group2")
    return y0, y1


PRE_OPS = {"add_rms_norm": 1, "swiglu": 2}  # GSQ_PRE_ADD_RMSNORM, GSQ_PRE_SWIGLU


def _overlap(a, b):
    """True if contiguous tensors ``a`` and ``b`` share a byte of device memory."""
    if a is None or b is None:
        return False
    pa, pb = a.data_ptr(), b.data_ptr()
    return pa < pb + b.numel() * b.element_size() and pb < pa + a.numel() * a.element_size()


def quantized_matvec_pre(x, packed, *, qtype: str, out_features: int, in_features: int, pre: str, pre_a=None,
                         pre_w=None, eps: float = 0.0, res_out=None, x_out=None, out_dtype=None, conv=None):
    """y = row @ W.T for one fp16 activation row that the QMV kernel forms itself (libgsq
    ``gsq_qmv_pre``; no counterpart in the reference, whose model runs these as separate
    operations):

    * ``pre="add_rms_norm"``: ``s = x + pre_a`` (``pre_a`` may be None), rounded to fp16 and
      written to ``res_out`` when given; ``row =
      rms_norm(s) * pre_w`` with ``eps``, as ``model_ops.add_rms_norm`` computes it;
    * ``pre="swiglu"``: ``x`` holds ``[gate | up]`` (``2 * in_features`` values); ``row =
      silu(gate) * up``, as ``model_ops.swiglu`` computes it.

    The row is also written to ``x_out`` when given. Neither ``res_out`` nor ``x_out`` may
    overlap ``x``, ``pre_a``, ``pre_w`` or each other (other workgroups of the launch still read
    the inputs while the first writes the outputs; ValueError). ``x`` and the vectors are fp16 and hold
    exactly one row (any leading shape of size 1); the result has shape ``x.shape[:-1] +
    (out_features,)``. ``conv=(state, weight, out)`` adds the GatedDeltaNet's depthwise causal
    convolution of the first ``state.shape[-1]`` outputs (fp16 result only): ``state`` (1, k-1,
    rows) fp16 shifted in place, ``weight`` (rows, k) fp16, ``out`` (rows,) float32 receives
    silu(convolution), as ``model_ops.gdn_step`` computes it.
    """
    if pre not in PRE_OPS:
        raise ValueError(f"unknown pre op {pre!r}")
    _validate_width(packed, qtype, out_features, in_features)
    if qtype not in QTYPES:
        raise KeyError(qtype)
    _check_tensors(x, packed)
    width = 2 * in_features if pre == "swiglu" else in_features
    if x.dtype != torch.float16 or x.shape[-1] != width or x.numel() != width:
        raise ValueError(f"x must be one fp16 row of {width} values")
    for name, t in (("pre_a", pre_a), ("pre_w", pre_w), ("res_out", res_out), ("x_out", x_out)):
        if t is None:
            continue
        if t.dtype != torch.float16 or t.numel() != in_features or not t.is_contiguous() or t.device != x.device:
            raise ValueError(f"{name} must be a contiguous fp16 vector of {in_features} values on x's device")
    if pre == "add_rms_norm" and pre_w is None:
        raise ValueError("add_rms_norm needs the norm weight pre_w")
    odt = out_dtype or x.dtype
    conv_rows = conv_k = 0
    if conv is not None:
        state, weight, cout = conv
        conv_rows, conv_k = state.shape[-1], weight.shape[-1]
        if (odt != torch.float16 or state.dtype != torch.float16 or weight.dtype != torch.float16
                or cout.dtype != torch.float32 or tuple(state.shape) != (1, conv_k - 1, conv_rows)
                or weight.numel() != conv_rows * conv_k or cout.numel() != conv_rows
                or not (state.is_contiguous() and weight.is_contiguous() and cout.is_contiguous())
                or conv_rows > out_features or any(t.device != x.device for t in conv)):
            raise ValueError("conv must be (state (1, k-1, rows) fp16, weight (rows, k) fp16, out (rows,) float32), "
                             "contiguous, rows <= out_features, fp16 output")
    flat = x.contiguous()
    # the first workgroup writes res_out / x_out while the others still read x, pre_a and pre_w
    outs = (("res_out", res_out if pre == "add_rms_norm" else None), ("x_out", x_out))
    ins = (flat,) + ((pre_a, pre_w) if pre == "add_rms_norm" else ())
    for name, o in outs:
        if o is not None and any(_overlap(o, t) for t in ins):
            raise ValueError(f"{name} must not alias x, pre_a or pre_w (other workgroups still read them)")
    if res_out is not None and x_out is not None and pre == "add_rms_norm" and _overlap(res_out, x_out):
        raise ValueError("res_out and x_out must not alias")
    packed = packed.contiguous()
    y = torch.empty(x.shape[:-1] + (out_features,), dtype=odt, device=x.device)

    def ptr(t):
        return None if t is None else t.data_ptr()
    _lib.ensure_tables(qtype, x.device)
    with torch.cuda.device(x.device):
        _lib.check(_lib.lib().gsq_qmv_pre(TYPE_IDS[qtype], packed.data_ptr(), PRE_OPS[pre], flat.data_ptr(),
                                          ptr(pre_a), ptr(pre_w), float(eps), ptr(res_out), ptr(x_out), y.data_ptr(),
                                          _lib.DTYPE_CODES[odt], out_features, in_features,
                                          None if conv is None else conv[0].data_ptr(),
                                          None if conv is None else conv[1].data_ptr(), conv_rows, conv_k,
                                          None if conv is None else conv[2].data_ptr(),
                                          _lib.stream_handle(x.device)),
                   "quantized_matvec_pre")
    return y

