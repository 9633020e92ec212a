"""ctypes binding of libgsq.so (the C ABI declared in include/gsq.h).

The library is built in-tree by ``mlx_gsq_amd.build`` (or ``__graft_entry__.build()``).
There is no fallback: if the library is missing or cannot be loaded, every operator raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (load torch's HIP runtime first so both share one instance)

from . import tables as _tables
from .formats import GRID_SHAPES, GRID_SOURCE, TYPE_IDS

LIB_PATH = os.environ.get("GSQ_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "libgsq.so")

GSQ_OK, GSQ_E_VALUE, GSQ_E_UNSUPPORTED, GSQ_E_TABLES, GSQ_E_HIP, GSQ_E_TYPE = range(6)
DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
ID_CODES = {torch.int32: 0, torch.int64: 1}

# Every symbol include/gsq.h declares, with its ctypes signature.
_I64, _I32, _VP, _F32 = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_float
EXPORTS = {
    "gsq_version": (_I32, []),
    "gsq_block_bytes": (_I32, [_I32]),
    "gsq_set_tables": (_I32, [_I32, _VP, _I64, _I64, _VP, _I64]),
    "gsq_prepare": (_I32, [_VP]),
    "gsq_tables_ready": (_I32, [_I32]),
    "gsq_dequant": (_I32, [_I32, _VP, _I64, _VP, _VP]),
    "gsq_qmv": (_I32, [_I32, _VP, _VP, _I32, _VP, _I32, _I64, _I64, _I64, _VP]),
    "gsq_qmv_group2": (_I32, [_I32, _VP, _I64, _VP, _I32, _VP, _I64, _VP, _VP, _I32, _I64, _VP]),
    "gsq_qmv_pre": (_I32, [_I32, _VP, _I32, _VP, _VP, _VP, _F32, _VP, _VP, _VP, _I32, _I64, _I64, _VP, _VP, _I64,
                           _I64, _VP, _VP]),
    "gsq_qmm": (_I32, [_I32, _VP, _VP, _I32, _VP, _I32, _I64, _I64, _I64, _VP]),
    "gsq_qmm_noalloc": (_I32, [_I32, _VP, _VP, _I32, _VP, _I32, _I64, _I64, _I64, _VP]),
    "gsq_embedding": (_I32, [_I32, _VP, _VP, _I32, _I64, _I64, _I64, _VP, _I32, _VP]),
    "gsq_add_rms_norm": (_I32, [_VP, _VP, _VP, _VP, _I64, _I64, _F32, _I32, _VP]),
    "gsq_swiglu": (_I32, [_VP, _VP, _I64, _I64, _I32, _VP]),
    "gsq_attn_decode": (_I32, [_VP, _I64, _VP, _I64, _VP, _I64, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64,
                               _I64, _I64, _I64, _I64, _F32, _VP, _I64, _I32, _VP]),
    "gsq_gdn_step": (_I32, [_VP, _I64, _VP, _I64, _VP, _I64, _VP, _I64, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _I64,
                            _VP, _I64, _I64, _I64, _I64, _I64, _I64, _F32, _I32, _VP]),
    "gsq_gdn_seq": (_I32, [_VP, _I64, _VP, _I64, _VP, _I64, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _I64, _VP, _I64,
                           _I64, _I64, _I64, _I64, _I64, _I64, _F32, _I32, _VP]),
    "gsq_last_error": (ctypes.c_char_p, []),
}

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libgsq.so not found at {LIB_PATH}; build it with "
                               "`python mlx-gsq-rco_amd/mlx_gsq_amd/build.py` or __graft_entry__.build()")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in EXPORTS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc == GSQ_OK:
        return
    msg = lib().gsq_last_error().decode(errors="replace")
    exc = {GSQ_E_VALUE: ValueError, GSQ_E_UNSUPPORTED: NotImplementedError,
           GSQ_E_TYPE: TypeError}.get(rc, RuntimeError)
    raise exc(f"{what}: {msg}")


_uploaded: dict = {}


def ensure_tables(qtype: str, device: torch.device) -> None:
    """Upload the codebook of a grid type to ``device`` once per table version."""
    if qtype not in GRID_SHAPES:
        return
    key = (device.index, qtype)
    if _uploaded.get(key) == _tables.version():
        return
    grid = _tables.grid(qtype)
    ks = _tables.ksigns()
    src = GRID_SOURCE.get(qtype, qtype)
    n, c = GRID_SHAPES[src]
    g = grid.reshape(n, c).astype("float32", copy=False)
    with torch.cuda.device(device):
        check(lib().gsq_set_tables(TYPE_IDS[qtype], g.ctypes.data, n, c, ks.ctypes.data, 128),
              f"gsq_set_tables({qtype})")
    _uploaded[key] = _tables.version()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def prepare(device=None, stream=None) -> None:
    """Build the fixed tables and the QMM workspace of ``stream`` (default: the current
    stream) on ``device`` so that later calls on that stream allocate nothing; required
    before capturing QMM calls on a stream into a HIP graph (``gsq_prepare``)."""
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    with torch.cuda.device(device):
        s = torch.cuda.current_stream(device) if stream is None else stream
        check(lib().gsq_prepare(s.cuda_stream), "gsq_prepare")
