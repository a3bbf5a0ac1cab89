"""GGUF block-format dequant-matmuls on the MI355X kernels (mirror of the engine's strategy-0
GGUF path for every format it decodes).

Reference: SparseInferenceEngine.cpp decodeSupportedGGUFQuantized (:276-469; block sizes
:181-231) then Kernels::linear_forward (kernels/blas_kernels.cpp:264-293):
out (M x R) = in (M x C) . W^T, W decoded with the reference's element orders and arithmetic.
"""
from __future__ import annotations

import ctypes as C

from . import _lib
from .hsdr import _check, _stream_ptr, _torch


def format_id(name: str) -> int:
    """CSDR_GGUF_* id of a GGUF type name (as a segment's data_format holds it)."""
    f = _lib.load().csdr_gguf_format(name.encode())
    if f < 0:
        raise ValueError(f"GGUF format {name!r} is not one the engine decodes")
    return f


def block(fmt: int):
    """(bytes, elements) per block."""
    bb, be = C.c_int(0), C.c_int(0)
    _check(_lib.load().csdr_gguf_block(fmt, C.byref(bb), C.byref(be)))
    return bb.value, be.value


def upload(blob: bytes):
    """Block bytes -> device uint8 tensor."""
    torch = _torch()
    import numpy as np

    return torch.from_numpy(np.frombuffer(blob, dtype=np.uint8).copy()).cuda()


def linear(w_dev, fmt: int, R: int, Cc: int, x, out=None, stream=None):
    """y (M, R) fp32 = x (M, C) . dequant(W)^T; x fp32 (M == 1) or fp16, on the device."""
    torch = _torch()
    if x.dim() == 1:
        x = x.reshape(1, -1)
    M = x.shape[0]
    if x.shape[1] != Cc or not x.is_contiguous() or not x.is_cuda:
        raise ValueError("x must be a contiguous device tensor of shape (M, C)")
    dt = 1 if x.dtype == torch.float16 else 0
    if out is None:
        out = torch.empty((M, R), dtype=torch.float32, device="cuda")
    _check(_lib.load().csdr_gguf_linear(w_dev.data_ptr(), fmt, R, Cc, x.data_ptr(), dt, M,
                                        out.data_ptr(), _stream_ptr(stream)))
    return out


def dequant(w_dev, fmt: int, n_blocks: int, stream=None):
    torch = _torch()
    _, be = block(fmt)
    out = torch.empty(n_blocks * be, dtype=torch.float32, device="cuda")
    _check(_lib.load().csdr_gguf_dequant(w_dev.data_ptr(), fmt, n_blocks, out.data_ptr(),
                                         _stream_ptr(stream)))
    return out
