"""Q4_K dequant-matmul on the MI355X kernels (mirror of the engine's GGUF q4_k path).

Reference: SparseInferenceEngine.cpp decodeSupportedGGUFQuantized (q4_k :362-384) then
Kernels::linear_forward (kernels/blas_kernels.cpp:264-293): out (M x R) = in (M x C) . W^T.
"""
from __future__ import annotations

from . import _lib
from .hsdr import _check, _stream_ptr, _torch

GGML = 0
INTERLEAVED = 1
BLOCK_BYTES = 144


def upload(blob: bytes):
    """Q4_K bytes -> device uint8 tensor (16-byte aligned allocation)."""
    torch = _torch()
    import numpy as np

    return torch.from_numpy(np.frombuffer(blob, dtype=np.uint8).copy()).cuda()


def linear(w_dev, R: int, C: int, x, order: int = GGML, out=None, stream=None):
    """y (M, R) fp32 = x (M, C) . dequant(W)^T; x fp32 (M == 1) or fp16, on the device."""
    torch = _torch()
    if x.dim() == 1:
        x = x.reshape(1, -1)
    M = x.shape[0]
    if x.shape[1] != C or not x.is_contiguous() or not x.is_cuda:
        raise ValueError("x must be a contiguous device tensor of shape (M, C)")
    dt = 1 if x.dtype == torch.float16 else 0
    if out is None:
        out = torch.empty((M, R), dtype=torch.float32, device="cuda")
    _check(_lib.load().csdr_q4k_linear(w_dev.data_ptr(), R, C, order, x.data_ptr(), dt, M,
                                       out.data_ptr(), _stream_ptr(stream)))
    return out


def dequant(w_dev, n_blocks: int, order: int = GGML, stream=None):
    torch = _torch()
    out = torch.empty(n_blocks * 256, dtype=torch.float32, device="cuda")
    _check(_lib.load().csdr_q4k_dequant(w_dev.data_ptr(), n_blocks, order, out.data_ptr(),
                                        _stream_ptr(stream)))
    return out
