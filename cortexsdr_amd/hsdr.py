"""Host-side mirror of the reference's HSDR operator interface, on the MI355X kernels.

Reference interface (cortexSDR tree):
  HierarchicalSDRStrategy::matmulRowMajor(const vector<byte>&, const float* x, size_t batch)
      -> vector<float>                     strategies/HierarchicalSDRStrategy.hpp:179-181
  HierarchicalSDRStrategy::decompress(const vector<byte>&, SegmentType, size_t originalSize)
      -> vector<byte>                      strategies/HierarchicalSDRStrategy.hpp:170-172
Errors: the reference throws CompressionError (CompressionStrategy.hpp:33-36); here the
C-ABI status is raised as CompressionError (a RuntimeError subclass) with the same cases:
bad magic/version, geometry mismatch, truncation.

HsdbSegment keeps a stream resident on the device (what SDRModelLoader's per-call file read
and parse, SparseInferenceEngine.cpp:1055-1091, becomes here): load once, matmul many times
on device tensors with inputs already in HBM.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib

CSDR_F32 = 0
CSDR_F16 = 1


class CompressionError(_lib.CsdrError):
    """Status of a rejected stream (the reference's CompressionError cases)."""


def _check(rc: int) -> None:
    if rc != 0:
        msg = _lib.load().csdr_last_error()
        raise CompressionError(rc, msg.decode() if msg else "")


def _torch():
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("cortexsdr_amd needs a HIP device (no CPU fallback)")
    return torch


def _stream_ptr(stream=None) -> int:
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


class HsdbSegment:
    """A device-resident HSDR (binary) or HSDB (block-coded) weight segment; with
    host_codes=True the code words stay in pinned host memory (csdr_hsdb_load_host: a
    decoder block of such segments is streamed to the device when it runs)."""

    def __init__(self, stream: bytes, hip_stream=None, host_codes: bool = False):
        lib = _lib.load()
        _torch()
        self._buf = C.create_string_buffer(bytes(stream), len(stream))
        h = C.c_void_p()
        loader = lib.csdr_hsdb_load_host if host_codes else lib.csdr_hsdb_load
        self.host_codes = bool(host_codes)
        _check(loader(C.cast(self._buf, C.c_void_p), len(stream), _stream_ptr(hip_stream),
                      C.byref(h)))
        self._h = h
        self._buf = None
        info = _lib.HsdbInfo()
        _check(lib.csdr_hsdb_get_info(self._h, C.byref(info)))
        self.info = {name: getattr(info, name) for name, _ in info._fields_}
        self.rows = info.rows
        self.cols = info.cols
        self._ws = {}

    @classmethod
    def from_handle(cls, h):
        """Wrap a csdr_hsdb* that another loader (HSDC/HSDA/archive) produced."""
        self = cls.__new__(cls)
        lib = _lib.load()
        self._buf = None
        self._h = h
        info = _lib.HsdbInfo()
        _check(lib.csdr_hsdb_get_info(self._h, C.byref(info)))
        self.info = {name: getattr(info, name) for name, _ in info._fields_}
        self.rows = info.rows
        self.cols = info.cols
        self._ws = {}
        return self

    # ------------------------------------------------------------------ lifetime
    def free(self) -> None:
        if getattr(self, "_h", None):
            _lib.load().csdr_hsdb_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    # ------------------------------------------------------------------ compute
    def workspace_bytes(self, M: int) -> int:
        return int(_lib.load().csdr_hsdb_workspace_bytes(self._h, M))

    def workspace(self, M: int):
        """A zero-filled device workspace for batch M (cached per M)."""
        torch = _torch()
        n = self.workspace_bytes(M)
        ws = self._ws.get(M)
        if ws is None or ws.numel() < n:
            ws = torch.zeros(n, dtype=torch.uint8, device="cuda")
            self._ws[M] = ws
        return ws

    def matmul(self, x, out=None, workspace=None, stream=None):
        """Y (R, M) fp32 = W . X for a device X (C, M) or (C,) in fp32/fp16."""
        torch = _torch()
        if x.dim() == 1:
            x = x.reshape(-1, 1)
        if x.shape[0] != self.cols:
            raise ValueError(f"x has {x.shape[0]} rows, segment expects {self.cols}")
        if not x.is_cuda or not x.is_contiguous():
            raise ValueError("x must be a contiguous device tensor")
        if x.dtype == torch.float32:
            dt = CSDR_F32
        elif x.dtype == torch.float16:
            dt = CSDR_F16
        else:
            raise ValueError("x must be float32 or float16")
        M = x.shape[1]
        if out is None:
            out = torch.empty((self.rows, M), dtype=torch.float32, device=x.device)
        ws = workspace if workspace is not None else self.workspace(M)
        _check(_lib.load().csdr_hsdb_matmul(self._h, x.data_ptr(), dt, M, out.data_ptr(),
                                            ws.data_ptr(), ws.numel(), _stream_ptr(stream)))
        return out

    def decompress(self, stream=None):
        """Dense W (R, C) fp32 on the device."""
        torch = _torch()
        w = torch.empty((self.rows, self.cols), dtype=torch.float32, device="cuda")
        _check(_lib.load().csdr_hsdb_decompress(self._h, w.data_ptr(), _stream_ptr(stream)))
        return w

    def export_codes(self, stream=None):
        """(packed, |c| fp16 bits) as numpy uint16 arrays in stream order."""
        torch = _torch()
        n = self.info["slots"] * (self.info["n_block_cols"] * self.rows
                                  if self.info["tile_rows"] == 1 else 0)
        if self.info["tile_rows"] != 1:
            tr, tc = self.info["tile_rows"], self.info["tile_cols"]
            n = self.info["slots"] * (self.rows // tr) * (self.cols // tc)
        packed = torch.empty(max(n, 1), dtype=torch.int16, device="cuda")
        coef = torch.empty(max(n, 1), dtype=torch.int16, device="cuda")
        _check(_lib.load().csdr_hsdb_export_codes(self._h, packed.data_ptr(), coef.data_ptr(),
                                                  _stream_ptr(stream)))
        torch.cuda.current_stream().synchronize()
        return (packed.cpu().numpy().view(np.uint16)[:n],
                coef.cpu().numpy().view(np.uint16)[:n])


def group_workspace(segs, M: int):
    """Zero-filled device workspace for matmul_group over `segs` at batch M."""
    torch = _torch()
    arr = (C.c_void_p * len(segs))(*[s._h.value for s in segs])
    n = int(_lib.load().csdr_hsdb_group_workspace_bytes(len(segs), arr, M))
    return torch.zeros(n, dtype=torch.uint8, device="cuda")


def matmul_group(segs, xs, ys=None, workspace=None, stream=None):
    """Y_i = W_i . X_i for up to 8 segments in one launch (same M and dtype for all)."""
    torch = _torch()
    n = len(segs)
    M = xs[0].shape[1] if xs[0].dim() == 2 else 1
    dt = CSDR_F16 if xs[0].dtype == torch.float16 else CSDR_F32
    for s, x in zip(segs, xs):
        if x.shape[0] != s.cols or not x.is_contiguous() or not x.is_cuda:
            raise ValueError("each x must be a contiguous device tensor with C rows")
        if (x.shape[1] if x.dim() == 2 else 1) != M or x.dtype != xs[0].dtype:
            raise ValueError("all x must share M and dtype")
    if ys is None:
        ys = [torch.empty((s.rows, M), dtype=torch.float32, device="cuda") for s in segs]
    ws = workspace if workspace is not None else group_workspace(segs, M)
    hs = (C.c_void_p * n)(*[s._h.value for s in segs])
    xp = (C.c_void_p * n)(*[x.data_ptr() for x in xs])
    yp = (C.c_void_p * n)(*[y.data_ptr() for y in ys])
    _check(_lib.load().csdr_hsdb_matmul_group(n, hs, xp, dt, M, yp, ws.data_ptr(), ws.numel(),
                                              _stream_ptr(stream)))
    return ys


def matmul_row_major(stream: bytes, x: np.ndarray, batch: int) -> np.ndarray:
    """Drop-in for HierarchicalSDRStrategy::matmulRowMajor: host x (C x batch) row-major
    fp32 in, host Y (R x batch) fp32 out. Loads the stream per call like the reference;
    use HsdbSegment to keep it resident."""
    torch = _torch()
    seg = HsdbSegment(stream)
    try:
        xd = torch.from_numpy(np.ascontiguousarray(x, np.float32).reshape(seg.cols, batch)).cuda()
        y = seg.matmul(xd)
        return y.cpu().numpy()
    finally:
        seg.free()


def decompress(stream: bytes) -> np.ndarray:
    """Drop-in for HierarchicalSDRStrategy::decompress (fp32 R x C)."""
    seg = HsdbSegment(stream)
    try:
        return seg.decompress().cpu().numpy()
    finally:
        seg.free()


class LazyHsdrEmbedding:
    """The text CLI's lazy HSDR embedding (csdr_lazy_hsdr_*): an HSDR stream with 1-row
    tiles (vocabulary x width) kept as codes on the device; rows decoded and the vocabulary
    scored from the codes. unpack: "packed" (packIndexSign's layout) or "cli" (the CLI's
    index = v >> 1, sign = v & 1 reading)."""

    def __init__(self, stream, unpack: str = "packed"):
        torch = _torch()
        lib = _lib.load()
        b = np.frombuffer(bytes(stream), np.uint8)
        h = C.c_void_p()
        _check(lib.csdr_lazy_hsdr_load(b.ctypes.data, b.size, {"packed": 0, "cli": 1}[unpack],
                                       torch.cuda.current_stream().cuda_stream, C.byref(h)))
        self._h = h
        r, c = C.c_uint32(), C.c_uint32()
        _check(lib.csdr_lazy_hsdr_info(h, C.byref(r), C.byref(c)))
        self.rows, self.cols = r.value, c.value

    def decode_rows(self, ids):
        """Rows of the given token ids (device int32 tensor or sequence), (n, width) fp32."""
        torch = _torch()
        ids = torch.as_tensor(ids, dtype=torch.int32, device="cuda").reshape(-1)
        out = torch.empty((ids.numel(), self.cols), dtype=torch.float32, device="cuda")
        _check(_lib.load().csdr_lazy_hsdr_decode_rows(self._h, ids.data_ptr(), 0, ids.numel(),
                                                      out.data_ptr(),
                                                      torch.cuda.current_stream().cuda_stream))
        return out

    def select(self, hidden, repeated=None, temperature: float = 0.8, penalty: float = 1.0):
        """(tokens, raw scores) for hidden states (rows, width) on the device."""
        torch = _torch()
        lib = _lib.load()
        hid = hidden.reshape(-1, self.cols).contiguous()
        rows = hid.shape[0]
        ws = torch.zeros(int(lib.csdr_lazy_hsdr_workspace_bytes(self._h, rows)),
                         dtype=torch.uint8, device="cuda")
        tok = torch.empty(rows, dtype=torch.int32, device="cuda")
        scores = torch.empty((rows, self.rows), dtype=torch.float32, device="cuda")
        rp = repeated.data_ptr() if repeated is not None else None
        _check(lib.csdr_lazy_hsdr_select(self._h, hid.data_ptr(), rows, rp, C.c_float(temperature),
                                         C.c_float(penalty), tok.data_ptr(), None, None,
                                         scores.data_ptr(), ws.data_ptr(), ws.numel(),
                                         torch.cuda.current_stream().cuda_stream))
        return tok, scores

    def free(self) -> None:
        if getattr(self, "_h", None):
            _lib.load().csdr_lazy_hsdr_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
