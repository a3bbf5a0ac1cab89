"""HSDR encoder on the MI355X kernels (the compress side of HierarchicalSDRStrategy).

Reference: HierarchicalSDRStrategy.cpp hierarchicalBinaryCode (:219-262), fitHierarchicalKSVD
(:495-602) and HierarchicalSDRStrategy::compress (:1064-1237).
  encode(tiles, D, stage_scales, n_stages, k)   -> packed codes (device, n_tiles x slots)
  init_dictionary(tiles, n_atoms, n_stages, k)  -> the fit's initial dictionary (host)
  compress(w, tile_rows, tile_cols, n_atoms, n_stages, k, ksvd_iters=0, stage_decay=0.5)
                                                -> HSDR v2 stream bytes
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from .hsdr import _check, _torch


def encode(tiles, D, stage_scales, n_stages: int, k_per_stage: int):
    """Packed (sign << 15 | index) codes of matching pursuit of device tiles (n x C fp32)
    against the device dictionary D (K x C fp32), as a device uint16 tensor (n x S*k)."""
    torch = _torch()
    if tiles.dtype != torch.float32 or D.dtype != torch.float32:
        raise TypeError("tiles and D must be float32")
    n, c = tiles.shape
    K = D.shape[0]
    if D.shape[1] != c:
        raise ValueError("D and tiles differ in tile size")
    g = np.ascontiguousarray(stage_scales, np.float32)
    if g.size < n_stages:
        raise ValueError("one stage scale per stage")
    codes = torch.empty((n, n_stages * k_per_stage), dtype=torch.int16, device=tiles.device)
    st = torch.cuda.current_stream(tiles.device).cuda_stream
    _check(_lib.load().csdr_hsdr_encode(tiles.data_ptr(), n, c, D.data_ptr(), K, n_stages,
                                        k_per_stage, g.ctypes.data, codes.data_ptr(), st))
    return codes


def init_dictionary(tiles: np.ndarray, n_atoms: int, n_stages: int, k_per_stage: int):
    """fitHierarchicalKSVD's initial dictionary (n_atoms x tile_dim, host fp32) of host
    tiles (n x tile_dim), in the reference build's arithmetic."""
    t = np.ascontiguousarray(tiles, np.float32)
    D = np.zeros((n_atoms, t.shape[1]), np.float32)
    _check(_lib.load().csdr_hsdr_init_dictionary(t.ctypes.data, t.shape[0], t.shape[1], n_atoms,
                                                 n_stages, k_per_stage, D.ctypes.data))
    return D


def compress(w: np.ndarray, tile_rows: int, tile_cols: int, n_atoms: int, n_stages: int,
             k_per_stage: int, ksvd_iters: int = 0, stage_decay: float = 0.5) -> bytes:
    """HSDR v2 stream of the fp32 matrix w (rows x cols), as HierarchicalSDRStrategy::compress
    with the given config (tile_rows == 1 widens the tiles to whole rows)."""
    torch = _torch()
    w = np.ascontiguousarray(w, np.float32)
    R, Cc = w.shape
    lib = _lib.load()
    n = lib.csdr_hsdr_compress_bytes(R, Cc, tile_rows, tile_cols, n_atoms, n_stages, k_per_stage)
    if n == 0:
        raise ValueError("shape cannot be compressed with this config (no full tile, or "
                         "fewer tiles than atoms)")
    out = np.zeros(n, np.uint8)
    st = torch.cuda.current_stream().cuda_stream
    _check(lib.csdr_hsdr_compress(w.ctypes.data, R, Cc, tile_rows, tile_cols, n_atoms, n_stages,
                                  k_per_stage, ksvd_iters, C.c_float(stage_decay),
                                  out.ctypes.data, n, st))
    return out.tobytes()


SOURCE_FORMATS = {"f32": 0, "f16": 1, "bf16": 2, "i8": 3, "q4_0": 4, "q8_0": 5, "q4_k": 6,
                  "q5_k": 7, "q6_k": 8}


def source_decode(src, fmt: str, scale: float = 1.0, zero_point: float = 0.0):
    """dequantizeSegmentToFP32's decode of segment bytes (a device uint8 torch tensor) in the
    compressor's element order: a device fp32 tensor."""
    torch = _torch()
    lib = _lib.load()
    f = SOURCE_FORMATS[fmt]
    n = int(lib.csdr_hsdr_source_elements(f, src.numel()))
    out = torch.empty(max(n, 1), dtype=torch.float32, device=src.device)
    _check(lib.csdr_hsdr_source_decode(src.data_ptr(), src.numel(), f, C.c_float(scale),
                                       C.c_float(zero_point), out.data_ptr(),
                                       torch.cuda.current_stream().cuda_stream))
    return out[:n]


def compress_source(src, fmt: str, rows: int, cols: int, tile_rows: int, tile_cols: int,
                    n_atoms: int, n_stages: int, k_per_stage: int, ksvd_iters: int = 0,
                    stage_decay: float = 0.5, scale: float = 1.0,
                    zero_point: float = 0.0) -> bytes:
    """compress of a quantized segment: the source bytes (device uint8 tensor) decoded on the
    GPU, then compressed as compress()."""
    torch = _torch()
    lib = _lib.load()
    n = lib.csdr_hsdr_compress_bytes(rows, cols, tile_rows, tile_cols, n_atoms, n_stages,
                                     k_per_stage)
    if n == 0:
        raise ValueError("shape cannot be compressed with this config")
    out = np.zeros(n, np.uint8)
    _check(lib.csdr_hsdr_compress_source(
        src.data_ptr(), src.numel(), SOURCE_FORMATS[fmt], C.c_float(scale),
        C.c_float(zero_point), rows, cols, tile_rows, tile_cols, n_atoms, n_stages, k_per_stage,
        ksvd_iters, C.c_float(stage_decay), out.ctypes.data, n,
        torch.cuda.current_stream().cuda_stream))
    return out.tobytes()


def hsda_build(mats: dict, tile_rows: int, tile_cols: int, n_atoms: int, n_stages: int,
               k_per_stage: int, ksvd_iters: int = 0, stage_decay: float = 0.5,
               max_tiles_for_fit: int = 0, original_types=None):
    """compressGroupedSegments + SharedDictArchive::writeToStream: {name: (R x C) fp32} ->
    (HSDA archive bytes, names the pipeline skipped)."""
    torch = _torch()
    lib = _lib.load()
    names = list(mats)
    arrs = [np.ascontiguousarray(mats[n], np.float32) for n in names]
    n = len(arrs)
    nm = (C.c_char_p * n)(*[x.encode() for x in names])
    ws = (C.c_void_p * n)(*[a.ctypes.data for a in arrs])
    rows = (C.c_uint32 * n)(*[a.shape[0] for a in arrs])
    cols = (C.c_uint32 * n)(*[a.shape[1] for a in arrs])
    types = None
    if original_types is not None:
        types = (C.c_uint8 * n)(*original_types)
    skipped = np.zeros(n, np.uint8)
    out = C.POINTER(C.c_uint8)()
    size = C.c_size_t()
    _check(lib.csdr_hsda_build(n, nm, ws, rows, cols, types, tile_rows, tile_cols, n_atoms,
                               n_stages, k_per_stage, ksvd_iters, C.c_float(stage_decay),
                               max_tiles_for_fit, C.byref(out), C.byref(size),
                               skipped.ctypes.data, torch.cuda.current_stream().cuda_stream))
    data = bytes(C.string_at(out, size.value))
    lib.csdr_free_buffer(out)
    return data, [nme for nme, s in zip(names, skipped) if s]


__all__ = ["encode", "init_dictionary", "compress", "source_decode", "compress_source",
           "hsda_build"]
