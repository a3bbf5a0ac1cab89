"""CPU oracle for the cortexSDR compressed-weight inference path.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker or the reported CPU
baseline. The product package ``cortexsdr_amd`` never imports it.

Two libraries are wrapped:

* ``liborc.so`` -- this repo's C restatement (``csdr_oracle.c``), each function citing the
  reference file:line it follows.
* ``_ref/libcsdr_ref.so`` -- the reference's own HSDR codec and attention kernels compiled
  from the reference sources by ``oracle/Makefile`` (present only where it was built;
  ``ref()`` returns None otherwise).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBORC = os.path.join(HERE, "liborc.so")
LIBREF = os.path.join(HERE, "_ref", "libcsdr_ref.so")

_orc = None
_ref = None

ORC_Q4K_GGML = 0
ORC_Q4K_INTERLEAVED = 1

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_sz = C.c_size_t


def build(ref: bool = False) -> None:
    """Compile liborc.so (and, with ref=True, the reference build) via oracle/Makefile."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    if ref:
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


class OrcHsdrView(C.Structure):
    _fields_ = [
        ("is_hsdb", C.c_int),
        ("version", C.c_uint32), ("rows", C.c_uint32), ("cols", C.c_uint32),
        ("n_tiles", C.c_uint32),
        ("tile_rows", C.c_uint32), ("tile_cols", C.c_uint32), ("n_atoms", C.c_uint32),
        ("n_stages", C.c_uint32), ("k_per_stage", C.c_uint32),
        ("stage_decay", C.c_float),
        ("edge_bytes", C.c_uint32),
        ("slots_per_tile", _sz), ("n_codes", _sz),
        ("off_gamma", _sz), ("off_dict", _sz), ("off_packed", _sz), ("off_coef", _sz),
        ("off_edge", _sz), ("end", _sz),
    ]


def orc():
    """The restatement library (built on first use if missing)."""
    global _orc
    if _orc is None:
        if not os.path.exists(LIBORC):
            build()
        L = C.CDLL(LIBORC)
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16_array.argtypes = [_f32p, _u16p, _sz]
        L.orc_f16_to_f32_array.argtypes = [_u16p, _f32p, _sz]
        L.orc_hsdr_parse.argtypes = [_u8p, _sz, C.POINTER(OrcHsdrView)]
        L.orc_hsdr_unpack.argtypes = [_u8p, _sz, _u16p, _i8p, _f32p]
        L.orc_hsdr_decompress.argtypes = [_u8p, _sz, _f32p, _sz]
        L.orc_hsdr_matmul_row_major.argtypes = [_u8p, _sz, _f32p, _sz, _f32p]
        L.orc_hsdb_matmul.argtypes = [_u8p, _sz, _f32p, _sz, _f32p]
        L.orc_set_threads.argtypes = [C.c_int]
        L.orc_set_threads.restype = C.c_int
        L.orc_q4k_dequant.argtypes = [_u8p, _sz, C.c_int, _f32p]
        L.orc_q5k_dequant.argtypes = [_u8p, _sz, _f32p]
        L.orc_q6k_dequant.argtypes = [_u8p, _sz, _f32p]
        L.orc_q4k_linear.argtypes = [_u8p, _sz, _sz, C.c_int, _f32p, _sz, _f32p]
        L.orc_gguf_block.argtypes = [C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int)]
        L.orc_gguf_dequant.argtypes = [_u8p, C.c_int, _sz, _f32p]
        L.orc_gguf_linear.argtypes = [_u8p, C.c_int, _sz, _sz, _f32p, _sz, _f32p]
        L.orc_mha_causal.argtypes = [_f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz, _sz]
        L.orc_attn_decode.argtypes = [_f32p, _u16p, _u16p, C.c_void_p, _sz, _sz, _sz, _sz,
                                      _sz, C.c_float, _f32p]
        L.orc_rms_norm.argtypes = [_f32p, _f32p, _sz, _sz, C.c_float, _f32p]
        L.orc_silu_mul.argtypes = [_f32p, _f32p, _sz, _f32p]
        L.orc_rope.argtypes = [_f32p, _sz, _sz, _sz, C.c_float, _sz]
        L.orc_select_best.argtypes = [_f32p, _sz, C.c_void_p, C.c_float, C.c_float]
        L.orc_hsdr_mp.argtypes = [_f32p, _sz, _sz, _f32p, _sz, _sz, _sz, _f32p, _u16p]
        L.orc_hsdr_mp.restype = None
        L.orc_select_best.restype = C.c_int
        L.orc_lazy_hsdr_info.argtypes = [_u8p, _sz, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)]
        L.orc_lazy_hsdr_decode_row.argtypes = [_u8p, _sz, C.c_int, C.c_uint32, _f32p]
        L.orc_lazy_hsdr_select.argtypes = [_u8p, _sz, C.c_int, _f32p, C.c_void_p, C.c_float,
                                           C.c_float, _f32p, C.POINTER(C.c_int)]
        _orc = L
    return _orc


def ref():
    """The reference build (oracle/_ref), or None where it was not built."""
    global _ref
    if _ref is None and os.path.exists(LIBREF):
        L = C.CDLL(LIBREF)
        L.ref_last_error.restype = C.c_char_p
        L.ref_hsdr_compress.argtypes = [_f32p, C.c_uint32, C.c_uint32, C.c_uint16, C.c_uint16,
                                        C.c_uint16, C.c_uint8, C.c_uint8, C.c_uint8, C.c_float,
                                        C.POINTER(C.POINTER(C.c_uint8)), C.POINTER(_sz)]
        L.ref_free.argtypes = [C.c_void_p]
        L.ref_hsdr_decompress.argtypes = [_u8p, _sz, _f32p, _sz]
        L.ref_hsdr_matmul_row_major.argtypes = [_u8p, _sz, _f32p, _sz, _f32p, _sz]
        L.ref_dequant.argtypes = [_u8p, _sz, C.c_char_p, C.c_uint32, C.c_uint32, _f32p, _sz]
        L.ref_mha.argtypes = [_f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, C.c_int]
        L.ref_flash_attention.argtypes = [_f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz, _sz,
                                          C.c_int]
        L.ref_hsda_build.argtypes = [C.c_uint32, C.POINTER(C.c_char_p), C.POINTER(C.c_void_p),
                                     C.POINTER(C.c_uint32), C.c_uint32, C.c_uint16, C.c_uint8,
                                     C.c_uint8, C.c_uint8, C.c_float,
                                     C.POINTER(C.POINTER(C.c_uint8)), C.POINTER(_sz)]
        L.ref_hsda_build_ex.argtypes = [C.c_uint32, C.POINTER(C.c_char_p),
                                        C.POINTER(C.c_void_p), C.POINTER(C.c_uint32),
                                        C.POINTER(C.c_uint32), C.c_uint16, C.c_uint16,
                                        C.c_uint16, C.c_uint8, C.c_uint8, C.c_uint8, C.c_float,
                                        C.c_uint32, C.c_void_p,
                                        C.POINTER(C.POINTER(C.c_uint8)), C.POINTER(_sz)]
        L.ref_hsda_matmul.argtypes = [_u8p, _sz, C.c_char_p, _f32p, _sz, _f32p, _sz]
        L.ref_hsda_decompress.argtypes = [_u8p, _sz, C.c_char_p, _f32p, _sz]
        _ref = L
    return _ref


# ------------------------------------------------------------------ numpy helpers

def _u8(buf) -> np.ndarray:
    return np.ascontiguousarray(np.frombuffer(bytes(buf), dtype=np.uint8))


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"oracle {what} failed with status {rc}")


def f32_to_f16(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32).ravel()
    out = np.empty(a.size, np.uint16)
    orc().orc_f32_to_f16_array(a, out, a.size)
    return out


def f16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16).ravel()
    out = np.empty(h.size, np.float32)
    orc().orc_f16_to_f32_array(h, out, h.size)
    return out


def hsdr_parse(stream) -> OrcHsdrView:
    b = _u8(stream)
    v = OrcHsdrView()
    rc = orc().orc_hsdr_parse(b, b.size, C.byref(v))
    if rc:
        raise ValueError(f"oracle parse failed: {rc}")
    return v


def hsdr_parse_status(stream) -> int:
    b = _u8(stream)
    v = OrcHsdrView()
    return orc().orc_hsdr_parse(b, b.size, C.byref(v))


def hsdr_unpack(stream):
    b = _u8(stream)
    v = hsdr_parse(b)
    idx = np.empty(v.n_codes, np.uint16)
    sign = np.empty(v.n_codes, np.int8)
    coef = np.empty(v.n_codes, np.float32)
    _check(orc().orc_hsdr_unpack(b, b.size, idx, sign, coef), "unpack")
    return idx, sign, coef


def hsdr_decompress(stream) -> np.ndarray:
    b = _u8(stream)
    v = hsdr_parse(b)
    out = np.zeros(v.rows * v.cols, np.float32)
    _check(orc().orc_hsdr_decompress(b, b.size, out, out.size), "decompress")
    return out.reshape(v.rows, v.cols)


def hsdr_matmul_row_major(stream, x: np.ndarray) -> np.ndarray:
    b = _u8(stream)
    v = hsdr_parse(b)
    x = np.ascontiguousarray(x, np.float32)
    batch = x.shape[1] if x.ndim == 2 else 1
    y = np.zeros(v.rows * batch, np.float32)
    _check(orc().orc_hsdr_matmul_row_major(b, b.size, x.ravel(), batch, y), "matmul")
    return y.reshape(v.rows, batch)


def hsdb_matmul(stream, x: np.ndarray) -> np.ndarray:
    """A0 fused block-coded matmul; x is (C, M) fp32, returns (R, M)."""
    b = _u8(stream)
    v = hsdr_parse(b)
    x = np.ascontiguousarray(x, np.float32)
    M = x.shape[1] if x.ndim == 2 else 1
    y = np.zeros(v.rows * M, np.float32)
    _check(orc().orc_hsdb_matmul(b, b.size, x.ravel(), M, y), "hsdb_matmul")
    return y.reshape(v.rows, M)


def q4k_dequant(blocks, order: int = ORC_Q4K_GGML) -> np.ndarray:
    b = _u8(blocks)
    nb = b.size // 144
    out = np.empty(nb * 256, np.float32)
    orc().orc_q4k_dequant(b, nb, order, out)
    return out


def q5k_dequant(blocks) -> np.ndarray:
    b = _u8(blocks)
    out = np.empty(b.size // 176 * 256, np.float32)
    orc().orc_q5k_dequant(b, b.size // 176, out)
    return out


def q6k_dequant(blocks) -> np.ndarray:
    b = _u8(blocks)
    out = np.empty(b.size // 210 * 256, np.float32)
    orc().orc_q6k_dequant(b, b.size // 210, out)
    return out


def q4k_linear(w, R: int, Cc: int, x: np.ndarray, order: int = ORC_Q4K_GGML) -> np.ndarray:
    """y (M, R) = x (M, C) . dequant(W)^T."""
    b = _u8(w)
    x = np.ascontiguousarray(x, np.float32)
    M = x.shape[0] if x.ndim == 2 else 1
    y = np.zeros(M * R, np.float32)
    _check(orc().orc_q4k_linear(b, R, Cc, order, x.ravel(), M, y), "q4k_linear")
    return y.reshape(M, R)


# engine GGUF formats (ids = ggml type numbers; include/cortexsdr_hip.h CSDR_GGUF_*)
GGUF_FORMATS = {"q4_0": 2, "q4_1": 3, "q5_0": 6, "q5_1": 7, "q8_0": 8, "q8_1": 9, "q2_k": 10,
                "q3_k": 11, "q4_k": 12, "q5_k": 13, "q6_k": 14, "q8_k": 15, "iq2_xxs": 16,
                "iq2_xs": 17, "iq3_xxs": 18, "iq1_s": 19, "iq4_nl": 20, "iq3_s": 21,
                "iq2_s": 22, "iq4_xs": 23, "iq1_m": 29, "q4_0_4_4": 31, "q4_0_4_8": 32,
                "q4_0_8_8": 33, "tq1_0": 34, "tq2_0": 35}


def gguf_block(fmt: int):
    """(bytes, elements) per block."""
    bb, be = C.c_int(0), C.c_int(0)
    _check(orc().orc_gguf_block(fmt, C.byref(bb), C.byref(be)), "gguf_block")
    return bb.value, be.value


def gguf_dequant(blocks, fmt: int) -> np.ndarray:
    b = _u8(blocks)
    bb, be = gguf_block(fmt)
    nb = b.size // bb
    out = np.empty(nb * be, np.float32)
    _check(orc().orc_gguf_dequant(b, fmt, nb, out), "gguf_dequant")
    return out


def gguf_linear(w, fmt: int, R: int, Cc: int, x: np.ndarray) -> np.ndarray:
    """y (M, R) = x (M, C) . dequant(W)^T."""
    b = _u8(w)
    x = np.ascontiguousarray(x, np.float32)
    M = x.shape[0] if x.ndim == 2 else 1
    y = np.zeros(M * R, np.float32)
    _check(orc().orc_gguf_linear(b, fmt, R, Cc, x.ravel(), M, y), "gguf_linear")
    return y.reshape(M, R)


def attn_decode(q, kcache_f16, vcache_f16, lens, Hq, Hkv, d, scale=None):
    """q (B, Hq, d) fp32; caches (B, T, Hkv, d) fp16 bits (uint16)."""
    q = np.ascontiguousarray(q, np.float32)
    kc = np.ascontiguousarray(kcache_f16, np.uint16)
    vc = np.ascontiguousarray(vcache_f16, np.uint16)
    B, T = kc.shape[0], kc.shape[1]
    out = np.zeros(B * Hq * d, np.float32)
    lp = None
    if lens is not None:
        lens = np.ascontiguousarray(lens, np.int32)
        lp = lens.ctypes.data_as(C.c_void_p)
    s = float(scale) if scale is not None else 1.0 / np.sqrt(d)
    orc().orc_attn_decode(q.ravel(), kc.ravel(), vc.ravel(), lp, B, T, Hq, Hkv, d, s, out)
    return out.reshape(B, Hq, d)


def mha_causal(q, k, v, heads):
    q = np.ascontiguousarray(q, np.float32)
    B, T, H = q.shape
    out = np.zeros_like(q)
    orc().orc_mha_causal(q.ravel(), np.ascontiguousarray(k, np.float32).ravel(),
                         np.ascontiguousarray(v, np.float32).ravel(), out.reshape(-1),
                         B, T, H, heads)
    return out


def rms_norm(x, w, eps=1e-5):
    x = np.ascontiguousarray(x, np.float32)
    n = x.shape[-1]
    y = np.empty_like(x)
    orc().orc_rms_norm(x.reshape(-1), np.ascontiguousarray(w, np.float32), x.size // n, n,
                       eps, y.reshape(-1))
    return y


def silu_mul(g, u):
    g = np.ascontiguousarray(g, np.float32)
    y = np.empty_like(g)
    orc().orc_silu_mul(g.reshape(-1), np.ascontiguousarray(u, np.float32).reshape(-1), g.size,
                       y.reshape(-1))
    return y


def rope(x, heads, head_dim, theta=1e6, pos0=0):
    x = np.array(x, np.float32, copy=True, order="C")
    ntok = x.size // (heads * head_dim)
    orc().orc_rope(x.reshape(-1), ntok, heads, head_dim, theta, pos0)
    return x


ORC_LAZY_PACKED, ORC_LAZY_CLI = 0, 1


def lazy_hsdr_info(stream):
    """(vocabulary rows, width) of an HSDR embedding as the text CLI's lazy parse reads it."""
    b = _u8(stream)
    r, c = C.c_uint32(), C.c_uint32()
    _check(orc().orc_lazy_hsdr_info(b, b.size, C.byref(r), C.byref(c)), "lazy parse")
    return r.value, c.value


def lazy_hsdr_decode_row(stream, row: int, unpack: int = ORC_LAZY_PACKED) -> np.ndarray:
    b = _u8(stream)
    _, cols = lazy_hsdr_info(b)
    out = np.zeros(cols, np.float32)
    _check(orc().orc_lazy_hsdr_decode_row(b, b.size, unpack, row, out), "lazy decode row")
    return out


def lazy_hsdr_select(stream, hidden, repeated=None, temperature=0.8, penalty=1.0,
                     unpack: int = ORC_LAZY_PACKED):
    """(token, raw scores) of the CLI's lazy HSDR vocabulary scoring."""
    b = _u8(stream)
    rows, _ = lazy_hsdr_info(b)
    h = np.ascontiguousarray(hidden, np.float32)
    scores = np.zeros(rows, np.float32)
    rp = None
    if repeated is not None:
        repeated = np.ascontiguousarray(repeated, np.uint8)
        rp = repeated.ctypes.data_as(C.c_void_p)
    tok = C.c_int()
    _check(orc().orc_lazy_hsdr_select(b, b.size, unpack, h, rp, temperature, penalty, scores,
                                      C.byref(tok)), "lazy select")
    return tok.value, scores


def select_best(logits, repeated=None, temperature=0.0, penalty=1.5) -> int:
    lg = np.ascontiguousarray(logits, np.float32)
    rp = None
    if repeated is not None:
        repeated = np.ascontiguousarray(repeated, np.uint8)
        rp = repeated.ctypes.data_as(C.c_void_p)
    return orc().orc_select_best(lg, lg.size, rp, temperature, penalty)


# ------------------------------------------------------------- shared-dictionary containers

HSDC_HEADER = "<4sIIIIHHHBBf"   # HSDRCodesHeader, HierarchicalSDRStrategy.cpp:680-691


def hsda_parse(data):
    """SharedDictArchive::readFromStream (HierarchicalSDRStrategy.cpp:2016-2063): returns
    (dictionaries, segments); a dictionary is a dict of its 20-byte HierarchicalSDRConfig
    fields (u16 tile_rows, tile_cols, n_atoms; u8 n_stages, k, ksvd_iters, pad; 2 padding
    bytes; f32 stage_decay; u32 max_tiles_for_fit), stage_scales and atoms; a segment is
    (name, dict_index, original_size, original_type, codes bytes)."""
    import struct

    b = bytes(data)
    if b[:4] != b"HSDA":
        raise ValueError("HSDA read: bad magic")
    version, nd, ns = struct.unpack_from("<III", b, 4)
    if version != 1:
        raise ValueError("HSDA read: unsupported version")
    off = 16
    dicts = []
    for _ in range(nd):
        tr, tc, K, S, k, iters, _pad = struct.unpack_from("<HHHBBBB", b, off)
        decay, _cap = struct.unpack_from("<fI", b, off + 12)
        off += 20
        (nsc,) = struct.unpack_from("<I", b, off)
        scales = np.frombuffer(b, np.float32, nsc, off + 4).copy()
        off += 4 + 4 * nsc
        (na,) = struct.unpack_from("<I", b, off)
        atoms = np.frombuffer(b, np.float32, na, off + 4).copy()
        off += 4 + 4 * na
        dicts.append(dict(tile_rows=tr, tile_cols=tc, n_atoms=K, n_stages=S, k=k,
                          stage_decay=decay, stage_scales=scales, atoms=atoms))
    segs = []
    for _ in range(ns):
        (nl,) = struct.unpack_from("<I", b, off)
        name = b[off + 4:off + 4 + nl].decode()
        off += 4 + nl
        di, orig, typ, cl = struct.unpack_from("<IQBI", b, off)
        off += 17
        segs.append((name, di, orig, typ, b[off:off + cl]))
        off += cl
    return dicts, segs


def hsdc_to_hsdr(codes, d) -> bytes:
    """An HSDC codes-only stream + its dictionary as the equivalent HSDR v2 stream: the
    dictionary's stage scales as gamma, its atoms as D, the packed codes unchanged, zero edge
    strips (decompressWithExternalDictionary leaves them zero, :1804-1828)."""
    import struct

    b = bytes(codes)
    mg, ver, R, Cc, nt, tr, tc, K, S, k, decay = struct.unpack_from(HSDC_HEADER, b, 0)
    if mg != b"HSDC" or ver != 1:
        raise ValueError("HSDR shared: bad codes-stream magic/version")
    if (tr, tc, K, S, k) != (d["tile_rows"], d["tile_cols"], d["n_atoms"], d["n_stages"], d["k"]):
        raise ValueError("HSDR shared: stream geometry doesn't match dictionary config")
    n_codes = nt * S * k
    hdr_n = struct.calcsize(HSDC_HEADER)
    Rf, Cf = R // tr * tr, Cc // tc * tc
    edge = (Rf * (Cc - Cf) + (R - Rf) * Cc) * 4
    head = struct.pack("<4sIIIIHHHBBfI", b"HSDR", 2, R, Cc, nt, tr, tc, K, S, k, decay, edge)
    return b"".join([head, np.asarray(d["stage_scales"][:S], np.float32).tobytes(),
                     np.asarray(d["atoms"], np.float32).tobytes(),
                     b[hdr_n:hdr_n + 2 * n_codes], bytes(edge)])


# ------------------------------------------------------------- reference build

def ref_hsda_build(mats: dict, n_atoms, n_stages, k_per_stage, ksvd_iters=4,
                   stage_decay=0.5) -> bytes:
    """{name: (R_i x C) fp32} -> HSDA bytes from the reference's compressGroupedSegments."""
    L = ref()
    names = list(mats)
    arrs = [np.ascontiguousarray(mats[n], np.float32) for n in names]
    Cc = arrs[0].shape[1]
    nm = (C.c_char_p * len(names))(*[n.encode() for n in names])
    ws = (C.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
    rows = (C.c_uint32 * len(arrs))(*[a.shape[0] for a in arrs])
    out = C.POINTER(C.c_uint8)()
    n = _sz()
    rc = L.ref_hsda_build(len(names), nm, ws, rows, Cc, n_atoms, n_stages, k_per_stage,
                          ksvd_iters, stage_decay, C.byref(out), C.byref(n))
    if rc:
        raise RuntimeError(L.ref_last_error().decode())
    data = bytes(C.string_at(out, n.value))
    L.ref_free(out)
    return data


def ref_hsda_build_ex(mats: dict, tile_rows, tile_cols, n_atoms, n_stages, k_per_stage,
                      ksvd_iters, stage_decay=0.5, max_tiles_for_fit=0):
    """{name: (R_i x C_i) fp32} -> (HSDA bytes, skipped flags) from the reference's
    compressGroupedSegments with the given tile geometry and fit-pool cap."""
    L = ref()
    names = list(mats)
    arrs = [np.ascontiguousarray(mats[n], np.float32) for n in names]
    nm = (C.c_char_p * len(names))(*[n.encode() for n in names])
    ws = (C.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
    rows = (C.c_uint32 * len(arrs))(*[a.shape[0] for a in arrs])
    cols = (C.c_uint32 * len(arrs))(*[a.shape[1] for a in arrs])
    skipped = np.zeros(len(arrs), np.uint8)
    out = C.POINTER(C.c_uint8)()
    n = _sz()
    rc = L.ref_hsda_build_ex(len(names), nm, ws, rows, cols, tile_rows, tile_cols, n_atoms,
                             n_stages, k_per_stage, ksvd_iters, stage_decay, max_tiles_for_fit,
                             skipped.ctypes.data, C.byref(out), C.byref(n))
    if rc:
        raise RuntimeError(L.ref_last_error().decode())
    data = bytes(C.string_at(out, n.value))
    L.ref_free(out)
    return data, skipped


def ref_hsda_matmul(data, name: str, x, R: int) -> np.ndarray:
    L = ref()
    b = _u8(data)
    x = np.ascontiguousarray(x, np.float32)
    batch = x.shape[1] if x.ndim == 2 else 1
    y = np.zeros(R * batch, np.float32)
    if L.ref_hsda_matmul(b, b.size, name.encode(), x.ravel(), batch, y, y.size):
        raise RuntimeError(L.ref_last_error().decode())
    return y.reshape(R, batch)


def ref_hsda_decompress(data, name: str, R: int, Cc: int) -> np.ndarray:
    L = ref()
    b = _u8(data)
    w = np.zeros(R * Cc, np.float32)
    if L.ref_hsda_decompress(b, b.size, name.encode(), w, w.size):
        raise RuntimeError(L.ref_last_error().decode())
    return w.reshape(R, Cc)


def ref_hsdr_compress(w: np.ndarray, tile_rows, tile_cols, n_atoms, n_stages, k_per_stage,
                      ksvd_iters=4, stage_decay=0.5) -> bytes:
    L = ref()
    w = np.ascontiguousarray(w, np.float32)
    R, Cc = w.shape
    out = C.POINTER(C.c_uint8)()
    n = _sz()
    rc = L.ref_hsdr_compress(w.ravel(), R, Cc, tile_rows, tile_cols, n_atoms, n_stages,
                             k_per_stage, ksvd_iters, stage_decay, C.byref(out), C.byref(n))
    if rc:
        raise RuntimeError(L.ref_last_error().decode())
    data = bytes(C.string_at(out, n.value))
    L.ref_free(out)
    return data


def ref_hsdr_decompress(stream, R, Cc) -> np.ndarray:
    L = ref()
    b = _u8(stream)
    out = np.zeros(R * Cc, np.float32)
    if L.ref_hsdr_decompress(b, b.size, out, out.size):
        raise RuntimeError(L.ref_last_error().decode())
    return out.reshape(R, Cc)


def ref_hsdr_matmul_row_major(stream, x, R) -> np.ndarray:
    L = ref()
    b = _u8(stream)
    x = np.ascontiguousarray(x, np.float32)
    batch = x.shape[1] if x.ndim == 2 else 1
    y = np.zeros(R * batch, np.float32)
    if L.ref_hsdr_matmul_row_major(b, b.size, x.ravel(), batch, y, y.size):
        raise RuntimeError(L.ref_last_error().decode())
    return y.reshape(R, batch)


def ref_dequant(data, fmt: str, R: int, Cc: int) -> np.ndarray:
    L = ref()
    b = _u8(data)
    out = np.zeros(R * Cc, np.float32)
    n = L.ref_dequant(b, b.size, fmt.encode(), R, Cc, out, out.size)
    if n < 0:
        raise RuntimeError(L.ref_last_error().decode())
    return out[:n]


def ref_mha(q, k, v, heads, causal=True, flash=False):
    L = ref()
    q = np.ascontiguousarray(q, np.float32)
    B, T, H = q.shape
    out = np.zeros_like(q)
    fn = L.ref_flash_attention if flash else L.ref_mha
    fn(q.ravel(), np.ascontiguousarray(k, np.float32).ravel(),
       np.ascontiguousarray(v, np.float32).ravel(), out.reshape(-1), B, T, H, heads,
       1 if causal else 0)
    return out


def hsdr_mp(tiles: np.ndarray, D: np.ndarray, gamma, S: int, k: int) -> np.ndarray:
    """Packed u16 codes (n_tiles x S*k) of hierarchical binary matching pursuit
    (hierarchicalBinaryCode, HierarchicalSDRStrategy.cpp:219-262) of tiles (n x C) against
    D (K x C) with stage scales gamma."""
    t = np.ascontiguousarray(tiles, np.float32)
    d = np.ascontiguousarray(D, np.float32)
    g = np.ascontiguousarray(gamma, np.float32)
    codes = np.zeros((t.shape[0], S * k), np.uint16)
    orc().orc_hsdr_mp(t.ravel(), t.shape[0], t.shape[1], d.ravel(), d.shape[0], S, k, g,
                      codes.ravel())
    return codes


def set_threads(n: int) -> int:
    """OpenMP threads of the restatement's parallel loops (previous setting returned)."""
    return int(orc().orc_set_threads(int(n)))
