"""Byte formats of the compressed-weight path (host side, numpy).

HSDR v2 (binary codes) -- the reference's strategy-5 payload:
    header (36 B, packed little-endian; HierarchicalSDRStrategy.cpp:49-66)
        magic "HSDR", u32 version=2, u32 rows, u32 cols, u32 n_tiles,
        u16 tile_rows, u16 tile_cols, u16 n_atoms, u8 n_stages, u8 k_per_stage,
        f32 stage_decay, u32 edge_bytes
    f32 gamma[n_stages]; f32 D[n_atoms * tile_rows * tile_cols];
    u16 packed[n_tiles * n_stages * k]  ((sign << 15) | index, :76-84)
    f32 edge[...]  (top-right strip R_full x (C - C_full), then bottom strip, :68-72)

HSDB v1 (block-coded, fp16 coefficients) -- this build's extension for the research
"fused_real" codes (exp_c_kernel/benchmark.py:46-130): the same header with magic "HSDB",
version 1, tile_rows = 1 and tile_cols = the block length B; after the packed codes comes
one u16 per slot holding the fp16 bits of |c| (sign lives in the packed code), then the
edge strip. Coefficient of slot j of a tile = gamma[j // k] * (-1 if sign else 1) * |c|.
A binary HSDR stream with tile_rows == 1 converts losslessly (|c| = 1.0).

Q4_K super-block (144 B): f16 d, f16 dmin, u8 scales12[12], u8 qs[128]
(SparseInferenceEngine.cpp:362-384; scale/min packing :266-274).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np

HEADER = struct.Struct("<4sIIIIHHHBBfI")
assert HEADER.size == 36


@dataclass
class HsdrHeader:
    magic: bytes
    version: int
    rows: int
    cols: int
    n_tiles: int
    tile_rows: int
    tile_cols: int
    n_atoms: int
    n_stages: int
    k_per_stage: int
    stage_decay: float
    edge_bytes: int

    @property
    def slots(self) -> int:
        return self.n_stages * self.k_per_stage

    @property
    def is_hsdb(self) -> bool:
        return self.magic == b"HSDB"


def parse_header(stream: bytes) -> HsdrHeader:
    if len(stream) < HEADER.size:
        raise ValueError("stream shorter than the 36-byte header")
    return HsdrHeader(*HEADER.unpack_from(stream, 0))


def pack_hsdb(rows: int, cols: int, D: np.ndarray, idx: np.ndarray, coef: np.ndarray,
              gamma=(1.0,), n_stages: int = 1, edge: np.ndarray | None = None,
              block: int | None = None) -> bytes:
    """Serialise a block-coded matrix.

    D: (K, B) fp32 dictionary. idx: (n_tiles, slots) atom indices (< K, < 2^15).
    coef: (n_tiles, slots) signed coefficients; stored as sign bit + fp16 |c|
    (round-to-nearest-even). n_tiles = rows * (cols // B), tile (r, b) at r * NB + b.
    edge: (rows, cols - C_full) fp32 strip, required when cols % B != 0.
    """
    D = np.ascontiguousarray(D, np.float32)
    K, B = D.shape
    if block is not None and block != B:
        raise ValueError("dictionary width must equal the block length")
    NB = cols // B
    c_full = NB * B
    idx = np.ascontiguousarray(idx).reshape(rows * NB, -1)
    slots = idx.shape[1]
    if slots % n_stages:
        raise ValueError("slots per tile must be a multiple of n_stages")
    k = slots // n_stages
    coef = np.asarray(coef).reshape(rows * NB, slots)
    if np.any(idx >= K) or np.any(idx < 0) or K > 32768:
        raise ValueError("atom index out of range")
    c16 = coef.astype(np.float16)
    sign = np.signbit(c16).astype(np.uint16)
    packed = (idx.astype(np.uint16) & 0x7FFF) | (sign << 15)
    mag = np.abs(c16).view(np.uint16)
    ce = cols - c_full
    if ce:
        if edge is None:
            raise ValueError("cols is not a multiple of the block length: edge strip needed")
        edge = np.ascontiguousarray(edge, np.float32).reshape(rows, ce)
    else:
        edge = np.zeros((rows, 0), np.float32)
    gamma = np.asarray(gamma, np.float32).reshape(n_stages)
    hdr = HEADER.pack(b"HSDB", 1, rows, cols, rows * NB, 1, B, K, n_stages, k,
                      float(gamma[1] / gamma[0]) if n_stages > 1 and gamma[0] else 1.0,
                      edge.nbytes)
    return b"".join([hdr, gamma.tobytes(), D.tobytes(), packed.astype("<u2").tobytes(),
                     mag.astype("<u2").tobytes(), edge.tobytes()])


def hsdr_to_hsdb(stream: bytes) -> bytes:
    """Lossless conversion of a 1-row-tile binary HSDR stream into HSDB (|c| = 1.0)."""
    h = parse_header(stream)
    if h.magic != b"HSDR" or h.version != 2:
        raise ValueError("not an HSDR v2 stream")
    if h.tile_rows != 1:
        raise ValueError("only 1-row tiles convert to HSDB")
    n_codes = h.n_tiles * h.slots
    off_codes = HEADER.size + 4 * h.n_stages + 4 * h.n_atoms * h.tile_cols
    off_edge = off_codes + 2 * n_codes
    hdr = HEADER.pack(b"HSDB", 1, h.rows, h.cols, h.n_tiles, h.tile_rows, h.tile_cols,
                      h.n_atoms, h.n_stages, h.k_per_stage, h.stage_decay, h.edge_bytes)
    ones = np.full(n_codes, 0x3C00, "<u2").tobytes()
    return b"".join([hdr, stream[HEADER.size:off_edge], ones,
                     stream[off_edge:off_edge + h.edge_bytes]])


def hsdb_unpack(stream: bytes):
    """(idx, sign, |c| fp16 bits, gamma) arrays of an HSDB/HSDR stream, stream order."""
    h = parse_header(stream)
    n_codes = h.n_tiles * h.slots
    off = HEADER.size
    gamma = np.frombuffer(stream, "<f4", h.n_stages, off)
    off += 4 * h.n_stages + 4 * h.n_atoms * h.tile_rows * h.tile_cols
    packed = np.frombuffer(stream, "<u2", n_codes, off)
    off += 2 * n_codes
    if h.is_hsdb:
        mag = np.frombuffer(stream, "<u2", n_codes, off)
    else:
        mag = np.full(n_codes, 0x3C00, np.uint16)
    return packed & 0x7FFF, packed >> 15, mag, gamma


# ------------------------------------------------------------------------ Q4_K

Q4K_BLOCK_BYTES = 144
Q4K_BLOCK_VALUES = 256


def pack_q4k_scales(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """Pack 8 six-bit scales and mins per block into the 12-byte field.

    Inverse of the unpack at SparseInferenceEngine.cpp:266-274: for j < 4 the low 6 bits
    of bytes j / j+4; for j >= 4 the low nibbles of byte j+4 plus the top 2 bits of bytes
    j-4 / j. sc, mn: (n_blocks, 8) uint8 in [0, 63]. Returns (n_blocks, 12) uint8.
    """
    sc = np.asarray(sc, np.uint8)
    mn = np.asarray(mn, np.uint8)
    out = np.zeros((sc.shape[0], 12), np.uint8)
    out[:, 0:4] = (sc[:, 0:4] & 0x3F) | ((sc[:, 4:8] >> 4) << 6)
    out[:, 4:8] = (mn[:, 0:4] & 0x3F) | ((mn[:, 4:8] >> 4) << 6)
    out[:, 8:12] = (sc[:, 4:8] & 0x0F) | ((mn[:, 4:8] & 0x0F) << 4)
    return out


def pack_q4k(d16: np.ndarray, dmin16: np.ndarray, sc: np.ndarray, mn: np.ndarray,
             q: np.ndarray, order: str = "ggml") -> bytes:
    """Serialise Q4_K super-blocks.

    d16/dmin16: (n,) fp16 bit patterns (uint16); sc/mn: (n, 8) in [0, 63];
    q: (n, 256) 4-bit values in super-block element order.
    order "ggml": per 32-byte group g, low nibbles = elements of sub-block 2g, high
    nibbles = sub-block 2g+1 (engine/SDK path). order "interleaved": element i in byte i//2,
    low nibble when i is even (HSDR compress-side dequant).
    """
    n = q.shape[0]
    q = np.asarray(q, np.uint8).reshape(n, 256)
    if order == "ggml":
        g = q.reshape(n, 4, 2, 32)
        qs = (g[:, :, 0, :] | (g[:, :, 1, :] << 4)).reshape(n, 128)
    elif order == "interleaved":
        qs = (q[:, 0::2] | (q[:, 1::2] << 4)).reshape(n, 128)
    else:
        raise ValueError("order must be 'ggml' or 'interleaved'")
    blk = np.zeros((n, 144), np.uint8)
    blk[:, 0:2] = np.asarray(d16, "<u2").reshape(n, 1).view(np.uint8)
    blk[:, 2:4] = np.asarray(dmin16, "<u2").reshape(n, 1).view(np.uint8)
    blk[:, 4:16] = pack_q4k_scales(sc, mn)
    blk[:, 16:144] = qs
    return blk.tobytes()


# ------------------------------------------------------------------ .sdr archive writer

# SegmentType (core/ModelSegment.hpp:35-55), stored as u8 in the archive index.
SEGMENT_TYPES = {
    "UNKNOWN": 0, "WEIGHTS_FP32": 1, "WEIGHTS_FP16": 2, "WEIGHTS_INT8": 3, "WEIGHTS_INT4": 4,
    "SPARSE_INDICES": 5, "METADATA_JSON": 6, "METADATA_TOML": 7, "TOKENIZER_VOCAB": 8,
    "TOKENIZER_MODEL": 9, "CONFIG": 10, "ATTENTION_WEIGHTS": 11, "FEED_FORWARD_WEIGHTS": 12,
    "EMBEDDING_WEIGHTS": 13, "LAYER_NORM_WEIGHTS": 14, "MODEL_INPUT": 15, "MODEL_OUTPUT": 16,
    "GRAPH_STRUCTURE_PROTO": 17,
}

HSDR_STRATEGY_ID = 5


@dataclass
class SdrEntry:
    """One segment of a .sdr archive (CompressedSegmentHeader, core/AICompressor.hpp:51-65)."""
    name: str
    payload: bytes
    strategy_id: int = 0
    data_format: str = "f32"
    layer_type: str = ""
    original_type: int = 1
    original_size: int | None = None
    layer_name: str = ""
    layer_index: int = 0
    dims: tuple | None = None
    sparsity: float = 0.0
    input_shape: tuple = ()
    output_shape: tuple = ()
    sorted_indices: bool = False       # metadata fields written only with dims (has_metadata)
    scale: float | None = None
    zero_point: float | None = None


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<I", len(b)) + b


def write_sdr(path: str, entries, version: int = 2) -> None:
    """A .sdr archive as AICompressor::compressModel writes it (AICompressor.cpp:233-309):
    magic "CORTEXSR", u32 version, u64 segment count, u64 index offset, the payloads, then
    the index (strings u32-length-prefixed, bools one byte)."""
    out = bytearray(b"CORTEXSR" + struct.pack("<IQQ", version, len(entries), 0))
    offsets = []
    for e in entries:
        offsets.append(len(out))
        out += bytes(e.payload)
    index_off = len(out)
    for e, off in zip(entries, offsets):
        out += _str(e.name)
        if version >= 2:
            out += _str(e.data_format)
        out += _str(e.layer_type)
        orig = e.original_size if e.original_size is not None else len(e.payload)
        out += struct.pack("<BBQQQ", e.original_type, e.strategy_id, orig, len(e.payload), off)
        out += _str(e.layer_name)
        out += struct.pack("<I", e.layer_index)
        if e.dims is not None:
            out += struct.pack("<BB", 1, len(e.dims))
            out += struct.pack(f"<{len(e.dims)}I", *e.dims)
            out += struct.pack("<fB", e.sparsity, 1 if e.sorted_indices else 0)
            for opt in (e.scale, e.zero_point):
                out += struct.pack("<Bf", 1, opt) if opt is not None else b"\x00"
        else:
            out += b"\x00"
        for shape in (e.input_shape, e.output_shape):
            if shape:
                out += struct.pack("<BB", 1, len(shape)) + struct.pack(f"<{len(shape)}I", *shape)
            else:
                out += b"\x00"
    struct.pack_into("<Q", out, 20, index_off)
    with open(path, "wb") as f:
        f.write(out)


def hsdb_entry(name: str, stream: bytes, **kw) -> SdrEntry:
    """A strategy-5 entry for an HSDR/HSDB stream (dims from its header)."""
    h = parse_header(stream)
    return SdrEntry(name=name, payload=stream, strategy_id=HSDR_STRATEGY_ID, data_format="f32",
                    original_size=h.rows * h.cols * 4, dims=(h.rows, h.cols), **kw)


def vector_entry(name: str, v: np.ndarray, original_type: int = 14) -> SdrEntry:
    v = np.ascontiguousarray(v, np.float32)
    return SdrEntry(name=name, payload=v.tobytes(), original_type=original_type, dims=(v.size,))


def decoder_entries(weights) -> list:
    """The segments of a DecoderWeights under GGUF tensor names (token_embd, output_norm,
    output, blk.N.attn_q ... ffn_down), the names discover_native_llm_paths keys on
    (api/cortex_sdk.cpp:477-545). Tied embeddings: token_embd holds the lm_head codes; a
    separate embedding goes to token_embd and the lm_head to output."""
    names = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output",
             "gate": "ffn_gate", "up": "ffn_up", "down": "ffn_down"}
    if weights.embedding is None:
        ents = [hsdb_entry("token_embd.weight", weights.lm_head, original_type=13)]
    else:
        ents = [hsdb_entry("token_embd.weight", weights.embedding, original_type=13),
                hsdb_entry("output.weight", weights.lm_head, original_type=11)]
    if weights.final_norm is not None:
        ents.append(vector_entry("output_norm.weight", weights.final_norm))
    for l, L in enumerate(weights.layers):
        ents.append(vector_entry(f"blk.{l}.attn_norm.weight", L["attn_norm"]))
        for key in ("q", "k", "v", "o"):
            ents.append(hsdb_entry(f"blk.{l}.{names[key]}.weight", L[key], original_type=11,
                                   layer_index=l))
        ents.append(vector_entry(f"blk.{l}.ffn_norm.weight", L["ffn_norm"]))
        for key in ("gate", "up", "down"):
            ents.append(hsdb_entry(f"blk.{l}.{names[key]}.weight", L[key], original_type=12,
                                   layer_index=l))
    return ents
