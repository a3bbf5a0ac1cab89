"""Pins the oracle's restatement of the engine's GGUF block decode (oracle.gguf_dequant,
SparseInferenceEngine.cpp decodeSupportedGGUFQuantized :276-469) before the device kernels
are checked against it.

  * q4_0 / q8_0: bit-exact against the reference's own dequantizeToFP32 (compiled from its
    sources; tests/golden/ref_fixtures.npz), whose decode of these two formats is the engine's;
  * q4_1 / q5_0 / q5_1 / q8_1 / q8_k and the generic packed-bit rule: hand-built blocks whose
    values follow from the format's definition (scales exact in fp16, products exact);
  * q6_k: blocks with one scale throughout decode like ggml's Q6_K (a separately written
    decoder of the public layout), and a round trip through an encoder of the reference's
    element order (its quarter scales 0, 2, 4, 6);
  * the linear: fp64 brute force over the oracle's own dequantised rows.
The engine's path has no test in the reference, so these closed forms are the pin.
"""
import numpy as np
import pytest

import oracle
from conftest import rel_l2

F = oracle.GGUF_FORMATS


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def f16b(v):
    return np.array([np.float16(v)], np.float16).view(np.uint8)


@pytest.mark.parametrize("key,fmt", [("q40", "q4_0"), ("q80", "q8_0")])
def test_matches_reference_bitexact(golden, key, fmt):
    out = oracle.gguf_dequant(golden[f"{key}_blocks"].ravel(), F[fmt])
    assert np.array_equal(bits(out), bits(golden[f"{key}_ref"]))


def test_block_table():
    # ggufBlockBytesForFormat / ggufBlockElementsForFormat (SparseInferenceEngine.cpp:181-231)
    want = {"q4_0": (18, 32), "q4_1": (20, 32), "q5_0": (22, 32), "q5_1": (24, 32),
            "q8_0": (34, 32), "q8_1": (40, 32), "q2_k": (84, 256), "q3_k": (110, 256),
            "q4_k": (144, 256), "q5_k": (176, 256), "q6_k": (210, 256), "q8_k": (292, 256),
            "iq4_nl": (18, 32), "q4_0_4_4": (72, 128), "tq1_0": (54, 256)}
    for name, bb_be in want.items():
        assert oracle.gguf_block(F[name]) == bb_be, name


def test_q4_1_closed_form():
    blk = np.zeros(20, np.uint8)
    blk[0:2], blk[2:4] = f16b(0.5), f16b(-1.0)
    nibs = np.arange(32) % 16
    for i in range(16):
        blk[4 + i] = nibs[2 * i] | (nibs[2 * i + 1] << 4)   # element i: byte i/2, low if even
    out = oracle.gguf_dequant(blk, F["q4_1"])
    assert np.array_equal(out, (nibs * 0.5 - 1.0).astype(np.float32))


@pytest.mark.parametrize("fmt", ["q5_0", "q5_1"])
def test_q5_closed_form(fmt):
    has_m = fmt == "q5_1"
    blk = np.zeros(24 if has_m else 22, np.uint8)
    blk[0:2] = f16b(0.25)
    if has_m:
        blk[2:4] = f16b(2.0)
    q = (np.arange(32) * 7) % 32                       # 5-bit values
    qh = sum(int(q[i] >> 4) << i for i in range(32))   # bit i of the u32 = high bit of element i
    o = 4 if has_m else 2
    blk[o:o + 4] = np.array([qh], "<u4").view(np.uint8)
    for i in range(16):
        blk[o + 4 + i] = (q[2 * i] & 15) | ((q[2 * i + 1] & 15) << 4)
    out = oracle.gguf_dequant(blk, F[fmt])
    want = q * 0.25 + 2.0 if has_m else (q - 16) * 0.25
    assert np.array_equal(out, want.astype(np.float32))


def test_q8_1_and_q8_k_closed_form():
    vals = np.arange(-16, 16, dtype=np.int8)
    b1 = np.zeros(40, np.uint8)
    b1[0:4] = np.array([0.125], "<f4").view(np.uint8)   # fp32 scale (the reference's read)
    b1[8:40] = vals.view(np.uint8)
    assert np.array_equal(oracle.gguf_dequant(b1, F["q8_1"]), vals * np.float32(0.125))
    bk = np.zeros(292, np.uint8)
    bk[0:2] = f16b(-2.0)
    v256 = (np.arange(256) - 128).astype(np.int8)
    bk[4:260] = v256.view(np.uint8)
    assert np.array_equal(oracle.gguf_dequant(bk, F["q8_k"]), v256 * np.float32(-2.0))


@pytest.mark.parametrize("fmt,bb,be,nb", [("q2_k", 84, 256, 2), ("q3_k", 110, 256, 3),
                                          ("q5_k", 176, 256, 5), ("iq1_s", 50, 256, 1),
                                          ("q4_0_4_4", 72, 128, 4)])
def test_packed_rule_closed_form(fmt, bb, be, nb):
    rng = np.random.default_rng(3)
    q = rng.integers(0, 1 << nb, be)
    packed = np.zeros((be * nb + 7) // 8, np.uint8)
    for i, v in enumerate(q):                           # LSB-first bit stream
        for k in range(nb):
            if (v >> k) & 1:
                packed[(i * nb + k) // 8] |= 1 << ((i * nb + k) % 8)
    for d, dd in ((1.5, 1.5), (float("nan"), 1.0), (0.0, 1.0), (float("inf"), 1.0)):
        blk = np.zeros(bb, np.uint8)
        blk[0:2] = f16b(d)
        blk[bb - packed.size:] = packed                 # data at the end of the block
        out = oracle.gguf_dequant(blk, F[fmt])
        assert np.array_equal(out, ((q - (1 << (nb - 1))) * dd).astype(np.float32)), d


def ggml_q6k(blk):
    """ggml's public Q6_K layout (per-16 scales), written independently of the oracle."""
    ql, qh = blk[0:128].astype(np.int32), blk[128:192].astype(np.int32)
    sc = blk[192:208].view(np.int8).astype(np.int32)
    d = np.float32(blk[208:210].view(np.float16)[0])
    y = np.zeros(256, np.float32)
    for n in range(2):
        for l in range(32):
            is_ = l // 16
            q1 = ((ql[64 * n + l] & 0xF) | (((qh[32 * n + l] >> 0) & 3) << 4)) - 32
            q2 = ((ql[64 * n + l + 32] & 0xF) | (((qh[32 * n + l] >> 2) & 3) << 4)) - 32
            q3 = ((ql[64 * n + l] >> 4) | (((qh[32 * n + l] >> 4) & 3) << 4)) - 32
            q4 = ((ql[64 * n + l + 32] >> 4) | (((qh[32 * n + l] >> 6) & 3) << 4)) - 32
            s = sc[8 * n:]
            y[128 * n + l + 0] = d * np.float32(s[is_ + 0] * q1)
            y[128 * n + l + 32] = d * np.float32(s[is_ + 2] * q2)
            y[128 * n + l + 64] = d * np.float32(s[is_ + 4] * q3)
            y[128 * n + l + 96] = d * np.float32(s[is_ + 6] * q4)
    return y


def test_q6k_uniform_scales_match_ggml_layout():
    rng = np.random.default_rng(5)
    for _ in range(4):
        blk = rng.integers(0, 256, 210, dtype=np.uint8)
        blk[192:208] = np.int8(rng.integers(-40, 40)).view(np.uint8)
        blk[208:210] = f16b(0.0625)
        assert np.array_equal(oracle.gguf_dequant(blk, F["q6_k"]), ggml_q6k(blk))


def test_q6k_encoder_round_trip():
    """Encode 6-bit values in the reference's element order, decode, compare; the scales
    differ per 16, so the reference's use of scales 0/2/4/6 per quarter is what is checked."""
    rng = np.random.default_rng(6)
    q = rng.integers(0, 64, 256)
    sc = rng.integers(-60, 60, 16).astype(np.int8)
    blk = np.zeros(210, np.uint8)
    for e in range(256):
        half, r = divmod(e, 128)
        t, l = divmod(r, 32)
        lo, hi = q[e] & 15, q[e] >> 4
        byte = 64 * half + l + (32 if t in (1, 3) else 0)
        blk[byte] |= lo << (4 if t >= 2 else 0)
        blk[128 + 32 * half + l] |= hi << (2 * t)
    blk[192:208] = sc.view(np.uint8)
    blk[208:210] = f16b(0.5)
    out = oracle.gguf_dequant(blk, F["q6_k"])
    e = np.arange(256)
    s = sc.astype(np.int32)[8 * (e // 128) + 2 * ((e % 128) // 32)]
    assert np.array_equal(out, (np.float32(0.5) * (s * (q - 32)).astype(np.float32)))


@pytest.mark.parametrize("fmt", ["q4_0", "q6_k", "q5_1", "q2_k"])
def test_linear_brute_force(fmt):
    rng = np.random.default_rng(9)
    bb, be = oracle.gguf_block(F[fmt])
    R, Cc = 7, 2 * be
    w = rng.integers(0, 256, (R * Cc // be, bb), dtype=np.uint8)
    off = 208 if fmt == "q6_k" else 0
    w[:, off:off + 2] = f16b(0.01)
    x = rng.normal(size=(3, Cc)).astype(np.float32)
    W = oracle.gguf_dequant(w.ravel(), F[fmt]).reshape(R, Cc).astype(np.float64)
    y = oracle.gguf_linear(w.ravel(), F[fmt], R, Cc, x)
    assert rel_l2(y, x.astype(np.float64) @ W.T) < 1e-6
