"""Pins the CPU oracle (oracle/) before anything is checked against it.

Sources of truth, in order:
  * reference golden fixtures (tests/golden/ref_fixtures.npz, written by the reference's
    own HierarchicalSDRStrategy / attention code compiled from its sources);
  * the reference's known-answer K-quant vectors (src/test_hsdr_kquants.cpp:69-203);
  * closed forms and brute force (fp64 dense products, textbook softmax attention,
    rotation invariants, tie rules) for what the reference does not test.
"""
import numpy as np
import pytest

import oracle
from cortexsdr_amd import formats, synth
from conftest import rel_l2


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ------------------------------------------------------------ reference fixtures

@pytest.mark.parametrize("key", ["hsdr1d", "hsdr1de", "hsdr2d", "hsdr2db"])
def test_decompress_matches_reference_bitexact(golden, key):
    w = oracle.hsdr_decompress(golden[f"{key}_stream"])
    assert np.array_equal(bits(w), bits(golden[f"{key}_w"]))


@pytest.mark.parametrize("key", ["hsdr1d", "hsdr1de"])
def test_matmul_row_major_matches_reference_bitexact(golden, key):
    y = oracle.hsdr_matmul_row_major(golden[f"{key}_stream"], golden[f"{key}_x"])
    assert np.array_equal(bits(y), bits(golden[f"{key}_y"]))


@pytest.mark.parametrize("key", ["hsdr1d", "hsdr1de"])
def test_fused_equals_decompress_then_dense(golden, key):
    # test_hsdr_roundtrip.cpp:184-265 invariant (max |diff| < 1e-3), here in fp64
    w = golden[f"{key}_w"].astype(np.float64)
    x = golden[f"{key}_x"].astype(np.float64)
    y = oracle.hsdr_matmul_row_major(golden[f"{key}_stream"], golden[f"{key}_x"])
    assert np.abs(y - w @ x).max() < 1e-5


@pytest.mark.parametrize("key,fn", [
    ("q4k", lambda b: oracle.q4k_dequant(b, oracle.ORC_Q4K_INTERLEAVED)),
    ("q5k", oracle.q5k_dequant),
    ("q6k", oracle.q6k_dequant),
])
def test_kquant_dequant_matches_reference_bitexact(golden, key, fn):
    out = fn(golden[f"{key}_blocks"].ravel())
    assert np.array_equal(bits(out), bits(golden[f"{key}_ref"]))


def test_mha_matches_reference(golden):
    o = oracle.mha_causal(golden["mha_q"], golden["mha_k"], golden["mha_v"], 4)
    assert np.abs(o - golden["mha_out"]).max() < 1e-6
    assert np.abs(o - golden["mha_flash_out"]).max() < 1e-6


# ------------------------------------------------------ K-quant known answers

def _f16(v):
    return np.array([np.float16(v).view(np.uint16)], "<u2").view(np.uint8)


def test_q4k_known_answers():
    # src/test_hsdr_kquants.cpp:69-95 (d=1, dmin=0, sc[0]=1, qs = 0x21, 0x43)
    b = np.zeros(144, np.uint8)
    b[0:2], b[2:4] = _f16(1.0), _f16(0.0)
    b[4], b[8], b[16], b[17] = 0x01, 0x00, 0x21, 0x43
    out = oracle.q4k_dequant(b, oracle.ORC_Q4K_INTERLEAVED)
    assert list(out[:4]) == [1.0, 2.0, 3.0, 4.0]
    assert not out[4:].any()
    # :106-122 (d=2, dmin=1, sc=3, m=4, qs[0]=5) -> 26, -4
    b = np.zeros(144, np.uint8)
    b[0:2], b[2:4] = _f16(2.0), _f16(1.0)
    b[4], b[8], b[16] = 3, 4, 0x05
    out = oracle.q4k_dequant(b, oracle.ORC_Q4K_INTERLEAVED)
    assert out[0] == 26.0 and out[1] == -4.0


def test_q5k_q6k_known_answers():
    # :133-150 Q5_K -> 18, 0
    b = np.zeros(176, np.uint8)
    b[0:2], b[2:4] = _f16(1.0), _f16(0.0)
    b[4], b[16], b[48] = 1, 0x01, 0x02
    out = oracle.q5k_dequant(b)
    assert out[0] == 18.0 and out[1] == 0.0
    # :162-178 and :188-203 Q6_K -> -62, -60 / 34, -60
    for qh, e0 in ((0x00, -62.0), (0x03, 34.0)):
        b = np.zeros(210, np.uint8)
        b[0], b[128], b[192] = 0x21, qh, 2
        b[208:210] = _f16(1.0)
        out = oracle.q6k_dequant(b)
        assert out[0] == e0 and out[1] == -60.0


def test_q4k_ggml_order_closed_form():
    # engine order (SparseInferenceEngine.cpp:375-382): byte g*32+j low nibble is element
    # (2g)*32 + j, high nibble element (2g+1)*32 + j; hand-built: d=1, dmin=0, scales 1..8
    rng = np.random.default_rng(5)
    q = rng.integers(0, 16, (1, 256)).astype(np.uint8)
    sc = np.arange(1, 9, dtype=np.uint8).reshape(1, 8) * 7  # exercise the high bits (>= 16)
    mn = np.arange(8, dtype=np.uint8).reshape(1, 8) * 9
    d = np.array([np.float16(0.5).view(np.uint16)])
    dmin = np.array([np.float16(0.25).view(np.uint16)])
    blob = formats.pack_q4k(d, dmin, sc, mn, q, "ggml")
    raw = np.frombuffer(blob, np.uint8)
    assert raw[16] & 0xF == q[0, 0] and raw[16] >> 4 == q[0, 32]
    out = oracle.q4k_dequant(raw, oracle.ORC_Q4K_GGML)
    expect = (0.5 * np.repeat(sc[0], 32).astype(np.float64) * q[0]
              - 0.25 * np.repeat(mn[0], 32).astype(np.float64))
    assert np.array_equal(out, expect.astype(np.float32))
    # the interleaved packing of the same values decodes to the same numbers
    blob_i = formats.pack_q4k(d, dmin, sc, mn, q, "interleaved")
    out_i = oracle.q4k_dequant(np.frombuffer(blob_i, np.uint8), oracle.ORC_Q4K_INTERLEAVED)
    assert np.array_equal(out, out_i)


def test_q4k_linear_brute_force():
    R, Cc, M = 5, 512, 3
    w = synth.q4k_matrix(R, Cc, seed=9)
    x = np.random.default_rng(1).normal(size=(M, Cc)).astype(np.float32)
    y = oracle.q4k_linear(w, R, Cc, x)
    wd = oracle.q4k_dequant(np.frombuffer(w, np.uint8)).reshape(R, Cc).astype(np.float64)
    assert rel_l2(y, x.astype(np.float64) @ wd.T) < 1e-6


# ------------------------------------------------------------- HSDB (A0)

def test_hsdb_matmul_brute_force_and_edge():
    R, Cc, K, s, M = 37, 200, 64, 5, 3  # ragged: 3 blocks + 8-column edge strip
    stream = synth.hsdb_layer(R, Cc, K, s, seed_dict=7, seed_codes=8)
    x = synth.activations(Cc, M, seed=9)
    y = oracle.hsdb_matmul(stream, x)
    w = oracle.hsdr_decompress(stream).astype(np.float64)
    assert rel_l2(y, w @ x.astype(np.float64)) < 1e-6


def test_hsdb_dense_decode_closed_form():
    # tile (r, b) = sum_j c_j D[idx_j]; checked against numpy fp64 from the raw arrays
    R, Cc, K, s = 6, 128, 16, 4
    D = synth.dictionary(K, 64, seed=3)
    idx, coef = synth.block_codes(R, Cc, K, s, seed=4)
    stream = formats.pack_hsdb(R, Cc, D, idx, coef)
    w = oracle.hsdr_decompress(stream)
    ref = np.einsum("ts,tsb->tb", coef.astype(np.float64), D[idx.astype(np.int64)].astype(np.float64))
    assert np.abs(w.reshape(R * 2, 64) - ref).max() < 1e-6


def test_hsdb_identity_dictionary_is_a_gather():
    # D = identity rows, one slot with c = 1: W[r, b*64 + idx] = 1 -> y[r] = sum_b x[b*64+idx]
    R, Cc, K = 4, 128, 64
    D = np.eye(64, dtype=np.float32)
    idx = np.array([[3], [10], [0], [63], [5], [5], [1], [2]], np.uint16)
    coef = np.ones((8, 1), np.float16)
    stream = formats.pack_hsdb(R, Cc, D, idx, coef)
    x = np.arange(Cc, dtype=np.float32).reshape(Cc, 1)
    y = oracle.hsdb_matmul(stream, x)[:, 0]
    expect = [x[3, 0] + x[64 + 10, 0], x[0, 0] + x[64 + 63, 0], x[5, 0] + x[64 + 5, 0],
              x[1, 0] + x[64 + 2, 0]]
    assert list(y) == expect


def test_binary_hsdr_converts_losslessly(golden):
    for key in ("hsdr1d", "hsdr1de"):
        s = bytes(golden[f"{key}_stream"])
        hb = formats.hsdr_to_hsdb(s)
        assert np.array_equal(bits(oracle.hsdr_decompress(hb)), bits(golden[f"{key}_w"]))
        y = oracle.hsdb_matmul(hb, golden[f"{key}_x"])
        assert np.array_equal(bits(y), bits(golden[f"{key}_y"]))


def test_parse_rejects_like_reference(golden):
    s = bytearray(golden["hsdr1d_stream"].tobytes())
    assert oracle.hsdr_parse_status(bytes(s)) == 0
    bad = bytearray(s)
    bad[0:4] = b"XXXX"
    assert oracle.hsdr_parse_status(bytes(bad)) == -1
    bad = bytearray(s)
    bad[4] = 3
    assert oracle.hsdr_parse_status(bytes(bad)) == -2
    assert oracle.hsdr_parse_status(bytes(s[:-2])) == -3
    bad = bytearray(s)
    bad[16] += 1  # n_tiles no longer matches the shape
    assert oracle.hsdr_parse_status(bytes(bad)) == -4


# --------------------------------------------------------------- attention

def _attn_fp64(q, k, v, lens, rep, scale):
    B, Hq, d = q.shape
    out = np.zeros((B, Hq, d))
    for b in range(B):
        L = lens[b]
        for h in range(Hq):
            kk = k[b, :L, h // rep].astype(np.float64)
            vv = v[b, :L, h // rep].astype(np.float64)
            s = kk @ q[b, h].astype(np.float64) * scale
            p = np.exp(s - s.max())
            out[b, h] = (p / p.sum()) @ vv
    return out


def test_attn_decode_textbook_gqa():
    rng = np.random.default_rng(2)
    B, T, Hq, Hkv, d = 2, 37, 14, 2, 64
    q = rng.normal(size=(B, Hq, d)).astype(np.float32)
    k = rng.normal(size=(B, T, Hkv, d)).astype(np.float16)
    v = rng.normal(size=(B, T, Hkv, d)).astype(np.float16)
    lens = np.array([37, 11], np.int32)
    o = oracle.attn_decode(q, k.view(np.uint16), v.view(np.uint16), lens, Hq, Hkv, d)
    ref = _attn_fp64(q, k, v, lens, Hq // Hkv, 1 / np.sqrt(d))
    assert np.abs(o - ref).max() < 1e-5


def test_attn_decode_single_key_returns_value():
    # softmax over one position is 1: output equals that value row exactly
    rng = np.random.default_rng(3)
    q = rng.normal(size=(1, 4, 8)).astype(np.float32)
    k = rng.normal(size=(1, 1, 4, 8)).astype(np.float16)
    v = rng.normal(size=(1, 1, 4, 8)).astype(np.float16)
    o = oracle.attn_decode(q, k.view(np.uint16), v.view(np.uint16), None, 4, 4, 8)
    assert np.array_equal(o[0], v[0, 0].astype(np.float32))


# ------------------------------------------------------------ decoder ops

def test_rms_norm_closed_form():
    rng = np.random.default_rng(4)
    x = rng.normal(size=(3, 896)).astype(np.float32)
    w = rng.normal(size=896).astype(np.float32)
    y = oracle.rms_norm(x, w)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-5) * w
    assert np.abs(y - ref).max() < 1e-5


def test_silu_mul_closed_form():
    g = np.linspace(-8, 8, 101).astype(np.float32)
    u = np.linspace(1, 2, 101).astype(np.float32)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.abs(oracle.silu_mul(g, u) - ref).max() < 1e-5


def test_rope_adjacent_pairs():
    rng = np.random.default_rng(6)
    heads, hd = 3, 64
    x = rng.normal(size=(5, heads, hd)).astype(np.float32)
    y = oracle.rope(x, heads, hd, theta=1e6, pos0=7)
    # rotation keeps each (2i, 2i+1) pair's norm
    n0 = np.hypot(x[..., 0::2], x[..., 1::2])
    n1 = np.hypot(y[..., 0::2], y[..., 1::2])
    assert np.abs(n0 - n1).max() < 1e-5
    # explicit angle for token t at pos 7+t, pair i: theta^(-2i/hd) * pos
    i = np.arange(0, hd, 2)
    for t in range(5):
        ang = (7 + t) * 1e6 ** (-(i / hd))
        c, s = np.cos(ang), np.sin(ang)
        ex0 = x[t, :, 0::2] * c - x[t, :, 1::2] * s
        ex1 = x[t, :, 0::2] * s + x[t, :, 1::2] * c
        assert np.abs(y[t, :, 0::2] - ex0).max() < 2e-4
        assert np.abs(y[t, :, 1::2] - ex1).max() < 2e-4
    # position 0 is the identity
    assert np.array_equal(oracle.rope(x[:1], heads, hd, pos0=0), x[:1])


def test_select_best_rules():
    lg = np.array([1.0, 3.0, 3.0, np.nan, -np.inf, 2.0], np.float32)
    assert oracle.select_best(lg) == 1  # strict '>' keeps the first maximum
    rep = np.array([0, 1, 0, 0, 0, 0], np.uint8)
    assert oracle.select_best(lg, rep, penalty=1.5) == 2
    assert oracle.select_best(np.array([np.nan, np.inf], np.float32)) == -1
    # temperature scales before the penalty: 3/0.8 - 1.5 = 2.25 < 2/0.8 = 2.5
    assert oracle.select_best(np.array([3.0, 2.0], np.float32), np.array([1, 0], np.uint8),
                              temperature=0.8, penalty=1.5) == 1


# ---------------------------------------------------------------- fp16

def test_f16_round_trip_matches_ieee():
    rng = np.random.default_rng(7)
    vals = np.concatenate([
        rng.normal(0, 1, 5000), rng.normal(0, 1e-5, 2000), rng.normal(0, 3e4, 500),
        [0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e-8, 5.96e-8, 2.98e-8, np.inf, -np.inf],
    ]).astype(np.float32)
    h = oracle.f32_to_f16(vals)
    assert np.array_equal(h, vals.astype(np.float16).view(np.uint16))
    allh = np.arange(65536, dtype=np.uint16)
    f = oracle.f16_to_f32(allh)
    ref = allh.view(np.float16).astype(np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(f[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isnan(f[~fin]) == np.isnan(ref[~fin]))
