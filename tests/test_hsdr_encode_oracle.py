"""Pins the oracle's restatement of the HSDR encoder's matching pursuit (oracle.hsdr_mp,
hierarchicalBinaryCode, HierarchicalSDRStrategy.cpp:219-262, with dot_product_simd's AVX2
summation order :157-190) against the reference's own compress (tests/golden/
hsdr_encode_fixtures.npz: HierarchicalSDRStrategy::compress with ksvd_iters = 0, i.e. the
dictionary initialised from random tiles and one encode pass; the codes in the stream are the
reference's matching pursuit over the stream's dictionary).

Bars: codes bit-exact. The symmetric-pair fixtures make projections tie in exact arithmetic,
so the float summation order decides picks: a plain sequential-order restatement (planted
here, on the CPU) disagrees with the reference on them, the oracle does not.
"""
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def enc():
    return np.load(os.path.join(GOLDEN, "hsdr_encode_fixtures.npz"), allow_pickle=False)


def cases(enc):
    n = len([k for k in enc.files if k.startswith("enc_") and k.endswith("_stream")])
    return [(enc[f"enc_{i}_w"], enc[f"enc_{i}_stream"].tobytes(), enc[f"enc_{i}_cfg"])
            for i in range(n)]


def tiles_of(w, tr, tc):
    """extractTiles (HierarchicalSDRStrategy.cpp:94-116) of the aligned top-left block."""
    R, Cc = w.shape
    Rf, Cf = (R // tr) * tr, (Cc // tc) * tc
    t = w[:Rf, :Cf].reshape(Rf // tr, tr, Cf // tc, tc).transpose(0, 2, 1, 3)
    return np.ascontiguousarray(t.reshape(-1, tr * tc))


def stream_parts(stream):
    v = oracle.hsdr_parse(stream)
    C = v.tile_rows * v.tile_cols
    D = np.frombuffer(stream, np.float32, v.n_atoms * C, v.off_dict).reshape(v.n_atoms, C)
    g = np.frombuffer(stream, np.float32, v.n_stages, v.off_gamma)
    codes = np.frombuffer(stream, np.uint16, v.n_codes, v.off_packed).reshape(v.n_tiles, -1)
    return v, D, g, codes


def test_mp_matches_reference_codes(enc):
    for i, (w, stream, cfg) in enumerate(cases(enc)):
        v, D, g, codes = stream_parts(stream)
        t = tiles_of(w, v.tile_rows, v.tile_cols)   # 1-row tiles span the whole row
        assert t.shape[0] == v.n_tiles
        got = oracle.hsdr_mp(t, D, g, v.n_stages, v.k_per_stage)
        assert np.array_equal(got, codes), f"case {i} cfg {cfg.tolist()}"


def sequential_mp(t, D, g, S, k):
    """The planted mistake: projections summed in plain element order (fp32 FMA chain)."""
    n, C = t.shape
    r = t.astype(np.float32).copy()
    out = np.zeros((n, S * k), np.uint16)
    D64 = D.astype(np.float64)
    for l in range(S):
        used = np.zeros((n, D.shape[0]), bool)
        for st in range(k):
            acc = np.zeros((n, D.shape[0]), np.float32)
            for c in range(C):   # fma(a, b, acc): the product is exact in fp64
                acc = (np.outer(r[:, c].astype(np.float64), D64[:, c]) + acc).astype(np.float32)
            acc[used] = 0.0
            a = np.abs(acc)
            best = np.argmax(a, axis=1)   # first maximum, as the strict '>' scan
            best[a.max(axis=1) <= 0] = 0
            pb = acc[np.arange(n), best]
            neg = pb < 0
            out[:, l * k + st] = best | np.where(neg, 0x8000, 0)
            used[np.arange(n), best] = True
            sc = (g[l] * np.where(neg, -1.0, 1.0)).astype(np.float32)
            r = (r.astype(np.float64) - D64[best] * sc[:, None]).astype(np.float32)
    return out


def test_fixtures_distinguish_summation_order(enc):
    wrong = 0
    for w, stream, cfg in cases(enc):
        if int(cfg[0]) != 1 or int(cfg[2]) != 48:   # the symmetric-pair fixtures
            continue
        v, D, g, codes = stream_parts(stream)
        wrong += int((sequential_mp(w, D, g, v.n_stages, v.k_per_stage) != codes).any(1).sum())
    assert wrong > 0


def test_init_dictionary_matches_reference(enc):
    """The library's host-side initialisation (csdr_hsdr_init_dictionary, host code: no GPU)
    against the dictionaries the reference's compress wrote for the same tiles: bit for bit on
    any host CPU. The reference's 1/sqrt is the approximate reciprocal square root of the CPU
    the fixtures were written on (recorded in them) plus a Newton step; the library takes that
    CPU's value from a table (csrc/hsdr_rsqrt_table.inc) rather than from the host's own
    instruction, whose result differs between CPU models."""
    from cortexsdr_amd import encode

    for i, (w, stream, cfg) in enumerate(cases(enc)):
        v, D, g, codes = stream_parts(stream)
        t = tiles_of(w, v.tile_rows, v.tile_cols)
        got = encode.init_dictionary(t, v.n_atoms, v.n_stages, v.k_per_stage)
        assert np.array_equal(got.view(np.uint32), D.view(np.uint32)), f"case {i}"



def test_rsqrt_table_within_the_instruction_bound():
    """csrc/hsdr_rsqrt_table.inc (the fixtures' CPU's rsqrtss of s = 2^p (1 + m / 1024)) against
    the mathematics: every entry within rsqrtss's documented relative error, 1.5 x 2^-12, of
    1 / sqrt(s), the entries decreasing in s, and p = 1 the p = 0 curve continued (the table
    reaches from 1 to 4)."""
    import re

    path = os.path.join(os.path.dirname(__file__), "..", "cortexsdr_amd", "csrc",
                        "hsdr_rsqrt_table.inc")
    words = [int(w, 16) for w in re.findall(r"0x([0-9a-f]{8})u", open(path).read())]
    assert len(words) == 2048
    y = np.array(words, np.uint32).view(np.float32).astype(np.float64)
    p = np.repeat([0, 1], 1024)
    m = np.tile(np.arange(1024), 2)
    s = 2.0 ** p * (1.0 + m / 1024.0)
    rel = np.abs(y * np.sqrt(s) - 1.0)
    assert rel.max() <= 1.5 * 2.0 ** -12, rel.max()
    assert np.all(np.diff(y) <= 0)
