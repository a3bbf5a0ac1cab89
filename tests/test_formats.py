"""Stream writers and the seeded generator (host side), checked with the oracle parser."""
import numpy as np

import oracle
from cortexsdr_amd import formats, synth


def test_pack_hsdb_round_trip():
    R, Cc, K, s = 9, 150, 40, 6
    D = synth.dictionary(K, 64, seed=1)
    idx, coef = synth.block_codes(R, Cc, K, s, seed=2)
    edge = np.arange(R * 22, dtype=np.float32).reshape(R, 22)
    st = formats.pack_hsdb(R, Cc, D, idx, coef, edge=edge)
    v = oracle.hsdr_parse(st)
    assert (v.is_hsdb, v.rows, v.cols, v.tile_rows, v.tile_cols) == (1, R, Cc, 1, 64)
    assert (v.n_atoms, v.n_stages * v.k_per_stage, v.edge_bytes, v.end) == (K, s, edge.nbytes,
                                                                           len(st))
    oi, osg, oc = oracle.hsdr_unpack(st)
    assert np.array_equal(oi, idx.ravel())
    assert np.array_equal(oc, coef.astype(np.float32).ravel())
    pi, ps, mag, gamma = formats.hsdb_unpack(st)
    assert np.array_equal(pi, idx.ravel()) and gamma[0] == 1.0
    assert np.array_equal(ps, np.signbit(coef).astype(np.uint16).ravel())
    w = oracle.hsdr_decompress(st)
    assert np.array_equal(w[:, 128:], edge)


def test_generator_is_seeded_and_distinct():
    a = synth.normal(5, 1000)
    assert np.array_equal(a, synth.normal(5, 1000))
    assert not np.array_equal(a, synth.normal(6, 1000))
    assert abs(a.mean()) < 0.15 and abs(a.std() - 1) < 0.1
    sel = synth.distinct_indices(3, 5000, 8, 1024)
    assert sel.min() >= 0 and sel.max() < 1024
    assert all(len(set(r)) == 8 for r in sel[:2000])
    # roughly uniform marginal
    h = np.bincount(sel.ravel(), minlength=1024)
    assert h.min() > 10 and h.max() < 80
    D = synth.dictionary(64, 64, seed=1)
    assert np.allclose(np.linalg.norm(D, axis=1), 1.0, atol=1e-6)


def test_q4k_matrix_decodes_in_range():
    w = synth.q4k_matrix(4, 512, seed=3)
    assert len(w) == 4 * 2 * 144
    v = oracle.q4k_dequant(np.frombuffer(w, np.uint8))
    # |value| <= d*63*15 + dmin*63 with d, dmin <= 0.05
    assert np.abs(v).max() <= 0.05 * 63 * 16
