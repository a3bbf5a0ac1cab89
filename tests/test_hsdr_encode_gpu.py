"""GPU parity of the HSDR encoder (csdr_hsdr_encode, csdr_hsdr_compress) through the C-ABI.

Bars:
  * matching pursuit: codes bit-exact against the reference's compress fixtures (given the
    stream's dictionary) and against the oracle (pinned in test_hsdr_encode_oracle.py) on
    larger random cases; K, tile sizes with and without an 8-element chunk, many tiles per
    workgroup and one;
  * compress, with and without K-SVD passes: the reference's stream byte for byte, on any
    host CPU (the initialisation takes the approximate reciprocal square root of the CPU the
    fixtures were written on from a table, and sums the tile norms in the reference build's
    order; the fixtures were written with one OpenMP thread).
"""
import os

import numpy as np
import pytest

import oracle
from test_hsdr_encode_oracle import stream_parts, tiles_of

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def enc():
    return np.load(os.path.join(GOLDEN, "hsdr_encode_fixtures.npz"), allow_pickle=False)


def n_cases(enc):
    return len([k for k in enc.files if k.startswith("enc_") and k.endswith("_stream")])


def gpu_codes(gpu, tiles, D, g, S, k):
    from cortexsdr_amd import encode

    t = gpu.from_numpy(np.array(tiles, np.float32)).cuda()
    d = gpu.from_numpy(np.array(D, np.float32)).cuda()
    return encode.encode(t, d, g, S, k).cpu().numpy().view(np.uint16)


def test_encode_matches_reference_fixtures(gpu, enc):
    for i in range(n_cases(enc)):
        v, D, g, codes = stream_parts(enc[f"enc_{i}_stream"].tobytes())
        t = tiles_of(enc[f"enc_{i}_w"], v.tile_rows, v.tile_cols)
        got = gpu_codes(gpu, t, D, g, v.n_stages, v.k_per_stage)
        assert np.array_equal(got, codes), f"case {i}"


@pytest.mark.parametrize("n,C,K,S,k", [(1000, 64, 256, 3, 5), (333, 200, 100, 2, 8),
                                       (40, 1024, 512, 3, 4), (7, 4096, 64, 2, 3),
                                       (1, 8, 8, 2, 4), (500, 60, 64, 2, 3), (300, 39, 48, 3, 2),
                                       (64, 5, 8, 2, 2), (2000, 100, 128, 2, 4)])
def test_encode_matches_oracle(gpu, n, C, K, S, k):
    rng = np.random.default_rng(n + C + K)
    t = (rng.standard_normal((n, C)) * 0.02).astype(np.float32)
    D = rng.standard_normal((K, C)).astype(np.float32)
    D /= np.linalg.norm(D, axis=1, keepdims=True)
    D *= 0.02 * np.sqrt(C / (S * k))
    g = (0.5 ** np.arange(S)).astype(np.float32)
    want = oracle.hsdr_mp(t, D, g, S, k)
    got = gpu_codes(gpu, t, D, g, S, k)
    assert np.array_equal(got, want)


# Each tiles-per-workgroup instantiation of the matching-pursuit kernel (1: the large-tile LDS
# fallback; 4 and 8: what matrices of >= 4096 tiles take, with 2 atoms per lane group and
# float4 tile loads), forced through the kernel's selection override, bit-exact against the
# oracle; ragged last workgroups (n not a multiple of TT), tiles with an 8-element chunk
# (C % 16 == 8) and without, and a case whose natural selection is TT = 1 (C x K too large
# for two tiles under the soft LDS size).
@pytest.mark.parametrize("tt", [1, 4, 8])
@pytest.mark.parametrize("n,C,K,S,k", [(203, 72, 128, 3, 4), (1031, 64, 256, 3, 5),
                                       (37, 200, 64, 2, 8), (45, 896, 160, 3, 3)])
def test_encode_tiles_per_workgroup_match_oracle(gpu, monkeypatch, tt, n, C, K, S, k):
    monkeypatch.setenv("CSDR_HSDR_TILES_PER_WG", str(tt))
    rng = np.random.default_rng(7 * n + C + K + tt)
    t = (rng.standard_normal((n, C)) * 0.02).astype(np.float32)
    D = rng.standard_normal((K, C)).astype(np.float32)
    D /= np.linalg.norm(D, axis=1, keepdims=True)
    D *= 0.02 * np.sqrt(C / (S * k))
    g = (0.5 ** np.arange(S)).astype(np.float32)
    want = oracle.hsdr_mp(t, D, g, S, k)
    got = gpu_codes(gpu, t, D, g, S, k)
    assert np.array_equal(got, want), f"TT={tt}"


def test_encode_large_tile_falls_back_to_one_per_workgroup(gpu, monkeypatch):
    # 2 x (C + K) x 4 bytes > 64 KiB: the natural choice is one tile per workgroup
    monkeypatch.delenv("CSDR_HSDR_TILES_PER_WG", raising=False)
    n, C, K, S, k = 9, 4096, 4096, 2, 3
    rng = np.random.default_rng(11)
    t = (rng.standard_normal((n, C)) * 0.02).astype(np.float32)
    D = rng.standard_normal((K, C)).astype(np.float32)
    D /= np.linalg.norm(D, axis=1, keepdims=True)
    D *= 0.02 * np.sqrt(C / (S * k))
    g = (0.5 ** np.arange(S)).astype(np.float32)
    assert np.array_equal(gpu_codes(gpu, t, D, g, S, k), oracle.hsdr_mp(t, D, g, S, k))


def test_compress_matches_reference(gpu, enc):
    """The whole stream (header, dictionary, stage scales, codes, edge strips) is the
    reference's byte for byte, whatever CPU this host has."""
    from cortexsdr_amd import encode

    for i in range(n_cases(enc)):
        w, ref = enc[f"enc_{i}_w"], enc[f"enc_{i}_stream"].tobytes()
        tr, tc, K, S, k = (int(x) for x in enc[f"enc_{i}_cfg"])
        s = encode.compress(w, tr, tc, K, S, k, ksvd_iters=0, stage_decay=0.5)
        assert len(s) == len(ref)
        v, D, g, codes = stream_parts(s)
        rv, rD, rg, rcodes = stream_parts(ref)
        ulp = np.abs(D.view(np.int32).astype(np.int64) - rD.view(np.int32).astype(np.int64))
        assert ulp.max() == 0, f"case {i}: dictionary differs by {ulp.max()} ulp"
        assert np.array_equal(codes, rcodes), f"case {i}"
        assert s == ref, f"case {i}"
        assert oracle.hsdr_decompress(s).shape == w.shape


def test_compress_refined_matches_reference(gpu, enc):
    """ksvd_iters > 0 (atomUpdateStep then matching pursuit again, per pass): the reference's
    stream byte for byte on any host CPU. Its per-atom corrections are double sums in its user
    order; its tile-norm mean and re-seed norms are sums in the order its -O3 -ffast-math
    AVX2 build executes (the mean with one OpenMP thread, as the fixtures were written); the
    initial dictionary takes the fixtures' CPU's reciprocal square root. Also: the GPU's
    matching pursuit over the reference's own refined dictionary gives its codes."""
    from cortexsdr_amd import encode

    n = len([k for k in enc.files if k.startswith("fit_") and k.endswith("_stream")])
    assert n >= 4
    for i in range(n):
        w, ref = enc[f"fit_{i}_w"], enc[f"fit_{i}_stream"].tobytes()
        tr, tc, K, S, k, it = (int(x) for x in enc[f"fit_{i}_cfg"])
        s = encode.compress(w, tr, tc, K, S, k, ksvd_iters=it, stage_decay=0.5)
        v, D, g, codes = stream_parts(s)
        rv, rD, rg, rcodes = stream_parts(ref)
        ulp = np.abs(D.view(np.int32).astype(np.int64) - rD.view(np.int32).astype(np.int64))
        print(f"fit {i}: dictionary {ulp.max()} ulp, codes {np.mean(codes == rcodes):.5f}")
        assert ulp.max() == 0, f"case {i}"
        assert np.array_equal(codes, rcodes), f"case {i}"
        assert s == ref, f"case {i}"
        t = tiles_of(w, rv.tile_rows, rv.tile_cols)
        assert np.array_equal(gpu_codes(gpu, t, rD, rg, S, k), rcodes), f"case {i}"


def test_compress_rejects(gpu):
    from cortexsdr_amd import _lib, encode

    w = np.zeros((10, 64), np.float32)
    with pytest.raises(ValueError):   # fewer tiles than atoms
        encode.compress(w, 1, 64, 16, 2, 2)
    with pytest.raises(_lib.CsdrError):   # K-SVD passes over tiles of more than 32768 values
        encode.compress(np.ones((2, 40000), np.float32), 1, 40000, 1, 1, 1, ksvd_iters=1)
