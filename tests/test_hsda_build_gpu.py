"""GPU parity of the shared-dictionary compressor (csdr_hsda_build: compressGroupedSegments
+ SharedDictArchive::writeToStream, HierarchicalSDRStrategy.cpp:1967-2002, 2212-2502) against
the reference's own archives for the same inputs (tests/golden/hsda_fixtures.npz and
hsda_grouped_fixtures.npz, written by the reference compiled here): a 1-row-tile group, a
capped fit pool (reservoir sampling), several tile widths (one dictionary each, in the
reference's bucket order) and 2-D tiles with a matrix that is skipped.

Bars, as for the single-matrix compress with K-SVD passes (test_hsdr_encode_gpu.py): archive
layout, dictionary configs (padding bytes aside), stage scales, segment names, dictionary
indices, sizes and types, HSDC headers and the skipped set exactly; codes equal in >= 99% of
slots; every dictionary within 1e-4 of its magnitude; each matrix's reconstruction error
within 0.1% of the reference archive's.
"""
import os

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _recon(dicts, seg, shape):
    d = dicts[seg[1]]
    return oracle.hsdr_decompress(oracle.hsdc_to_hsdr(seg[4], d)).reshape(shape)


def _compare(ours, ref, mats, skipped_ours, skipped_ref):
    assert ours[:16] == ref[:16]   # magic, version, dictionary and segment counts
    assert skipped_ours == skipped_ref
    od, osg = oracle.hsda_parse(ours)
    rd, rsg = oracle.hsda_parse(ref)
    for a, b in zip(od, rd):
        for key in ("tile_rows", "tile_cols", "n_atoms", "n_stages", "k", "stage_decay"):
            assert a[key] == b[key], key
        assert np.array_equal(a["stage_scales"], b["stage_scales"])
        assert np.abs(a["atoms"] - b["atoms"]).max() <= 1e-4 * np.abs(b["atoms"]).max()
    for a, b in zip(osg, rsg):
        assert a[:4] == b[:4]              # name, dictionary index, original size, type
        assert a[4][:32] == b[4][:32]      # HSDC header
        ca = np.frombuffer(a[4][32:], "<u2")
        cb = np.frombuffer(b[4][32:], "<u2")
        assert (ca == cb).mean() >= 0.99, a[0]
        w = mats[a[0]]
        em = np.linalg.norm(_recon(od, a, w.shape) - w)
        er = np.linalg.norm(_recon(rd, b, w.shape) - w)
        assert abs(em - er) <= 1e-3 * er, a[0]


def test_group_matches_reference_archive(gpu):
    from cortexsdr_amd.encode import hsda_build

    fx = np.load(os.path.join(GOLDEN, "hsda_fixtures.npz"))
    # the inputs make_fixtures.py's hsda_main drew
    rng = np.random.default_rng(20261202)
    names = ["blk.0.attn_q.weight", "blk.0.attn_k.weight", "blk.1.ffn_up.weight"]
    mats = {n: rng.normal(0, 0.05, (R, 64)).astype(np.float32) for n, R in zip(names, (32, 20, 45))}
    ours, skipped = hsda_build(mats, 1, 64, 16, 2, 2, ksvd_iters=3)
    _compare(ours, fx["hsda_bytes"].tobytes(), mats, skipped, [])


@pytest.mark.parametrize("case", [0, 1, 2])
def test_grouped_cases_match_reference(gpu, case):
    from cortexsdr_amd.encode import hsda_build

    fx = np.load(os.path.join(GOLDEN, "hsda_grouped_fixtures.npz"))
    tr, tc, K, S, k, it, cap = (int(v) for v in fx[f"g{case}_cfg"])
    mats = {}
    j = 0
    while f"g{case}_name_{j}" in fx.files:
        mats[fx[f"g{case}_name_{j}"].tobytes().decode()] = fx[f"g{case}_w_{j}"]
        j += 1
    ours, skipped = hsda_build(mats, tr, tc, K, S, k, ksvd_iters=it, max_tiles_for_fit=cap)
    ref_skipped = [n for n, s in zip(mats, fx[f"g{case}_skipped"]) if s]
    _compare(ours, fx[f"g{case}_bytes"].tobytes(), mats, skipped, ref_skipped)


def test_archive_loads_and_multiplies(gpu):
    """The built archive through the device reader (csdr_hsda_load): each segment's product
    against the oracle's product of the archive's own reconstruction."""
    from cortexsdr_amd.archive import HsdaArchive
    from cortexsdr_amd.encode import hsda_build

    rng = np.random.default_rng(8)
    mats = {"x.weight": rng.normal(0, 0.05, (48, 64)).astype(np.float32),
            "y.weight": rng.normal(0, 0.05, (40, 64)).astype(np.float32)}
    data, skipped = hsda_build(mats, 1, 64, 16, 2, 2, ksvd_iters=1)
    assert skipped == []
    dicts, segs = oracle.hsda_parse(data)
    x = rng.normal(0, 1, (64, 3)).astype(np.float32)
    arc = HsdaArchive(data=data)
    try:
        assert len(arc) == 2 and arc.num_dictionaries() == 1
        for seg in segs:
            w = _recon(dicts, seg, mats[seg[0]].shape)
            dev = arc.load(seg[0])
            y = dev.matmul(gpu.from_numpy(x).cuda()).cpu().numpy()
            dev.free()
            assert np.abs(y - w @ x).max() <= 1e-4 * np.abs(w @ x).max()
    finally:
        arc.close()
