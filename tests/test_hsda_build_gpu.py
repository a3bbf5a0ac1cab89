"""GPU parity of the shared-dictionary compressor (csdr_hsda_build: compressGroupedSegments
+ SharedDictArchive::writeToStream, HierarchicalSDRStrategy.cpp:1967-2002, 2212-2502) against
the reference's own archives for the same inputs (tests/golden/hsda_fixtures.npz and
hsda_grouped_fixtures.npz, written by the reference compiled here): a 1-row-tile group, a
capped fit pool (reservoir sampling), several tile widths (one dictionary each, in the
reference's bucket order) and 2-D tiles with a matrix that is skipped.

Bar, as for the single-matrix compress (test_hsdr_encode_gpu.py): the reference's archive
byte for byte on any host CPU, except the two padding bytes of each dictionary's
HierarchicalSDRConfig record, which the reference writes uninitialised; and the skipped set.
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


def _config_padding(b):
    """Offsets of the two compiler padding bytes of every dictionary's 20-byte config record
    (after u16 x 3 and u8 x 4; the layout oracle.hsda_parse reads)."""
    import struct

    (nd,) = struct.unpack_from("<I", b, 8)
    off, pad = 16, set()
    for _ in range(nd):
        pad |= {off + 10, off + 11}
        off += 20
        (nsc,) = struct.unpack_from("<I", b, off)
        off += 4 + 4 * nsc
        (na,) = struct.unpack_from("<I", b, off)
        off += 4 + 4 * na
    return pad


def _compare(ours, ref, mats, skipped_ours, skipped_ref):
    assert skipped_ours == skipped_ref
    assert len(ours) == len(ref)
    a = np.frombuffer(ours, np.uint8)
    b = np.frombuffer(ref, np.uint8)
    differ = set(np.nonzero(a != b)[0].tolist())
    assert differ <= _config_padding(ref), sorted(differ)[:8]
    # and each matrix reconstructs from our archive as from the reference's
    od, osg = oracle.hsda_parse(ours)
    rd, rsg = oracle.hsda_parse(ref)
    for sa, sb in zip(osg, rsg):
        w = mats[sa[0]]
        assert np.array_equal(_recon(od, sa, w.shape), _recon(rd, sb, w.shape)), sa[0]


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
