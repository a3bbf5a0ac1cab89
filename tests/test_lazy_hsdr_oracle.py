"""Pins of the oracle's restatement of the text CLI's lazy HSDR embedding
(cortexsdr_cli.cpp:488-554 parse and row decode, :687-732 vocabulary scoring).

* Row decode with the packIndexSign reading equals the reference's own decompressed matrix
  (tests/golden/ref_fixtures.npz hsdr1d_w, HierarchicalSDRStrategy::decompress of the same
  stream) bit for bit: the same (gamma * sign) * atom accumulation, stage-major.
* The CLI's code reading (index = v >> 1, sign = v & 1) on a stream re-packed that way decodes
  to the same rows.
* Scores against a float64 brute force (each token's dense row times the hidden state):
  within 1e-5 relative; the chosen token is the brute force's penalised argmax unless its top
  two are within 1e-5.
"""
import numpy as np

import oracle


def _repack_cli(stream):
    """The same stream with every code word rewritten as (index << 1) | sign."""
    b = np.frombuffer(bytes(stream), np.uint8).copy()
    v = oracle.hsdr_parse(b)
    codes = b[v.off_packed:v.off_packed + 2 * v.n_codes].view("<u2")
    idx, sign = codes & 0x7FFF, codes >> 15
    b[v.off_packed:v.off_packed + 2 * v.n_codes] = ((idx << 1) | sign).astype("<u2").view(np.uint8)
    return b


def test_row_decode_matches_reference_decompress(golden):
    s, w = golden["hsdr1d_stream"], golden["hsdr1d_w"]
    rows, cols = oracle.lazy_hsdr_info(s)
    assert (rows, cols) == w.shape
    for r in range(rows):
        got = oracle.lazy_hsdr_decode_row(s, r)
        assert np.array_equal(got.view(np.uint32), w[r].view(np.uint32)), r


def test_cli_code_reading(golden):
    s = golden["hsdr1d_stream"]
    cli = _repack_cli(s)
    for r in (0, 17, 63):
        assert np.array_equal(oracle.lazy_hsdr_decode_row(cli, r, oracle.ORC_LAZY_CLI),
                              oracle.lazy_hsdr_decode_row(s, r, oracle.ORC_LAZY_PACKED))


def test_scores_against_brute_force(golden):
    s, w = golden["hsdr1d_stream"], golden["hsdr1d_w"].astype(np.float64)
    rng = np.random.default_rng(4)
    for trial in range(5):
        h = rng.standard_normal(w.shape[1]).astype(np.float32)
        rep = (rng.random(w.shape[0]) < 0.2).astype(np.uint8)
        tok, scores = oracle.lazy_hsdr_select(s, h, rep, 0.8, 1.0)
        ref = w @ h.astype(np.float64)
        assert np.abs(scores - ref).max() <= 1e-5 * np.abs(ref).max()
        pen = ref / 0.8 - 1.0 * rep
        top = np.sort(pen)[-2:]
        if top[1] - top[0] > 1e-5 * max(1.0, abs(top[1])):
            assert tok == int(np.argmax(pen)), trial
    # temperature <= 0 leaves the scores unscaled; no repeated set
    h = rng.standard_normal(w.shape[1]).astype(np.float32)
    tok, scores = oracle.lazy_hsdr_select(s, h, None, 0.0, 1.0)
    assert tok == int(np.argmax(scores))
