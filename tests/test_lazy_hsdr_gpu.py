"""GPU parity of the text CLI's lazy HSDR embedding (csdr_lazy_hsdr_*; cortexsdr_cli.cpp:
488-554, 687-732) and of the decoder's token choice by it, through the C-ABI, against the
oracle's restatement (pinned in test_lazy_hsdr_oracle.py).

Bars: decoded rows bit-exact (the reference's own decompressed matrix for the packed reading;
the CLI reading of a re-packed stream gives the same rows); scores within 1e-6 relative L2 of
the oracle's (the fp64 atom . hidden sums are rounded to float in either order) and the chosen
token the oracle's unless its top two penalised scores are within 1e-5; in the decoder, every
step's token against the oracle's scoring of the oracle decoder's hidden state (scores within
1e-3, the decoder's bar), near-ties aside.
"""
import numpy as np
import pytest

import oracle
from conftest import rel_l2

pytestmark = pytest.mark.gpu


def _repack_cli(stream):
    b = np.frombuffer(bytes(stream), np.uint8).copy()
    v = oracle.hsdr_parse(b)
    codes = b[v.off_packed:v.off_packed + 2 * v.n_codes].view("<u2")
    idx, sign = codes & 0x7FFF, codes >> 15
    b[v.off_packed:v.off_packed + 2 * v.n_codes] = ((idx << 1) | sign).astype("<u2").view(np.uint8)
    return b.tobytes()


def _near_tie(pen, tol=1e-5):
    top = np.sort(pen)[-2:]
    return top[1] - top[0] <= tol * max(1.0, abs(float(top[1])))


def test_decode_rows_bitexact(gpu, golden):
    from cortexsdr_amd.hsdr import LazyHsdrEmbedding

    s, w = golden["hsdr1d_stream"], golden["hsdr1d_w"]
    emb = LazyHsdrEmbedding(s)
    assert (emb.rows, emb.cols) == w.shape
    ids = [0, 5, 63, 17, 5]
    got = emb.decode_rows(ids).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), w[ids].view(np.uint32))
    cli = LazyHsdrEmbedding(_repack_cli(s), unpack="cli")
    assert np.array_equal(cli.decode_rows(ids).cpu().numpy().view(np.uint32),
                          w[ids].view(np.uint32))
    # ids outside the vocabulary decode to zero rows
    assert not emb.decode_rows([64, -1]).cpu().numpy().any()


@pytest.mark.parametrize("unpack", ["packed", "cli"])
@pytest.mark.parametrize("temperature", [0.8, 0.0])
def test_select_matches_oracle(gpu, golden, unpack, temperature):
    from cortexsdr_amd.hsdr import LazyHsdrEmbedding

    s = golden["hsdr1d_stream"]
    if unpack == "cli":   # the CLI's reading of the stream as written (indices past K skipped)
        stream, mode = bytes(s), oracle.ORC_LAZY_CLI
    else:
        stream, mode = bytes(s), oracle.ORC_LAZY_PACKED
    emb = LazyHsdrEmbedding(stream, unpack=unpack)
    rng = np.random.default_rng(7)
    rows = 4
    h = rng.standard_normal((rows, emb.cols)).astype(np.float32)
    rep = (rng.random((rows, emb.rows)) < 0.25).astype(np.uint8)
    tok, sc = emb.select(gpu.from_numpy(h).cuda(), gpu.from_numpy(rep).cuda(), temperature, 1.0)
    tok, sc = tok.cpu().numpy(), sc.cpu().numpy()
    for r in range(rows):
        want_tok, want = oracle.lazy_hsdr_select(stream, h[r], rep[r], temperature, 1.0, mode)
        # atom . hidden as the CLI sums it (fp64, feature order) and the slot sums in stream
        # order: the scores are the oracle's bit for bit, so is the choice, near-ties included
        assert np.array_equal(sc[r].view(np.uint32), want.view(np.uint32)), r
        assert tok[r] == want_tok, r
        ts = 1.0 / temperature if temperature > 0 else 1.0
        pen = want * np.float32(ts) - rep[r]
        if not _near_tie(pen):
            assert tok[r] == want_tok, r


def test_select_updates_position_and_generated_set(gpu, golden):
    import ctypes as C

    from cortexsdr_amd import _lib
    from cortexsdr_amd.hsdr import LazyHsdrEmbedding

    emb = LazyHsdrEmbedding(golden["hsdr1d_stream"])
    lib = _lib.load()
    rows = 2
    h = gpu.from_numpy(np.random.default_rng(3).standard_normal((rows, emb.cols))
                       .astype(np.float32)).cuda()
    rep = gpu.zeros((rows, emb.rows), dtype=gpu.uint8, device="cuda")
    pos = gpu.tensor([5], dtype=gpu.int32, device="cuda")
    tok = gpu.empty(rows, dtype=gpu.int32, device="cuda")
    ws = gpu.zeros(int(lib.csdr_lazy_hsdr_workspace_bytes(emb._h, rows)), dtype=gpu.uint8,
                   device="cuda")
    st = gpu.cuda.current_stream().cuda_stream
    _lib.check(lib.csdr_lazy_hsdr_select(emb._h, h.data_ptr(), rows, rep.data_ptr(),
                                         C.c_float(0.8), C.c_float(1.0), tok.data_ptr(),
                                         pos.data_ptr(), rep.data_ptr(), None, ws.data_ptr(),
                                         ws.numel(), st))
    t = tok.cpu().numpy()
    assert int(pos.cpu()[0]) == 6
    r = rep.cpu().numpy()
    for i in range(rows):
        assert r[i].sum() == 1 and r[i, t[i]] == 1
    with pytest.raises(_lib.CsdrError):   # workspace too small
        _lib.check(lib.csdr_lazy_hsdr_select(emb._h, h.data_ptr(), rows, None, C.c_float(0.8),
                                             C.c_float(1.0), tok.data_ptr(), None, None, None,
                                             ws.data_ptr(), 16, st))


def test_decoder_lazy_selection_matches_oracle(gpu):
    from cortexsdr_amd.decoder import Decoder, DecoderSpec, synthetic_weights
    from cortexsdr_amd.encode import compress
    from cortexsdr_amd.hsdr import LazyHsdrEmbedding
    from oracle import decoder as odec

    spec = DecoderSpec(2, 128, 2, 1, 64, 200, 160, 40)
    w = synthetic_weights(spec, n_atoms=128, nnz=8, seed=31, sigma=0.1, norm_jitter=0.1)
    table = np.random.default_rng(9).standard_normal((spec.vocab, spec.hidden)).astype(np.float32)
    stream = compress(table, 1, spec.hidden, 32, 2, 4)   # vocab x hidden, 1-row tiles
    emb = LazyHsdrEmbedding(stream)
    prompt = ((np.arange(9) * 7919 + 5) % spec.vocab).astype(np.int32)
    n_new = 6
    dec = Decoder(w)
    try:
        dec.set_lazy_selection(emb, 1.0)
        dec.prefill(prompt, 0.8, 0.0)
        scores = [dec.logits()]
        for _ in range(n_new - 1):
            dec.decode(1, 0.8, 0.0)
            scores.append(dec.logits())
        toks = dec.tokens(len(prompt), n_new)
        seq = list(prompt)
        rep = np.zeros(spec.vocab, np.uint8)
        for i in range(n_new):
            hid = odec.hidden_last(w, np.array(seq, np.int32))
            want_tok, want = oracle.lazy_hsdr_select(stream, hid, rep, 0.8, 1.0)
            assert rel_l2(scores[i], want) < 1e-3, i
            pen = want * np.float32(1 / 0.8) - rep
            if not _near_tie(pen, 2e-3):
                assert toks[i] == want_tok, i
            seq.append(int(toks[i]))   # continue along the device's choice
            rep[toks[i]] = 1
        # the lm_head choice again
        dec.set_lazy_selection(None)
        dec.prefill(prompt, 0.8, 1.5)
        _, ref = odec.generate(w, prompt, 1, 0.8, 1.5)
        assert rel_l2(dec.logits(), ref[0]) < 1e-3
    finally:
        dec.close()
        emb.free()


def test_decoder_rejects_mismatched_embedding(gpu, golden):
    from cortexsdr_amd._lib import CsdrError
    from cortexsdr_amd.decoder import Decoder, DecoderSpec, synthetic_weights
    from cortexsdr_amd.hsdr import LazyHsdrEmbedding

    spec = DecoderSpec(1, 128, 2, 1, 64, 128, 100, 16)
    w = synthetic_weights(spec, n_atoms=64, nnz=4, seed=2, sigma=0.1)
    emb = LazyHsdrEmbedding(golden["hsdr1d_stream"])   # 64 x 256
    dec = Decoder(w)
    try:
        with pytest.raises(CsdrError):
            dec.set_lazy_selection(emb, 1.0)
    finally:
        dec.close()
