"""Pins the oracle decoder (oracle/decoder.py) on tiny models against an independent float64
dense restatement of the reference's block (api/cortex_sdk.cpp:1543-1696): dense W from the
(reference-pinned) decompress, float64 RMSNorm, RoPE angles, grouped attention, SwiGLU and
residuals written from the textbook definitions. A wrong residual, GQA mapping, RoPE pairing
or norm placement in the oracle fails these."""
import numpy as np
import pytest

import oracle
from oracle import decoder as odec
from cortexsdr_amd.decoder import DecoderSpec, synthetic_weights
from conftest import rel_l2


def dense_forward(w, tokens):
    s = w.spec
    T, hd, Hq, Hkv = len(tokens), s.head_dim, s.n_heads, s.n_kv_heads
    dense = {}

    def W(stream):
        key = id(stream)
        if key not in dense:
            dense[key] = oracle.hsdr_decompress(stream).astype(np.float64)
        return dense[key]

    def norm(x, g):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + s.rms_eps) * g

    def rot(x, heads):
        x = x.reshape(T, heads, hd).copy()
        i = np.arange(0, hd, 2)
        ang = np.arange(T)[:, None] * (float(s.rope_theta) ** (-i / hd))[None, :]
        c, sn = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        a, b = x[..., 0::2].copy(), x[..., 1::2].copy()
        x[..., 0::2] = a * c - b * sn
        x[..., 1::2] = a * sn + b * c
        return x

    x = W(w.lm_head)[np.asarray(tokens)]
    for L in w.layers:
        h = norm(x, L["attn_norm"])
        q = h @ W(L["q"]).T + L.get("bq", 0.0)
        k = h @ W(L["k"]).T + L.get("bk", 0.0)
        v = h @ W(L["v"]).T + L.get("bv", 0.0)
        q, k = rot(q, Hq), rot(k, Hkv)
        v = v.reshape(T, Hkv, hd)
        a = np.zeros((T, Hq, hd))
        for hh in range(Hq):
            g = hh // (Hq // Hkv)
            sc = q[:, hh] @ k[:, g].T / np.sqrt(hd)
            sc[np.triu_indices(T, 1)] = -np.inf
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            a[:, hh] = p @ v[:, g]
        x = x + a.reshape(T, -1) @ W(L["o"]).T
        h = norm(x, L["ffn_norm"])
        gt, up = h @ W(L["gate"]).T, h @ W(L["up"]).T
        x = x + (gt / (1 + np.exp(-gt)) * up) @ W(L["down"]).T
    return norm(x, w.final_norm)[-1], W(w.lm_head)


SPECS = [
    DecoderSpec(2, 128, 2, 1, 64, 200, 150, 32),   # GQA 2:1, FFN with an edge strip
    DecoderSpec(1, 256, 2, 2, 128, 128, 97, 32),   # head_dim 128, MHA
]


@pytest.mark.parametrize("spec", SPECS)
def test_oracle_decoder_matches_dense_float64(spec):
    w = synthetic_weights(spec, n_atoms=64, nnz=4, seed=5, sigma=0.1, norm_jitter=0.1,
                          bias_sigma=0.1)
    tokens = [3, 17, 42, 8, 99 % spec.vocab, 1, 0, 64]
    h32 = odec.hidden_last(w, tokens)
    h64, lm = dense_forward(w, tokens)
    assert rel_l2(h32, h64) < 1e-5
    lg = odec.step_scores(w, tokens)
    assert rel_l2(lg, lm @ h64) < 1e-5


def test_oracle_sanitize():
    h = np.array([1.0, np.nan, -3000.0, np.inf, 10.0], np.float32)
    out = odec.sanitize(h)
    np.testing.assert_allclose(out, [1 / 3, 0, -1000, 0, 10 / 3], rtol=1e-6)
    small = np.array([5.0, -999.0], np.float32)
    assert np.array_equal(odec.sanitize(small), small)


def test_oracle_generate_forced_matches_free():
    # the forced form equals the free run when forced with the free run's own tokens
    spec = SPECS[0]
    w = synthetic_weights(spec, n_atoms=64, nnz=4, seed=6, sigma=0.1)
    toks, sc = odec.generate(w, [5, 6, 7], 4)
    toks2, sc2 = odec.generate(w, [5, 6, 7], 4, forced=toks)
    assert np.array_equal(toks, toks2)
    assert all(np.array_equal(a, b) for a, b in zip(sc, sc2))
    # the repeat penalty is applied to generated tokens: a repeated token only wins when its
    # lead exceeds penalty * temperature-scaled margin
    for i in range(1, 4):
        ts = sc[i] / 0.8
        rep = np.zeros(spec.vocab, bool)
        rep[toks[:i]] = True
        ts = np.where(rep, ts - 1.5, ts)
        assert toks[i] == int(np.argmax(ts))


@pytest.mark.parametrize("spec", [DecoderSpec(2, 256, 4, 2, 64, 96, 150, 32),
                                  DecoderSpec(1, 256, 2, 2, 128, 128, 90, 32)])
def test_cached_step_equals_whole_context_recompute(spec):
    """oracle.decoder.step_cached (cached fp16 K/V context, the device decoder's form) against
    the whole-context recompute of the same sequences: the scores after a context of n tokens
    plus one more agree to the fp16 rounding of the context's K/V, per sequence of a batch of
    sequences that differ; the returned K/V row of position n is the recompute's (fp16)."""
    w = synthetic_weights(spec, n_atoms=64, nnz=4, seed=23, sigma=0.1, norm_jitter=0.1)
    rng = np.random.default_rng(5)
    B, n = 3, 9
    seqs = rng.integers(0, spec.vocab, size=(B, n + 1)).astype(np.int32)
    ctx = [odec.context_kv(w, seqs[b, :n]) for b in range(B)]
    kv = []
    for l in range(spec.n_layers):
        k = np.stack([ctx[b][l][0] for b in range(B)])
        v = np.stack([ctx[b][l][1] for b in range(B)])
        kv.append((oracle.f32_to_f16(k).reshape(k.shape), oracle.f32_to_f16(v).reshape(v.shape)))
    scores, rows = odec.step_cached(w, seqs[:, n], kv, n)
    assert scores.shape == (B, spec.vocab)
    for b in range(B):
        full = odec.step_scores(w, seqs[b])
        assert rel_l2(scores[b], full) < 1e-3, b
        kn, vn = odec.context_kv(w, seqs[b])[0]
        assert np.allclose(oracle.f16_to_f32(rows[0][0][b]).reshape(kn[n].shape), kn[n],
                           rtol=2e-3, atol=2e-3)
        assert np.allclose(oracle.f16_to_f32(rows[0][1][b]).reshape(vn[n].shape), vn[n],
                           rtol=2e-3, atol=2e-3)
    # the batch rows are independent: one sequence alone gives its row
    s1, _ = odec.step_cached(w, seqs[1:2, n], [(k[1:2], v[1:2]) for k, v in kv], n)
    assert np.array_equal(s1[0], scores[1])


@pytest.mark.parametrize("spec", [DecoderSpec(2, 256, 4, 2, 64, 96, 150, 32),
                                  DecoderSpec(1, 256, 2, 2, 128, 128, 90, 32)])
def test_cached_fp32_dense_steps_equal_whole_context_recompute(spec):
    """The forms the long-run GPU checks use: the prompt forward with dense (decoded-once)
    weights, then fp32-cache steps written in place into preallocated caches, against the
    whole-context recompute through the fused product at every step (same scores to float
    summation order: dense and fused products differ only there), and the fp16 path of
    step_cached on the same preallocated layout against its concatenating form."""
    w = synthetic_weights(spec, n_atoms=64, nnz=4, seed=29, sigma=0.1, norm_jitter=0.1,
                          bias_sigma=0.05)
    rng = np.random.default_rng(8)
    n0, steps = 7, 4
    seq = rng.integers(0, spec.vocab, size=n0 + steps).astype(np.int32)
    dense = odec.DenseWeights()
    sc0, kvs = odec.prompt_state(w, seq[:n0], dense)
    assert rel_l2(sc0, odec.step_scores(w, seq[:n0])) < 1e-5
    cap = n0 + steps
    kv = []
    for k, v in kvs:
        kb = np.zeros((1, cap, spec.n_kv_heads, spec.head_dim), np.float32)
        vb = np.zeros_like(kb)
        kb[0, :n0], vb[0, :n0] = k, v
        kv.append((kb, vb))
    for i in range(steps - 1):
        n = n0 + i
        sc, rows = odec.step_cached(w, seq[n:n + 1], kv, n, dense)
        assert rel_l2(sc[0], odec.step_scores(w, seq[:n + 1])) < 1e-5, i
        # the row was written into the preallocated caches at position n
        assert np.array_equal(kv[0][0][0, n], rows[0][0][0])
    # fp16 caches: in place over a preallocated cache == the concatenating form
    n = n0
    kv16 = [(oracle.f32_to_f16(k).reshape(1, n, *k.shape[1:]),
             oracle.f32_to_f16(v).reshape(1, n, *v.shape[1:])) for k, v in kvs]
    a, _ = odec.step_cached(w, seq[n:n + 1], kv16, n)
    pre = []
    for k, v in kv16:
        kb = np.zeros((1, n + 3) + k.shape[2:], np.uint16)
        vb = np.zeros_like(kb)
        kb[:, :n], vb[:, :n] = k, v
        pre.append((kb, vb))
    b, _ = odec.step_cached(w, seq[n:n + 1], pre, n)
    assert np.array_equal(a, b)


def test_attn_cached_f32_matches_orc_attn_decode():
    """The float64 textbook attention of the fp32-cache step against orc_attn_decode on
    fp16-representable caches (the same values in both element types)."""
    rng = np.random.default_rng(3)
    B, n, Hq, Hkv, hd = 2, 40, 6, 2, 64
    q = rng.standard_normal((B, Hq, hd)).astype(np.float32)
    k16 = oracle.f32_to_f16(rng.standard_normal((B, n + 1, Hkv, hd)).astype(np.float32))
    v16 = oracle.f32_to_f16(rng.standard_normal((B, n + 1, Hkv, hd)).astype(np.float32))
    k16 = k16.reshape(B, n + 1, Hkv, hd)
    v16 = v16.reshape(B, n + 1, Hkv, hd)
    kf = oracle.f16_to_f32(k16).reshape(k16.shape)
    vf = oracle.f16_to_f32(v16).reshape(v16.shape)
    got = odec.attn_cached_f32(q, kf, vf, n, Hq, Hkv, hd)
    want = oracle.attn_decode(q, k16, v16, None, Hq, Hkv, hd)
    assert rel_l2(got, want) < 1e-6
