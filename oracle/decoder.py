"""CPU oracle of the SDK decoder (TEST INFRASTRUCTURE ONLY; see the package docstring).

A restatement of run_transformer_decode (api/cortex_sdk.cpp:1543-1696) with the reference's
whole-context recompute and fp32 K/V, built from this package's pinned ops:
  build_token_embeddings (tied: the token's lm_head row)      cortex_sdk.cpp:1480-1541
  rms_norm                                                     cortex_sdk.cpp:1208-1232
  q/k/v/o/gate/up/down linears on HSDB codes (A0 closed form)  orc_hsdb_matmul
  apply_rope_inplace over positions 0..T-1                     cortex_sdk.cpp:1395-1423
  repeat_kv_heads (q head h reads kv head h / (Hq / Hkv))      cortex_sdk.cpp:1453-1478
  Kernels::multi_head_attention, causal, scale 1/sqrt(d)       attention_kernels.cpp:26-113
  add_vectors / silu_mul                                       cortex_sdk.cpp:1234-1256
  output norm, last position                                   cortex_sdk.cpp:1682-1695
and the token choice of select_next_token_from_embedding_transpose (:1032-1206):
sanitize_hidden_for_sampling (:959-976), lm_head scores, select_best_from_logits (:1005-1030).
Weights are the duck type of cortexsdr_amd.decoder.DecoderWeights (spec, layers, lm_head,
final_norm, embedding) so the checker reads the same serialized streams as the device.

step_cached continues B sequences from a given fp16 K/V context (a cached prompt prefix, the
decode step of configs[4]): the same block with the new K/V row appended to the cache at fp16
(as the device cache stores it) and cached decode attention (orc_attn_decode).

DenseWeights decodes every linear once to dense fp32 (hsdr_decompress, bit-exact with the
reference's decompress) so that long contexts run as dense products: the fused product equals
decode-then-dense (pinned in tests/test_oracle.py), so this changes only the summation order.
step_cached also continues fp32 K/V caches (the device decoder's default precision, the
reference recompute's) with textbook attention in float64.

Parity status: every op above is pinned on its own (tests/test_oracle.py); the composition
follows the reference's call sequence, which cannot be compiled here (the SDK needs protobuf
headers), and is checked against an independent float64 dense restatement on tiny models
(tests/test_decoder_oracle.py).
"""
from __future__ import annotations

import numpy as np

from . import (attn_decode, f32_to_f16, hsdb_matmul, hsdr_decompress, mha_causal, rms_norm,
               rope, select_best, silu_mul)


class DenseWeights:
    """Each coded linear decoded once to dense fp32 R x C (hsdr_decompress), keyed by stream."""

    def __init__(self):
        self._w = {}

    def get(self, stream) -> np.ndarray:
        key = id(stream)
        hit = self._w.get(key)
        if hit is None or hit[0] is not stream:
            hit = (stream, hsdr_decompress(stream))
            self._w[key] = hit
        return hit[1]


def _linear(stream, x_tc: np.ndarray, bias=None, dense: DenseWeights | None = None) -> np.ndarray:
    """(T, C) -> (T, R): the reference's run_cached_linear per token on feature-major x (with
    `dense`: x times the decoded W^T, an fp32 dense product)."""
    if dense is not None:
        W = dense.get(stream)
        y = np.asarray(x_tc, np.float32) @ W.T
    else:
        y = hsdb_matmul(stream, np.ascontiguousarray(x_tc.T, np.float32)).T
    if bias is not None:
        y = y + bias[None, :]
    return np.ascontiguousarray(y, np.float32)


def embed_rows(w, tokens) -> np.ndarray:
    table = w.embedding if w.embedding is not None else w.lm_head
    dense = hsdr_decompress(table)
    return dense[np.asarray(tokens, np.int64)].astype(np.float32)


def hidden_last(w, tokens, dense_embed: np.ndarray | None = None) -> np.ndarray:
    """Output-normed hidden state of the last position after the full-context forward."""
    return _forward(w, tokens, dense_embed)[0]


def context_kv(w, tokens, dense_embed: np.ndarray | None = None, dense=None):
    """Per layer the rotated K and the V of every position of the full-context forward,
    (T, Hkv, hd) fp32 each: the context a cached decoder holds after these tokens."""
    return _forward(w, tokens, dense_embed, dense)[1]


def prompt_state(w, tokens, dense=None):
    """The full-context forward over a prompt: (lm_head scores of the position after it,
    per layer (K, V) of every prompt position, (T, Hkv, hd) fp32 each)."""
    h, kvs = _forward(w, tokens, None, dense)
    return _scores(w, sanitize(h)[None, :], dense)[0], kvs


def _scores(w, hs: np.ndarray, dense=None) -> np.ndarray:
    """(B, hidden) sanitized hidden states -> (B, vocab) lm_head scores."""
    if dense is not None:
        return _linear(w.lm_head, hs, None, dense)
    return np.ascontiguousarray(hsdb_matmul(w.lm_head, np.ascontiguousarray(hs.T)).T, np.float32)


def _forward(w, tokens, dense_embed=None, dense=None):
    s = w.spec
    T = len(tokens)
    hd, Hq, Hkv = s.head_dim, s.n_heads, s.n_kv_heads
    rep = Hq // Hkv
    if dense_embed is None and dense is not None:
        dense_embed = dense.get(w.embedding if w.embedding is not None else w.lm_head)
    x = (dense_embed[np.asarray(tokens, np.int64)] if dense_embed is not None
         else embed_rows(w, tokens)).astype(np.float32)
    kvs = []
    for L in w.layers:
        h = rms_norm(x, L["attn_norm"], s.rms_eps)
        q = _linear(L["q"], h, L.get("bq"), dense)
        k = _linear(L["k"], h, L.get("bk"), dense)
        v = _linear(L["v"], h, L.get("bv"), dense)
        q = rope(q, Hq, hd, s.rope_theta, 0)
        k = rope(k, Hkv, hd, s.rope_theta, 0)
        kvs.append((k.reshape(T, Hkv, hd).copy(), v.reshape(T, Hkv, hd).copy()))
        ke = np.repeat(k.reshape(T, Hkv, hd), rep, axis=1).reshape(T, Hq * hd)
        ve = np.repeat(v.reshape(T, Hkv, hd), rep, axis=1).reshape(T, Hq * hd)
        a = mha_causal(q[None], ke[None], ve[None], Hq)[0]
        x = (x + _linear(L["o"], a, None, dense)).astype(np.float32)
        h = rms_norm(x, L["ffn_norm"], s.rms_eps)
        f = silu_mul(_linear(L["gate"], h, None, dense), _linear(L["up"], h, None, dense))
        x = (x + _linear(L["down"], f, None, dense)).astype(np.float32)
    if w.final_norm is not None:
        x = rms_norm(x, w.final_norm, s.rms_eps)
    return x[-1].copy(), kvs


def sanitize(h: np.ndarray) -> np.ndarray:
    """sanitize_hidden_for_sampling (cortex_sdk.cpp:959-976)."""
    out = np.where(np.isfinite(h), h, 0.0).astype(np.float32)
    m = float(np.max(np.abs(out))) if out.size else 0.0
    if m > 1000.0:
        out = (out * np.float32(1000.0 / m)).astype(np.float32)
    return out


def step_scores(w, tokens, dense_embed=None) -> np.ndarray:
    """lm_head scores for the position after `tokens` (before temperature/penalty)."""
    h = sanitize(hidden_last(w, tokens, dense_embed))
    return hsdb_matmul(w.lm_head, h.reshape(-1, 1))[:, 0]


def generate(w, prompt, max_new_tokens, temperature=0.8, penalty=1.5, forced=None):
    """generate_text's loop (cortex_sdk.cpp:1951-2054): returns (tokens, per-step scores).

    With `forced`, step i continues from forced[:i] instead of its own choices (the caller
    compares its own tokens step by step)."""
    s = w.spec
    dense_embed = embed_rows(w, np.arange(s.vocab))
    gen, scores = [], []
    for i in range(max(1, max_new_tokens)):
        ctx = list(prompt) + (list(forced[:i]) if forced is not None else gen)
        lg = step_scores(w, ctx, dense_embed)
        scores.append(lg)
        hist = forced[:i] if forced is not None else gen
        rep = np.zeros(s.vocab, np.uint8)
        rep[np.asarray(hist, np.int64)] = 1
        gen.append(select_best(lg, rep, temperature, penalty))
    return np.asarray(gen, np.int32), scores


def attn_cached_f32(q, kc, vc, n: int, Hq: int, Hkv: int, hd: int) -> np.ndarray:
    """Textbook attention of B queries over positions [0, n] of fp32 caches, in float64:
    q (B, Hq, hd); kc, vc (B, >= n + 1, Hkv, hd); query head h reads KV head h / (Hq / Hkv),
    scale 1 / sqrt(hd) (attention_kernels.cpp:26-113 at the last position)."""
    B = q.shape[0]
    rep = Hq // Hkv
    out = np.empty((B, Hq, hd), np.float32)
    for b in range(B):
        K = np.asarray(kc[b, :n + 1], np.float64)
        V = np.asarray(vc[b, :n + 1], np.float64)
        for h in range(Hq):
            sc = K[:, h // rep, :] @ np.asarray(q[b, h], np.float64) / np.sqrt(hd)
            p = np.exp(sc - sc.max())
            p /= p.sum()
            out[b, h] = p @ V[:, h // rep, :]
    return out


def step_cached(w, tokens, kv, n: int, dense: DenseWeights | None = None):
    """One decode step of B sequences at position n over a cached context.

    tokens: (B,) the token at position n of each sequence; kv: per layer (K, V), each
    (B, T, Hkv, hd) with T >= n, holding positions [0, n): fp16 bits (uint16; the new row is
    rounded to fp16 as the device's fp16 cache stores it) or float32 (fp32 cache). When
    T > n the new row is also written into position n of the given arrays, so a caller can
    keep one preallocated cache per layer. Returns (scores (B, vocab), new rows: per layer
    (K, V) of position n, (B, Hkv, hd), in the cache's element type)."""
    s = w.spec
    hd, Hq, Hkv = s.head_dim, s.n_heads, s.n_kv_heads
    tokens = np.asarray(tokens, np.int64)
    B = tokens.size
    table = w.embedding if w.embedding is not None else w.lm_head
    if dense is not None:
        x = dense.get(table)[tokens].astype(np.float32)
    else:
        x = hsdr_decompress(table)[tokens].astype(np.float32)
    rows = []
    for L, (kc, vc) in zip(w.layers, kv):
        f32 = np.asarray(kc).dtype == np.float32
        h = rms_norm(x, L["attn_norm"], s.rms_eps)
        q = _linear(L["q"], h, L.get("bq"), dense)
        k = _linear(L["k"], h, L.get("bk"), dense)
        v = _linear(L["v"], h, L.get("bv"), dense)
        for b in range(B):  # every sequence at position n
            q[b] = rope(q[b], Hq, hd, s.rope_theta, n)
            k[b] = rope(k[b], Hkv, hd, s.rope_theta, n)
        if f32:
            kr = k.reshape(B, 1, Hkv, hd).astype(np.float32)
            vr = v.reshape(B, 1, Hkv, hd).astype(np.float32)
        else:
            kr = f32_to_f16(k).reshape(B, 1, Hkv, hd)
            vr = f32_to_f16(v).reshape(B, 1, Hkv, hd)
        rows.append((kr[:, 0].copy(), vr[:, 0].copy()))
        kc4 = np.asarray(kc).reshape(B, -1, Hkv, hd)
        vc4 = np.asarray(vc).reshape(B, -1, Hkv, hd)
        if kc4.shape[1] > n:  # room for position n: write it in place
            kc4[:, n] = kr[:, 0]
            vc4[:, n] = vr[:, 0]
            kfull, vfull = kc4, vc4
        else:
            kfull = np.concatenate([kc4[:, :n], kr], axis=1)
            vfull = np.concatenate([vc4[:, :n], vr], axis=1)
        if f32:
            a = attn_cached_f32(q.reshape(B, Hq, hd), kfull, vfull, n, Hq, Hkv, hd)
        else:
            lens = np.full(B, n + 1, np.int32)
            a = attn_decode(q.reshape(B, Hq, hd), kfull, vfull, lens, Hq, Hkv, hd)
        x = (x + _linear(L["o"], a.reshape(B, Hq * hd), None, dense)).astype(np.float32)
        h = rms_norm(x, L["ffn_norm"], s.rms_eps)
        f = silu_mul(_linear(L["gate"], h, None, dense), _linear(L["up"], h, None, dense))
        x = (x + _linear(L["down"], f, None, dense)).astype(np.float32)
    if w.final_norm is not None:
        x = rms_norm(x, w.final_norm, s.rms_eps)
    hs = np.stack([sanitize(x[b]) for b in range(B)])
    return _scores(w, hs, dense), rows
