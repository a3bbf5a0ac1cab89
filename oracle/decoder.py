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

Parity status: every op above is pinned on its own (tests/test_oracle.py); the composition
follows the reference's call sequence, which cannot be compiled here (the SDK needs protobuf
headers), and is checked against an independent float64 dense restatement on tiny models
(tests/test_decoder_oracle.py).
"""
from __future__ import annotations

import numpy as np

from . import (attn_decode, f32_to_f16, hsdb_matmul, hsdr_decompress, mha_causal, rms_norm,
               rope, select_best, silu_mul)


def _linear(stream, x_tc: np.ndarray, bias=None) -> np.ndarray:
    """(T, C) -> (T, R): the reference's run_cached_linear per token on feature-major x."""
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


def context_kv(w, tokens, dense_embed: np.ndarray | None = None):
    """Per layer the rotated K and the V of every position of the full-context forward,
    (T, Hkv, hd) fp32 each: the context a cached decoder holds after these tokens."""
    return _forward(w, tokens, dense_embed)[1]


def _forward(w, tokens, dense_embed=None):
    s = w.spec
    T = len(tokens)
    hd, Hq, Hkv = s.head_dim, s.n_heads, s.n_kv_heads
    rep = Hq // Hkv
    x = (dense_embed[np.asarray(tokens, np.int64)] if dense_embed is not None
         else embed_rows(w, tokens)).astype(np.float32)
    kvs = []
    for L in w.layers:
        h = rms_norm(x, L["attn_norm"], s.rms_eps)
        q = _linear(L["q"], h, L.get("bq"))
        k = _linear(L["k"], h, L.get("bk"))
        v = _linear(L["v"], h, L.get("bv"))
        q = rope(q, Hq, hd, s.rope_theta, 0)
        k = rope(k, Hkv, hd, s.rope_theta, 0)
        kvs.append((k.reshape(T, Hkv, hd).copy(), v.reshape(T, Hkv, hd).copy()))
        ke = np.repeat(k.reshape(T, Hkv, hd), rep, axis=1).reshape(T, Hq * hd)
        ve = np.repeat(v.reshape(T, Hkv, hd), rep, axis=1).reshape(T, Hq * hd)
        a = mha_causal(q[None], ke[None], ve[None], Hq)[0]
        x = (x + _linear(L["o"], a)).astype(np.float32)
        h = rms_norm(x, L["ffn_norm"], s.rms_eps)
        f = silu_mul(_linear(L["gate"], h), _linear(L["up"], h))
        x = (x + _linear(L["down"], f)).astype(np.float32)
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


def step_cached(w, tokens, kv, n: int):
    """One decode step of B sequences at position n over a cached context.

    tokens: (B,) the token at position n of each sequence; kv: per layer (K, V), each
    (B, n, Hkv, hd) fp16 bits (uint16) for positions [0, n). Returns (scores (B, vocab),
    new rows: per layer (K, V) of position n, (B, Hkv, hd) fp16 bits) -- the rows the next
    step's context appends."""
    s = w.spec
    hd, Hq, Hkv = s.head_dim, s.n_heads, s.n_kv_heads
    tokens = np.asarray(tokens, np.int64)
    B = tokens.size
    table = w.embedding if w.embedding is not None else w.lm_head
    x = hsdr_decompress(table)[tokens].astype(np.float32)
    rows = []
    for L, (kc, vc) in zip(w.layers, kv):
        h = rms_norm(x, L["attn_norm"], s.rms_eps)
        q = _linear(L["q"], h, L.get("bq"))
        k = _linear(L["k"], h, L.get("bk"))
        v = _linear(L["v"], h, L.get("bv"))
        for b in range(B):  # every sequence at position n
            q[b] = rope(q[b], Hq, hd, s.rope_theta, n)
            k[b] = rope(k[b], Hkv, hd, s.rope_theta, n)
        k16 = f32_to_f16(k).reshape(B, 1, Hkv, hd)
        v16 = f32_to_f16(v).reshape(B, 1, Hkv, hd)
        rows.append((k16[:, 0], v16[:, 0]))
        kfull = np.concatenate([np.asarray(kc, np.uint16).reshape(B, n, Hkv, hd), k16], axis=1)
        vfull = np.concatenate([np.asarray(vc, np.uint16).reshape(B, n, Hkv, hd), v16], axis=1)
        a = attn_decode(q.reshape(B, Hq, hd), kfull, vfull, None, Hq, Hkv, hd)
        x = (x + _linear(L["o"], a.reshape(B, Hq * hd))).astype(np.float32)
        h = rms_norm(x, L["ffn_norm"], s.rms_eps)
        f = silu_mul(_linear(L["gate"], h), _linear(L["up"], h))
        x = (x + _linear(L["down"], f)).astype(np.float32)
    if w.final_norm is not None:
        x = rms_norm(x, w.final_norm, s.rms_eps)
    hs = np.stack([sanitize(x[b]) for b in range(B)])
    scores = hsdb_matmul(w.lm_head, np.ascontiguousarray(hs.T)).T
    return np.ascontiguousarray(scores, np.float32), rows
