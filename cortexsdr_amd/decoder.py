"""Host side of the native decoder: model description, seeded synthetic weights and the
device engine behind csdr_decoder_* (include/cortexsdr_hip.h).

Reference roles (cortexSDR tree):
  CortexInferenceEngine + ensure_native_generation_ready   api/cortex_sdk.cpp:72-111, 1698-1760
  run_transformer_decode (one Llama/Qwen block stack)       api/cortex_sdk.cpp:1543-1696
  cortex_inference_engine_generate_text (the token loop)    api/cortex_sdk.cpp:1951-2054
The reference reads the block weights by name from a .sdr archive (transformer_blocks, one
LayerInfo per linear); here every linear is an HSDB segment already resident on the device.
Errors are raised as CsdrError with the C-ABI status.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import zlib

import numpy as np

from . import _lib, synth
from .hsdr import HsdbSegment

LINEARS = ("q", "k", "v", "o", "gate", "up", "down")


@dataclasses.dataclass(frozen=True)
class DecoderSpec:
    n_layers: int
    hidden: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    max_ctx: int
    rope_theta: float = 1e6
    rms_eps: float = 1e-5
    kv_dtype: str = "f32"   # K/V cache element: "f32" (the reference's precision) or "f16"

    def shapes(self) -> dict:
        """(rows, cols) of each linear of one block (y = W x, W row-major R x C)."""
        H, F, kv = self.hidden, self.ffn, self.n_kv_heads * self.head_dim
        return {"q": (H, H), "k": (kv, H), "v": (kv, H), "o": (H, H), "gate": (F, H),
                "up": (F, H), "down": (H, F)}


# The Qwen2-0.5B shape of the measured decode workload (24 layers, hidden 896, 14 query /
# 2 KV heads of 64, SwiGLU 4864, vocab 151936); context for a 512-token prompt + 128 tokens.
QWEN2_0_5B = DecoderSpec(24, 896, 14, 2, 64, 4864, 151936, 640)


@dataclasses.dataclass
class DecoderWeights:
    """Serialized weights: HSDB streams per linear plus fp32 norm/bias vectors."""
    spec: DecoderSpec
    layers: list            # per layer: {name: stream bytes} | {"attn_norm", "ffn_norm", "bq"...}
    lm_head: bytes
    final_norm: np.ndarray | None
    embedding: bytes | None = None  # None = tied to lm_head

    def code_bytes(self) -> int:
        """Device bytes of the per-slot code words (4 B per slot) of all linears."""
        def slots_bytes(stream):
            from .formats import parse_header
            h = parse_header(stream)
            return h.n_tiles * h.slots * 4
        n = sum(slots_bytes(L[name]) for L in self.layers for name in LINEARS)
        return n + slots_bytes(self.lm_head)


def _seed(base: int, *parts) -> int:
    return (base * 1000003 + zlib.crc32(repr(parts).encode())) & 0x7FFFFFFF


def synthetic_weights(spec: DecoderSpec, n_atoms: int = 1024, nnz: int = 8, seed: int = 0,
                      sigma: float = 0.5, norm_jitter: float = 0.0, bias_sigma: float = 0.0,
                      final_norm_scale: float = 1.0) -> DecoderWeights:
    """Random-init weights: every linear block-coded against ONE shared dictionary of n_atoms
    unit-norm atoms of 64 (nnz atoms per 64-column block, coefficients N(0, sigma)); RMSNorm
    weights 1 (+ N(0, norm_jitter)); q/k/v biases N(0, bias_sigma) when bias_sigma > 0."""
    D = synth.dictionary(n_atoms, 64, _seed(seed, "dict"))
    layers = []
    for l in range(spec.n_layers):
        L = {}
        for name, (R, Cc) in spec.shapes().items():
            L[name] = synth.hsdb_layer(R, Cc, n_atoms, nnz, D=D, sigma=sigma,
                                       seed_codes=_seed(seed, l, name),
                                       edge_seed=_seed(seed, l, name, "edge"))
        for nm in ("attn_norm", "ffn_norm"):
            w = np.ones(spec.hidden, np.float32)
            if norm_jitter:
                w += synth.normal(_seed(seed, l, nm), spec.hidden, sigma=norm_jitter)
            L[nm] = w.astype(np.float32)
        if bias_sigma:
            kvw = spec.n_kv_heads * spec.head_dim
            for nm, n in (("bq", spec.hidden), ("bk", kvw), ("bv", kvw)):
                L[nm] = synth.normal(_seed(seed, l, nm), n, sigma=bias_sigma).astype(np.float32)
        layers.append(L)
    lm = synth.hsdb_layer(spec.vocab, spec.hidden, n_atoms, nnz, D=D, sigma=sigma,
                          seed_codes=_seed(seed, "lm_head"))
    fn = np.full(spec.hidden, final_norm_scale, np.float32)
    if norm_jitter:
        fn *= (1.0 + synth.normal(_seed(seed, "final_norm"), spec.hidden,
                                  sigma=norm_jitter)).astype(np.float32)
    return DecoderWeights(spec, layers, lm, fn.astype(np.float32))


def _fptr(a):
    if a is None:
        return None
    return a.ctypes.data_as(C.c_void_p)


class Decoder:
    """A device decoder over resident HSDB segments (greedy / penalised argmax) decoding
    `batch` sequences in lockstep; per-sequence arrays are sequence-major (batch, ...)."""

    def __init__(self, weights: DecoderWeights, batch: int = 1, prefill_chunk: int | None = None,
                 stream_layers: bool = False, prefetch: bool = True):
        """stream_layers: the blocks' code words stay in pinned host memory and each block is
        copied to the device when it runs (csdr_decoder_set_layer_prefetch: with prefetch,
        the next block's copy overlaps the current block's kernels)."""
        import torch

        if not torch.cuda.is_available():
            raise RuntimeError("cortexsdr_amd.Decoder needs a HIP device (no CPU fallback)")
        self._lib = _lib.load()
        self.spec = s = weights.spec
        if s.kv_dtype not in ("f32", "f16"):
            raise ValueError("kv_dtype must be 'f32' or 'f16'")
        cfg = _lib.DecoderConfig(s.n_layers, s.hidden, s.n_heads, s.n_kv_heads, s.head_dim,
                                 s.ffn, s.vocab, s.max_ctx, s.rope_theta, s.rms_eps,
                                 0 if s.kv_dtype == "f32" else 1)
        h = C.c_void_p()
        _lib.check(self._lib.csdr_decoder_create_batched(C.byref(cfg), int(batch), C.byref(h)))
        self._h = h
        self.batch = int(batch)
        self._segs = []
        self._keep = []
        try:
            for l, L in enumerate(weights.layers):
                segs = [HsdbSegment(L[name], host_codes=stream_layers) for name in LINEARS]
                self._segs += segs
                vecs = [np.ascontiguousarray(L[nm], np.float32) if L.get(nm) is not None
                        else None for nm in ("attn_norm", "ffn_norm", "bq", "bk", "bv")]
                self._keep.append(vecs)
                _lib.check(self._lib.csdr_decoder_set_layer(
                    self._h, l, *[sg._h for sg in segs], *[_fptr(v) for v in vecs]))
            self._lm = HsdbSegment(weights.lm_head)
            self._emb = HsdbSegment(weights.embedding) if weights.embedding else None
            self._segs += [self._lm] + ([self._emb] if self._emb else [])
            fn = (np.ascontiguousarray(weights.final_norm, np.float32)
                  if weights.final_norm is not None else None)
            _lib.check(self._lib.csdr_decoder_set_output(
                self._h, self._lm._h, _fptr(fn), self._emb._h if self._emb else None))
            if prefill_chunk is not None:
                self.set_prefill_chunk(prefill_chunk)
            if not prefetch:
                self.set_layer_prefetch(False)
        except Exception:
            self.close()
            raise

    def device_bytes(self) -> int:
        return sum(int(sg.info["device_bytes"]) for sg in self._segs)

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.csdr_decoder_free(self._h)
            self._h = None
        for sg in getattr(self, "_segs", []):
            sg.free()
        self._segs = []

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_lazy_selection(self, emb, penalty: float = 1.0) -> None:
        """Choose tokens by the text CLI's lazy HSDR scoring against emb (a
        LazyHsdrEmbedding of vocab x hidden, kept alive here), or by the lm_head scores
        again when emb is None."""
        self._lazy = emb
        _lib.check(self._lib.csdr_decoder_set_lazy_selection(self._h, emb._h if emb else None,
                                                             penalty))

    def set_layer_prefetch(self, enable: bool) -> None:
        _lib.check(self._lib.csdr_decoder_set_layer_prefetch(self._h, int(bool(enable))))

    def streamed_bytes(self) -> int:
        """Code bytes the streamed blocks copy to the device per step."""
        return int(self._lib.csdr_decoder_streamed_bytes(self._h))

    def set_prefill_chunk(self, tokens: int) -> None:
        """Prompt tokens per sequence in one multi-token prefill pass (0: one decode step
        per prompt position)."""
        _lib.check(self._lib.csdr_decoder_set_prefill_chunk(self._h, int(tokens)))

    # ------------------------------------------------------------------ generation
    def prefill(self, prompt, temperature: float = 0.8, penalty: float = 1.5) -> None:
        """prompt: n ids (batch 1) or (batch, n) ids."""
        p = np.ascontiguousarray(prompt, np.int32).reshape(self.batch, -1)
        _lib.check(self._lib.csdr_decoder_prefill(self._h, _fptr(p), p.shape[1], temperature,
                                                  penalty))

    def decode(self, n_steps: int, temperature: float = 0.8, penalty: float = 1.5) -> None:
        _lib.check(self._lib.csdr_decoder_decode(self._h, n_steps, temperature, penalty))

    def tokens(self, first: int, count: int) -> np.ndarray:
        """(count,) at batch 1, else (batch, count)."""
        out = np.empty((self.batch, count), np.int32)
        _lib.check(self._lib.csdr_decoder_tokens(self._h, first, count, _fptr(out)))
        return out[0] if self.batch == 1 else out

    def logits(self) -> np.ndarray:
        """(vocab,) at batch 1, else (batch, vocab)."""
        out = np.empty((self.batch, self.spec.vocab), np.float32)
        _lib.check(self._lib.csdr_decoder_logits(self._h, _fptr(out)))
        return out[0] if self.batch == 1 else out

    def load_kv(self, layer: int, k, v, n: int) -> None:
        """Import fp16 K/V of positions [0, n), (batch, n, kv heads, head_dim) contiguous
        (device torch tensors or host numpy arrays)."""
        kp = k.data_ptr() if hasattr(k, "data_ptr") else k.ctypes.data
        vp = v.data_ptr() if hasattr(v, "data_ptr") else v.ctypes.data
        _lib.check(self._lib.csdr_decoder_load_kv(self._h, layer, kp, vp, n))

    def set_position(self, position: int, token) -> None:
        """token: one id for every sequence, or batch ids."""
        t = np.ascontiguousarray(np.broadcast_to(np.asarray(token, np.int32), (self.batch,)))
        _lib.check(self._lib.csdr_decoder_set_position_batch(self._h, position, _fptr(t)))

    def position(self) -> int:
        return int(self._lib.csdr_decoder_position(self._h))

    def generate(self, prompt, max_new_tokens: int, temperature: float = 0.8,
                 penalty: float = 1.5, eos_id: int = -1) -> np.ndarray:
        """generate_text's loop (api/cortex_sdk.cpp:1951-2054) on token ids."""
        p = np.ascontiguousarray(prompt, np.int32).reshape(self.batch, -1)
        n = max(1, int(max_new_tokens))
        out = np.empty((self.batch, n), np.int32)
        ng = (C.c_int * self.batch)()
        _lib.check(self._lib.csdr_decoder_generate(self._h, _fptr(p), p.shape[1], n, temperature,
                                                   penalty, eos_id, _fptr(out), ng))
        if self.batch == 1:
            return out[0, :ng[0]]
        return [out[b, :ng[b]] for b in range(self.batch)]
