"""Host-side mirror of the reference's archive and inference-engine surfaces on the C-ABI.

Reference roles (cortexSDR tree):
  SdrArchive        AIDecompressor::readArchiveHeaders / readCompressedBytes
                    (core/AIDecompressor.cpp:78-262, 418-435) as SDRModelLoader uses them
                    (SparseInferenceEngine.cpp:1055-1072)
  HsdaArchive       HSDAReader (strategies/HierarchicalSDRStrategy.hpp:368-411): by-name
                    matmul / decompress over a shared-dictionary archive
  InferenceEngine   the SDK handle (api/cortex_sdk.h:37-281): run_layer, generate_text,
                    the option setters and the last-run stats
Index parsing needs no device; loads and products run the HIP library (no CPU fallback).
"""
from __future__ import annotations

import ctypes as C
import json

import numpy as np

from . import _lib


def _chk(rc):
    _lib.check(rc)


class SdrArchive:
    """A .sdr archive's index and payloads."""

    def __init__(self, path: str):
        self._lib = _lib.load()
        h = C.c_void_p()
        _chk(self._lib.csdr_archive_open(path.encode(), C.byref(h)))
        self._h = h

    def close(self):
        if getattr(self, "_h", None):
            self._lib.csdr_archive_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self) -> int:
        return int(self._lib.csdr_archive_count(self._h))

    def info(self, i: int) -> dict:
        si = _lib.SegmentInfo()
        _chk(self._lib.csdr_archive_info(self._h, i, C.byref(si)))
        return {
            "name": si.name.decode(), "data_format": si.data_format.decode(),
            "layer_type": si.layer_type.decode(), "layer_name": si.layer_name.decode(),
            "original_type": si.original_type, "strategy_id": si.strategy_id,
            "original_size": si.original_size, "compressed_size": si.compressed_size,
            "data_offset": si.data_offset, "layer_index": si.layer_index,
            "dims": tuple(si.dims[:si.n_dims]) if si.has_metadata else None,
            "sparsity_ratio": si.sparsity_ratio,
            "input_shape": tuple(si.input_shape[:si.n_input_dims]),
            "output_shape": tuple(si.output_shape[:si.n_output_dims]),
        }

    def find(self, name: str) -> int:
        i = C.c_size_t()
        _chk(self._lib.csdr_archive_find(self._h, name.encode(), C.byref(i)))
        return i.value

    def read(self, name_or_index) -> bytes:
        i = name_or_index if isinstance(name_or_index, int) else self.find(name_or_index)
        n = C.c_size_t()
        _chk(self._lib.csdr_archive_read(self._h, i, None, 0, C.byref(n)))
        buf = C.create_string_buffer(max(n.value, 1))
        _chk(self._lib.csdr_archive_read(self._h, i, buf, n.value, C.byref(n)))
        return buf.raw[:n.value]


class HsdaArchive:
    """A shared-dictionary archive: segments by name, loaded to the device on request."""

    def __init__(self, path: str | None = None, data: bytes | None = None):
        self._lib = _lib.load()
        h = C.c_void_p()
        if data is not None:
            self._buf = bytes(data)
            _chk(self._lib.csdr_hsda_open_memory(self._buf, len(self._buf), C.byref(h)))
        else:
            _chk(self._lib.csdr_hsda_open(path.encode(), C.byref(h)))
        self._h = h

    def close(self):
        if getattr(self, "_h", None):
            self._lib.csdr_hsda_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self) -> int:
        return int(self._lib.csdr_hsda_count(self._h))

    def num_dictionaries(self) -> int:
        return int(self._lib.csdr_hsda_dictionary_count(self._h))

    def segment(self, i: int):
        name = C.c_char_p()
        di = C.c_uint32()
        orig = C.c_uint64()
        _chk(self._lib.csdr_hsda_segment(self._h, i, C.byref(name), C.byref(di), C.byref(orig)))
        return name.value.decode(), di.value, orig.value

    def load(self, name: str):
        """The named segment as a device-resident HsdbSegment."""
        from .hsdr import HsdbSegment

        h = C.c_void_p()
        _chk(self._lib.csdr_hsda_load(self._h, name.encode(), None, C.byref(h)))
        return HsdbSegment.from_handle(h)


class EngineError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def _ce(err):
    if err.code != 0:
        raise EngineError(err.code, err.message.decode() if err.message else "")


class InferenceEngine:
    """cortex_inference_engine_* on a .sdr archive."""

    def __init__(self, path: str):
        self._lib = _lib.load()
        h = C.c_void_p()
        _ce(self._lib.cortex_inference_engine_create(path.encode(), C.byref(h)))
        self._h = h

    def close(self):
        if getattr(self, "_h", None):
            _ce(self._lib.cortex_inference_engine_free(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def run_layer(self, name: str, x: np.ndarray, out_size: int | None = None) -> np.ndarray:
        """x: (M, C) or (C,) fp32 host array -> (M, R) (linear_forward's layout)."""
        x = np.ascontiguousarray(x, np.float32)
        n = C.c_size_t()
        cap = out_size if out_size is not None else 1 << 26
        out = np.empty(max(cap, 1), np.float32)
        while True:
            err = self._lib.cortex_inference_engine_run_layer(
                self._h, name.encode(), x.ctypes.data, x.size, out.ctypes.data, cap, C.byref(n))
            if err.code == -3 and out_size is None and n.value > cap:  # grow and retry
                cap = n.value
                out = np.empty(cap, np.float32)
                continue
            _ce(err)
            return out[:n.value].copy()

    def run(self, x: np.ndarray, out_size: int | None = None) -> np.ndarray:
        """cortex_inference_engine_run: the archive's layer chain on x (M x C floats)."""
        x = np.ascontiguousarray(x, np.float32).ravel()
        cap = out_size if out_size is not None else max(1 << 16, 64 * x.size)
        y = np.empty(cap, np.float32)
        n = C.c_size_t()
        _ce(self._lib.cortex_inference_engine_run(self._h, x.ctypes.data_as(C.c_void_p), x.size,
                                                  y.ctypes.data_as(C.c_void_p), cap,
                                                  C.byref(n)))
        return y[:n.value].copy()

    def generate(self, prompt_ids, max_new_tokens: int) -> list:
        txt = C.c_void_p()
        p = " ".join(str(int(t)) for t in prompt_ids).encode()
        _ce(self._lib.cortex_inference_engine_generate_text(self._h, p, max_new_tokens,
                                                            C.byref(txt)))
        s = C.cast(txt, C.c_char_p).value.decode()
        self._lib.cortex_free_string(txt)
        return [int(t) for t in s.split()]

    def stats(self) -> dict:
        txt = C.c_void_p()
        _ce(self._lib.cortex_inference_engine_get_last_run_stats_json(self._h, C.byref(txt)))
        s = C.cast(txt, C.c_char_p).value.decode()
        self._lib.cortex_free_string(txt)
        return json.loads(s)

    def memory_usage(self) -> int:
        n = C.c_size_t()
        _ce(self._lib.cortex_inference_engine_get_memory_usage(self._h, C.byref(n)))
        return n.value

    def set_memory_pool(self, mb: int):
        _ce(self._lib.cortex_inference_engine_init_memory_pool(self._h, mb))

    def set_aggressive_memory(self, enable: bool):
        """Also the decoder's residency: on, generate_text's blocks stay in pinned host memory
        and are streamed to the device when they run."""
        _ce(self._lib.cortex_inference_engine_enable_aggressive_memory(self._h, int(enable)))

    def set_layer_prefetch(self, enable: bool):
        """Streamed blocks: copy the next block while the current one runs (default on)."""
        _ce(self._lib.cortex_inference_engine_enable_layer_prefetch(self._h, int(enable)))

    def matmul_device(self, name: str, x, y, stream=None):
        """Device x (C, M) fp32/fp16 torch tensor -> device y (R, M) fp32."""
        import torch

        dt = 1 if x.dtype == torch.float16 else 0
        M = x.shape[1] if x.dim() == 2 else 1
        sp = int((stream or torch.cuda.current_stream()).cuda_stream)
        _ce(self._lib.cortex_inference_engine_matmul_device(
            self._h, name.encode(), x.data_ptr(), dt, M, y.data_ptr(), sp))
        return y
