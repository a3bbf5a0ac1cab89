"""Loader for the in-tree HIP library (libcortexsdr_amd.so) and its C-ABI signatures.

The library must be built (python -m cortexsdr_amd.build); there is no CPU fallback: every
compute entry point of this package runs the HIP kernels or raises.

torch is imported before the library is loaded so that both bind the same HIP runtime
(torch ships its own libamdhip64 with the same SONAME); load() then checks that only one
HIP runtime is mapped into the process.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcortexsdr_amd.so")

_lib = None


class CsdrError(RuntimeError):
    """A negative status from the C-ABI; .code holds it."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class HsdbInfo(C.Structure):
    _fields_ = [
        ("rows", C.c_uint32), ("cols", C.c_uint32), ("tile_rows", C.c_uint32),
        ("tile_cols", C.c_uint32), ("n_atoms", C.c_uint32), ("n_stages", C.c_uint32),
        ("k_per_stage", C.c_uint32), ("slots", C.c_uint32), ("n_block_cols", C.c_uint32),
        ("chunk_blocks", C.c_uint32), ("edge_cols", C.c_uint32), ("is_hsdb", C.c_uint32),
        ("code_bytes", C.c_uint64), ("device_bytes", C.c_uint64),
    ]


_vp = C.c_void_p
_sz = C.c_size_t

# name -> (restype, argtypes); every symbol declared in include/cortexsdr_hip.h
SIGNATURES = {
    "csdr_last_error": (C.c_char_p, []),
    "csdr_version": (C.c_char_p, []),
    "csdr_hsdb_load": (C.c_int, [_vp, _sz, _vp, C.POINTER(_vp)]),
    "csdr_hsdb_free": (C.c_int, [_vp]),
    "csdr_hsdb_get_info": (C.c_int, [_vp, C.POINTER(HsdbInfo)]),
    "csdr_hsdb_workspace_bytes": (_sz, [_vp, C.c_int]),
    "csdr_hsdb_matmul": (C.c_int, [_vp, _vp, C.c_int, C.c_int, _vp, _vp, _sz, _vp]),
    "csdr_hsdb_group_workspace_bytes": (_sz, [C.c_int, C.POINTER(_vp), C.c_int]),
    "csdr_hsdb_matmul_group": (C.c_int, [C.c_int, C.POINTER(_vp), C.POINTER(_vp), C.c_int,
                                         C.c_int, C.POINTER(_vp), _vp, _sz, _vp]),
    "csdr_hsdb_dx_group": (C.c_int, [C.c_int, C.POINTER(_vp), C.POINTER(_vp), C.c_int,
                                     C.c_int, C.POINTER(_vp), _vp, _sz, _vp]),
    "csdr_hsdb_gather_group": (C.c_int, [C.c_int, C.POINTER(_vp), C.POINTER(_vp), C.c_int,
                                         C.c_int, C.POINTER(_vp), _vp, _sz, _vp]),
    "csdr_hsdb_decompress": (C.c_int, [_vp, _vp, _vp]),
    "csdr_hsdb_export_codes": (C.c_int, [_vp, _vp, _vp, _vp]),
    "csdr_q4k_linear": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _vp, C.c_int, C.c_int, _vp,
                                  _vp]),
    "csdr_q4k_dequant": (C.c_int, [_vp, _sz, C.c_int, _vp, _vp]),
    "csdr_gguf_format": (C.c_int, [C.c_char_p]),
    "csdr_gguf_block": (C.c_int, [C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "csdr_gguf_linear": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _vp, C.c_int, C.c_int, _vp,
                                   _vp]),
    "csdr_gguf_dequant": (C.c_int, [_vp, C.c_int, _sz, _vp, _vp]),
    "csdr_hsdb_matmul_group_ex": (C.c_int, [C.c_int, C.POINTER(_vp), C.POINTER(_vp), C.c_int,
                                            C.c_int, C.POINTER(_vp), C.POINTER(_vp), C.c_int,
                                            _vp, _sz, _vp]),
    "csdr_hsdb_decode_row": (C.c_int, [_vp, _vp, C.c_int, _vp, _vp]),
    "csdr_hsdb_decode_rows": (C.c_int, [_vp, _vp, C.c_int, _vp, _vp]),
    "csdr_rms_norm": (C.c_int, [_vp, _vp, C.c_int, C.c_int, C.c_float, _vp, _vp]),
    "csdr_silu_mul": (C.c_int, [_vp, _vp, _sz, _vp, _vp]),
    "csdr_rope_kv": (C.c_int, [_vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int, _vp,
                               C.c_float, _vp, _vp, C.c_int, _vp]),
    "csdr_attn_decode_workspace_bytes": (_sz, [C.c_int, C.c_int, C.c_int, C.c_int]),
    "csdr_attn_decode": (C.c_int, [_vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int,
                                   C.c_int, C.c_int, C.c_float, _vp, _vp, _sz, _vp]),
    "csdr_select_workspace_bytes": (_sz, []),
    "csdr_select_best": (C.c_int, [_vp, C.c_int, _vp, C.c_float, C.c_float, _vp, _vp, _vp,
                                   _vp, _sz, _vp]),
    "csdr_decoder_create": (C.c_int, [_vp, C.POINTER(_vp)]),
    "csdr_decoder_free": (C.c_int, [_vp]),
    "csdr_decoder_set_layer": (C.c_int, [_vp, C.c_int] + [_vp] * 7 + [_vp] * 5),
    "csdr_decoder_set_output": (C.c_int, [_vp, _vp, _vp, _vp]),
    "csdr_decoder_prefill": (C.c_int, [_vp, _vp, C.c_int, C.c_float, C.c_float]),
    "csdr_decoder_decode": (C.c_int, [_vp, C.c_int, C.c_float, C.c_float]),
    "csdr_decoder_tokens": (C.c_int, [_vp, C.c_int, C.c_int, _vp]),
    "csdr_decoder_generate": (C.c_int, [_vp, _vp, C.c_int, C.c_int, C.c_float, C.c_float,
                                        C.c_int, _vp, _vp]),
    "csdr_decoder_logits": (C.c_int, [_vp, _vp]),
    "csdr_decoder_position": (C.c_int, [_vp]),
    "csdr_decoder_load_kv": (C.c_int, [_vp, C.c_int, _vp, _vp, C.c_int]),
    "csdr_decoder_set_position": (C.c_int, [_vp, C.c_int, C.c_int32]),
    "csdr_decoder_create_batched": (C.c_int, [_vp, C.c_int, C.POINTER(_vp)]),
    "csdr_decoder_batch": (C.c_int, [_vp]),
    "csdr_decoder_set_position_batch": (C.c_int, [_vp, C.c_int, _vp]),
}


class SegmentInfo(C.Structure):
    _fields_ = [
        ("name", C.c_char_p), ("data_format", C.c_char_p), ("layer_type", C.c_char_p),
        ("layer_name", C.c_char_p), ("original_type", C.c_uint32), ("strategy_id", C.c_uint32),
        ("original_size", C.c_uint64), ("compressed_size", C.c_uint64),
        ("data_offset", C.c_uint64), ("layer_index", C.c_uint32), ("has_metadata", C.c_uint32),
        ("n_dims", C.c_uint32), ("dims", C.c_uint32 * 8), ("sparsity_ratio", C.c_float),
        ("n_input_dims", C.c_uint32), ("input_shape", C.c_uint32 * 8),
        ("n_output_dims", C.c_uint32), ("output_shape", C.c_uint32 * 8),
    ]


class Dictionary(C.Structure):
    _fields_ = [
        ("tile_rows", C.c_uint32), ("tile_cols", C.c_uint32), ("n_atoms", C.c_uint32),
        ("n_stages", C.c_uint32), ("k_per_stage", C.c_uint32), ("stage_decay", C.c_float),
        ("stage_scales", C.c_void_p), ("n_stage_scales", C.c_uint32), ("atoms", C.c_void_p),
        ("n_atom_floats", C.c_size_t),
    ]


class CortexError(C.Structure):
    _fields_ = [("message", C.c_char_p), ("code", C.c_int)]


_ce = CortexError
SIGNATURES.update({
    "csdr_archive_open": (C.c_int, [C.c_char_p, C.POINTER(_vp)]),
    "csdr_archive_close": (C.c_int, [_vp]),
    "csdr_archive_count": (_sz, [_vp]),
    "csdr_archive_info": (C.c_int, [_vp, _sz, C.POINTER(SegmentInfo)]),
    "csdr_archive_find": (C.c_int, [_vp, C.c_char_p, C.POINTER(_sz)]),
    "csdr_archive_read": (C.c_int, [_vp, _sz, _vp, _sz, C.POINTER(_sz)]),
    "csdr_hsdb_load_codes": (C.c_int, [_vp, _sz, C.POINTER(Dictionary), _vp, C.POINTER(_vp)]),
    "csdr_hsda_open": (C.c_int, [C.c_char_p, C.POINTER(_vp)]),
    "csdr_hsda_open_memory": (C.c_int, [_vp, _sz, C.POINTER(_vp)]),
    "csdr_hsda_close": (C.c_int, [_vp]),
    "csdr_hsda_count": (_sz, [_vp]),
    "csdr_hsda_dictionary_count": (_sz, [_vp]),
    "csdr_hsda_segment": (C.c_int, [_vp, _sz, C.POINTER(C.c_char_p), C.POINTER(C.c_uint32),
                                    C.POINTER(C.c_uint64)]),
    "csdr_hsda_load": (C.c_int, [_vp, C.c_char_p, _vp, C.POINTER(_vp)]),
    "csdr_dense_linear": (C.c_int, [_vp, C.c_int, C.c_int, _vp, C.c_int, _vp, _vp]),
    "csdr_hsdb_matmul_group_xop": (C.c_int, [C.c_int, C.POINTER(_vp), C.POINTER(_vp),
                                             C.POINTER(_vp), C.c_int, C.POINTER(_vp),
                                             C.POINTER(_vp), C.c_int, C.c_int, _vp, C.c_float,
                                             C.c_int, C.c_int, _vp, _sz, _vp]),
    "csdr_attn_decode_splits": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    "csdr_hsdr_encode": (C.c_int, [_vp, _sz, C.c_int, _vp, C.c_int, C.c_int, C.c_int, _vp, _vp,
                                   _vp]),
    "csdr_hsdr_init_dictionary": (C.c_int, [_vp, C.c_uint32, C.c_uint32, C.c_uint16,
                                            C.c_uint8, C.c_uint8, _vp]),
    "csdr_hsdr_compress_bytes": (_sz, [C.c_uint32, C.c_uint32, C.c_uint16, C.c_uint16,
                                       C.c_uint16, C.c_uint8, C.c_uint8]),
    "csdr_hsdr_compress": (C.c_int, [_vp, C.c_uint32, C.c_uint32, C.c_uint16, C.c_uint16,
                                     C.c_uint16, C.c_uint8, C.c_uint8, C.c_uint8, C.c_float,
                                     _vp, _sz, _vp]),
    "csdr_attn_decode_rope": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int,
                                        C.c_int, C.c_int, C.c_float, C.c_float, _vp, _vp, _sz,
                                        _vp]),
    "cortex_inference_engine_create": (_ce, [C.c_char_p, C.POINTER(_vp)]),
    "cortex_inference_engine_free": (_ce, [_vp]),
    "cortex_inference_engine_set_batch_size": (_ce, [_vp, _sz]),
    "cortex_inference_engine_enable_dropout": (_ce, [_vp, C.c_int]),
    "cortex_inference_engine_set_mode": (_ce, [_vp, C.c_int]),
    "cortex_inference_engine_init_memory_pool": (_ce, [_vp, _sz]),
    "cortex_inference_engine_enable_aggressive_memory": (_ce, [_vp, C.c_int]),
    "cortex_inference_engine_get_memory_usage": (_ce, [_vp, C.POINTER(_sz)]),
    "cortex_inference_engine_enable_layer_prefetch": (_ce, [_vp, C.c_int]),
    "cortex_inference_engine_get_last_run_stats_json": (_ce, [_vp, C.POINTER(C.c_void_p)]),
    "cortex_free_string": (None, [C.c_void_p]),
    "cortex_error_free": (None, [C.POINTER(CortexError)]),
    "cortex_inference_engine_run": (_ce, [_vp, _vp, _sz, _vp, _sz, C.POINTER(_sz)]),
    "cortex_inference_engine_run_layer": (_ce, [_vp, C.c_char_p, _vp, _sz, _vp, _sz,
                                                C.POINTER(_sz)]),
    "cortex_inference_engine_generate_text": (_ce, [_vp, C.c_char_p, C.c_int,
                                                    C.POINTER(C.c_void_p)]),
    "cortex_sdk_version": (C.c_char_p, []),
    "cortex_inference_engine_matmul_device": (_ce, [_vp, C.c_char_p, _vp, C.c_int, C.c_int,
                                                    _vp, _vp]),
})


class CompressionOptions(C.Structure):
    _fields_ = [
        ("num_threads", C.c_size_t), ("verbose", C.c_int), ("show_stats", C.c_int),
        ("use_delta_encoding", C.c_int), ("use_rle", C.c_int), ("compression_level", C.c_int),
        ("use_quantization", C.c_int), ("quantization_bits", C.c_int), ("use_hsdr", C.c_int),
        ("sparsity", C.c_float),
    ]


SIGNATURES["csdr_attn_decode_rope_kv"] = (C.c_int, [_vp, _vp, _vp, _vp, _vp, C.c_int, _vp, C.c_int,
                                                  C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                                                  C.c_float, _vp, _vp, _sz, _vp])
SIGNATURES["csdr_attn_decode_splits_kv"] = (C.c_int, [C.c_int] * 6)
SIGNATURES["csdr_hsdb_matmul_noalloc"] = (C.c_int, [_vp, _vp, C.c_int, C.c_int, _vp, _vp])


# the rest of the reference SDK surface (compressor family: unsupported here)
SIGNATURES.update({
    "cortex_compression_options_init": (_ce, [C.POINTER(CompressionOptions)]),
    "cortex_error_string": (C.c_char_p, [C.c_int]),
    "cortex_model_get_parts": (C.c_int, [C.c_char_p, C.POINTER(C.POINTER(C.c_void_p)),
                                         C.POINTER(C.c_int)]),
    "cortex_archive_get_tokenizer_info": (_ce, [C.c_char_p, C.POINTER(C.c_int),
                                                C.POINTER(C.c_void_p)]),
    "cortex_compressor_create": (_ce, [C.c_char_p, C.c_char_p, C.POINTER(CompressionOptions),
                                       C.POINTER(_vp)]),
    "cortex_compressor_add_file": (_ce, [_vp, C.c_char_p]),
    "cortex_compressor_compress": (_ce, [_vp, C.c_char_p]),
    "cortex_compressor_get_stats": (_ce, [_vp, C.POINTER(_sz), C.POINTER(_sz),
                                          C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "cortex_compressor_free": (_ce, [_vp]),
    "cortex_decompressor_create": (_ce, [C.c_char_p, C.POINTER(_vp), C.c_float]),
    "cortex_decompressor_decompress": (_ce, [_vp, C.c_char_p, C.c_char_p]),
    "cortex_decompressor_free": (_ce, [_vp]),
    "cortex_archive_extract": (_ce, [C.c_char_p, C.c_char_p, C.c_float]),
    "cortex_compress_from_url": (_ce, [C.c_char_p, C.c_char_p, C.c_char_p, C.c_float]),
})


class DecoderConfig(C.Structure):
    _fields_ = [
        ("n_layers", C.c_int), ("hidden", C.c_int), ("n_heads", C.c_int),
        ("n_kv_heads", C.c_int), ("head_dim", C.c_int), ("ffn", C.c_int), ("vocab", C.c_int),
        ("max_ctx", C.c_int), ("rope_theta", C.c_float), ("rms_eps", C.c_float),
        ("kv_dtype", C.c_int),
    ]


SIGNATURES["csdr_dense_linear_ex"] = (C.c_int, [_vp, C.c_int, C.c_int, _vp, C.c_int, _vp, _vp,
                                              C.c_int, _vp])
SIGNATURES["csdr_rope_kv_rows"] = (C.c_int, [_vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int,
                                           C.c_int, C.c_int, C.c_float, _vp, _vp, C.c_int,
                                           C.c_int, _vp])
SIGNATURES["csdr_attn_prefill"] = (C.c_int, [_vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int,
                                           C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, _vp,
                                           _vp])
SIGNATURES["csdr_decoder_set_prefill_chunk"] = (C.c_int, [_vp, C.c_int])
SIGNATURES["csdr_hsdb_load_host"] = (C.c_int, [_vp, _sz, _vp, C.POINTER(_vp)])
SIGNATURES["csdr_decoder_set_layer_prefetch"] = (C.c_int, [_vp, C.c_int])
SIGNATURES["csdr_decoder_streamed_bytes"] = (C.c_int64, [_vp])
SIGNATURES["csdr_hsdr_source_format"] = (C.c_int, [C.c_char_p, C.c_int])
SIGNATURES["csdr_hsdr_source_elements"] = (_sz, [C.c_int, _sz])
SIGNATURES["csdr_hsdr_source_decode"] = (C.c_int, [_vp, _sz, C.c_int, C.c_float, C.c_float, _vp,
                                                 _vp])
SIGNATURES["csdr_hsdr_compress_source"] = (C.c_int, [_vp, _sz, C.c_int, C.c_float, C.c_float,
                                                   C.c_uint32, C.c_uint32, C.c_uint16,
                                                   C.c_uint16, C.c_uint16, C.c_uint8, C.c_uint8,
                                                   C.c_uint8, C.c_float, _vp, _sz, _vp])
SIGNATURES["csdr_lazy_hsdr_load"] = (C.c_int, [_vp, _sz, C.c_int, _vp, _vp])
SIGNATURES["csdr_lazy_hsdr_free"] = (C.c_int, [_vp])
SIGNATURES["csdr_lazy_hsdr_info"] = (C.c_int, [_vp, _vp, _vp])
SIGNATURES["csdr_lazy_hsdr_decode_rows"] = (C.c_int, [_vp, _vp, C.c_int, C.c_int, _vp, _vp])
SIGNATURES["csdr_lazy_hsdr_workspace_bytes"] = (_sz, [_vp, C.c_int])
SIGNATURES["csdr_lazy_hsdr_select"] = (C.c_int, [_vp, _vp, C.c_int, _vp, C.c_float, C.c_float,
                                               _vp, _vp, _vp, _vp, _vp, _sz, _vp])
SIGNATURES["csdr_decoder_set_lazy_selection"] = (C.c_int, [_vp, _vp, C.c_float])
SIGNATURES["cortex_inference_engine_set_lazy_hsdr_selection"] = (_ce, [_vp, C.c_int])
SIGNATURES["csdr_hsda_build"] = (C.c_int, [C.c_int, _vp, _vp, _vp, _vp, _vp, C.c_uint16,
                                         C.c_uint16, C.c_uint16, C.c_uint8, C.c_uint8, C.c_uint8,
                                         C.c_float, C.c_uint32, _vp, _vp, _vp, _vp])
SIGNATURES["csdr_free_buffer"] = (None, [_vp])


def _hip_runtimes_mapped() -> set[str]:
    paths = set()
    try:
        with open("/proc/self/maps") as f:
            for line in f:
                if "libamdhip64" in line:
                    paths.add(os.path.realpath(line.split()[-1]))
    except OSError:
        pass
    return paths


def load():
    """Load the library (once). Raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"HIP library {LIB_PATH} is not built; run `python -m cortexsdr_amd.build` "
            "(there is no CPU fallback)")
    try:
        import torch  # noqa: F401  (binds torch's HIP runtime first)
    except ImportError:
        pass
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    rts = _hip_runtimes_mapped()
    if len(rts) > 1:
        raise RuntimeError(f"two HIP runtimes mapped into this process: {sorted(rts)}")
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != 0:
        msg = load().csdr_last_error()
        raise CsdrError(rc, msg.decode() if msg else "")


def exported_symbols() -> list[str]:
    return list(SIGNATURES)
