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
    "csdr_hsdb_matmul_group_ex": (C.c_int, [C.c_int, C.POINTER(_vp), C.POINTER(_vp), C.c_int,
                                            C.c_int, C.POINTER(_vp), C.POINTER(_vp), C.c_int,
                                            _vp, _sz, _vp]),
    "csdr_hsdb_decode_row": (C.c_int, [_vp, _vp, C.c_int, _vp, _vp]),
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
                                        C.c_int, _vp, C.POINTER(C.c_int)]),
    "csdr_decoder_logits": (C.c_int, [_vp, _vp]),
    "csdr_decoder_position": (C.c_int, [_vp]),
}


class DecoderConfig(C.Structure):
    _fields_ = [
        ("n_layers", C.c_int), ("hidden", C.c_int), ("n_heads", C.c_int),
        ("n_kv_heads", C.c_int), ("head_dim", C.c_int), ("ffn", C.c_int), ("vocab", C.c_int),
        ("max_ctx", C.c_int), ("rope_theta", C.c_float), ("rms_eps", C.c_float),
    ]


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
