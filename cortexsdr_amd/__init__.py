"""cortexsdr_amd -- MI355X-native (gfx950 HIP) compressed-weight inference path of cortexSDR.

The compute lives in libcortexsdr_amd.so (hand-written HIP kernels behind the C-ABI of
include/cortexsdr_hip.h). This package holds the host-side mirror of the reference's
operator interface (hsdr.HsdbSegment, hsdr.matmul_row_major), the stream formats
(formats) and the seeded synthetic workloads (synth).
"""
from . import formats, synth  # noqa: F401

__version__ = "0.1.0"


def library_path() -> str:
    from . import _lib

    return _lib.LIB_PATH
