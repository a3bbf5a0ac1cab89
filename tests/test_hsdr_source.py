"""Host side of the compressor's source decode (no GPU): format dispatch as
dequantizeSegmentToFP32 (HierarchicalSDRStrategy.cpp:713-989) orders it, data_format name
first (case-insensitive), then the f32 / f16 / int8 segment types, and the decoded value
counts per block size."""
import ctypes as C

from cortexsdr_amd import _lib

F32, F16, BF16, I8, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = range(9)
WEIGHTS_FP32, WEIGHTS_FP16, WEIGHTS_INT8 = 1, 2, 3


def test_format_dispatch():
    lib = _lib.load()
    fmt = lambda name, t=0: lib.csdr_hsdr_source_format(name.encode() if name is not None
                                                          else None, t)
    assert fmt("BF16") == BF16 and fmt("bfloat16", WEIGHTS_FP16) == BF16  # name before type
    assert fmt("q4_0", WEIGHTS_INT8) == Q4_0 and fmt("Q8_0", WEIGHTS_INT8) == Q8_0
    assert (fmt("q4_k"), fmt("Q5_K"), fmt("q6_k")) == (Q4_K, Q5_K, Q6_K)
    assert fmt("", WEIGHTS_FP32) == F32 and fmt("float32") == F32
    assert fmt("half") == F16 and fmt(None, WEIGHTS_FP16) == F16
    assert fmt("int8") == I8 and fmt("", WEIGHTS_INT8) == I8
    assert fmt("q8_k") == -1 and fmt("", 0) == -1


def test_element_counts():
    lib = _lib.load()
    n = lambda f, b: lib.csdr_hsdr_source_elements(f, C.c_size_t(b))
    assert (n(Q4_K, 144 * 3), n(Q5_K, 176), n(Q6_K, 210 * 2)) == (768, 256, 512)
    assert (n(Q4_0, 18 * 5), n(Q8_0, 34)) == (160, 32)
    assert (n(F32, 40), n(F16, 40), n(BF16, 6), n(I8, 7)) == (10, 20, 3, 7)
    assert n(Q6_K, 211) == 0 and n(F32, 6) == 0 and n(99, 64) == 0
