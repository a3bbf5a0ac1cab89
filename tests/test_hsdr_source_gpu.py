"""GPU parity of the compressor's source decode (csdr_hsdr_source_decode, the reference's
dequantizeSegmentToFP32, HierarchicalSDRStrategy.cpp:713-989) and of compress from a
quantized source (csdr_hsdr_compress_source), through the C-ABI.

Bars, all bit-exact: the reference's own outputs for random q4_k / q5_k / q6_k / q4_0 / q8_0
blocks (tests/golden/ref_fixtures.npz, written by the reference compiled here); the
reference's hand-computed known answers (src/test_hsdr_kquants.cpp:69-203); the oracle's
decoders on fresh random blocks; numpy for f32 / f16 / bf16 / int8; and the compressed stream
of a quantized source equal byte for byte to compressing the oracle-decoded matrix.
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def dec(gpu, blocks, fmt, **kw):
    from cortexsdr_amd.encode import source_decode

    src = gpu.from_numpy(np.ascontiguousarray(np.asarray(blocks, np.uint8).ravel())).cuda()
    return source_decode(src, fmt, **kw).cpu().numpy()


@pytest.mark.parametrize("key,fmt", [("q4k", "q4_k"), ("q5k", "q5_k"), ("q6k", "q6_k"),
                                     ("q40", "q4_0"), ("q80", "q8_0")])
def test_reference_outputs_bitexact(gpu, golden, key, fmt):
    out = dec(gpu, golden[f"{key}_blocks"], fmt)
    assert np.array_equal(bits(out), bits(golden[f"{key}_ref"]))


def _f16(v):
    return np.array([np.float16(v).view(np.uint16)], "<u2").view(np.uint8)


def test_known_answers(gpu):
    # src/test_hsdr_kquants.cpp:69-95 and :106-122 (Q4_K)
    b = np.zeros(144, np.uint8)
    b[0:2], b[2:4] = _f16(1.0), _f16(0.0)
    b[4], b[8], b[16], b[17] = 0x01, 0x00, 0x21, 0x43
    out = dec(gpu, b, "q4_k")
    assert list(out[:4]) == [1.0, 2.0, 3.0, 4.0] and not out[4:].any()
    b = np.zeros(144, np.uint8)
    b[0:2], b[2:4] = _f16(2.0), _f16(1.0)
    b[4], b[8], b[16] = 3, 4, 0x05
    out = dec(gpu, b, "q4_k")
    assert out[0] == 26.0 and out[1] == -4.0
    # :133-150 (Q5_K) -> 18, 0
    b = np.zeros(176, np.uint8)
    b[0:2], b[2:4] = _f16(1.0), _f16(0.0)
    b[4], b[16], b[48] = 1, 0x01, 0x02
    out = dec(gpu, b, "q5_k")
    assert out[0] == 18.0 and out[1] == 0.0
    # :162-178 and :188-203 (Q6_K) -> -62, -60 and 34, -60
    for qh, e0 in ((0x00, -62.0), (0x03, 34.0)):
        b = np.zeros(210, np.uint8)
        b[0], b[128], b[192] = 0x21, qh, 2
        b[208:210] = _f16(1.0)
        out = dec(gpu, b, "q6_k")
        assert out[0] == e0 and out[1] == -60.0


def _random_kblocks(rng, nblk, nbytes, scale_offsets):
    b = rng.integers(0, 256, (nblk, nbytes), dtype=np.uint8)
    for off in scale_offsets:  # finite fp16 scales of moderate size
        b[:, off:off + 2] = rng.uniform(-2, 2, nblk).astype(np.float16).view(np.uint8).reshape(
            nblk, 2)
    return b


def test_random_blocks_against_oracle(gpu):
    rng = np.random.default_rng(11)
    b = _random_kblocks(rng, 37, 144, [0, 2])
    assert np.array_equal(bits(dec(gpu, b, "q4_k")),
                          bits(oracle.q4k_dequant(b.ravel(), oracle.ORC_Q4K_INTERLEAVED)))
    b = _random_kblocks(rng, 29, 176, [0, 2])
    assert np.array_equal(bits(dec(gpu, b, "q5_k")), bits(oracle.q5k_dequant(b.ravel())))
    b = _random_kblocks(rng, 31, 210, [208])
    assert np.array_equal(bits(dec(gpu, b, "q6_k")), bits(oracle.q6k_dequant(b.ravel())))


def test_plain_formats(gpu):
    rng = np.random.default_rng(3)
    w = rng.standard_normal(1000).astype(np.float32)
    assert np.array_equal(bits(dec(gpu, w.view(np.uint8), "f32")), bits(w))
    h = w.astype(np.float16)
    assert np.array_equal(bits(dec(gpu, h.view(np.uint8), "f16")), bits(h.astype(np.float32)))
    bf = (w.view(np.uint32) >> 16).astype(np.uint16)
    want = (bf.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(bits(dec(gpu, bf.view(np.uint8), "bf16")), bits(want))
    q = rng.integers(-128, 128, 777).astype(np.int8)
    got = dec(gpu, q.view(np.uint8), "i8", scale=0.037, zero_point=3.5)
    want = (q.astype(np.float32) - np.float32(3.5)) * np.float32(0.037)
    assert np.array_equal(bits(got), bits(want))


def test_compress_from_quantized_source(gpu):
    from cortexsdr_amd.encode import compress, compress_source

    rng = np.random.default_rng(21)
    rows, cols = 96, 256          # one q6_k / q5_k super-block per row, 1-row tiles
    for fmt, nbytes, offs, fn in (("q6_k", 210, [208], oracle.q6k_dequant),
                                  ("q5_k", 176, [0, 2], oracle.q5k_dequant)):
        b = _random_kblocks(rng, rows, nbytes, offs)
        w = fn(b.ravel()).reshape(rows, cols)
        src = gpu.from_numpy(b.ravel().copy()).cuda()
        got = compress_source(src, fmt, rows, cols, 1, cols, 16, 2, 2)
        want = compress(w, 1, cols, 16, 2, 2)
        assert got == want, fmt


def test_source_errors(gpu):
    from cortexsdr_amd import _lib
    from cortexsdr_amd._lib import CsdrError

    lib = _lib.load()
    buf = gpu.zeros(4096, dtype=gpu.uint8, device="cuda")
    out = gpu.zeros(4096, dtype=gpu.float32, device="cuda")
    st = gpu.cuda.current_stream().cuda_stream
    with pytest.raises(CsdrError):   # not a whole number of 210-byte blocks
        _lib.check(lib.csdr_hsdr_source_decode(buf.data_ptr(), 211, 8, 1.0, 0.0,
                                               out.data_ptr(), st))
    with pytest.raises(CsdrError):   # unknown format
        _lib.check(lib.csdr_hsdr_source_decode(buf.data_ptr(), 64, 42, 1.0, 0.0,
                                               out.data_ptr(), st))
    with pytest.raises(CsdrError):   # decoded count does not match rows x cols
        _lib.check(lib.csdr_hsdr_compress_source(buf.data_ptr(), 210, 8, 1.0, 0.0, 2, 256, 1,
                                                 256, 1, 1, 1, 0, 0.5, out.data_ptr(), 4096, st))
