"""GPU parity of the HSDR/HSDB path (HK1 gather GEMV, HK3 1-row HSDR, HK4 dense decode)
against the CPU oracle and the reference's golden fixtures, through the C-ABI.

Bar: relative L2 <= 1e-3 at fp32 accumulation for products; bit-exact for decoded
weights, decoded indices/signs/coefficients and block layout.
"""
import functools

import numpy as np
import pytest

import oracle
from conftest import rel_l2
from cortexsdr_amd import formats, synth

pytestmark = pytest.mark.gpu
TOL = 1e-3


@functools.lru_cache(maxsize=None)
def layer(R, Cc, K, s, seed=2):
    return synth.hsdb_layer(R, Cc, K, s, seed_dict=1, seed_codes=seed)


def seg_of(stream):
    from cortexsdr_amd.hsdr import HsdbSegment

    return HsdbSegment(stream)


def run(gpu, stream, x_np, dtype):
    seg = seg_of(stream)
    xd = gpu.from_numpy(np.ascontiguousarray(x_np.astype(dtype))).cuda()
    y = seg.matmul(xd)
    gpu.cuda.synchronize()
    return seg, y.cpu().numpy()


@pytest.mark.parametrize("R,Cc,K,s,dtype", [
    (4096, 4096, 512, 4, np.float32),     # config 1
    (4096, 11008, 1024, 8, np.float16),   # config 2, W 4096 x 11008
    (11008, 4096, 1024, 8, np.float16),   # config 2, W 11008 x 4096
])
def test_gemv_configs(gpu, R, Cc, K, s, dtype):
    stream = layer(R, Cc, K, s)
    x = synth.activations(Cc, 1, seed=3, dtype=dtype)
    seg, y = run(gpu, stream, x, dtype)
    ref = oracle.hsdb_matmul(stream, x.astype(np.float32))
    err = rel_l2(y, ref)
    print(f"R={R} C={Cc} K={K} s={s} rel_l2={err:.3e}")
    assert err <= TOL
    # repeatable: row partials are accumulated with float atomics, so calls agree to
    # rounding
    xd = gpu.from_numpy(np.ascontiguousarray(x)).cuda()
    ws = seg.workspace(1)
    y2 = seg.matmul(xd, workspace=ws).cpu().numpy()
    assert rel_l2(y2, y) <= 1e-6


@pytest.mark.parametrize("M", [2, 4, 7, 16])
def test_batched_small(gpu, M):
    stream = layer(1024, 2048, 1024, 8)
    x = synth.activations(2048, M, seed=5, dtype=np.float16)
    _, y = run(gpu, stream, x, np.float16)
    ref = oracle.hsdb_matmul(stream, x.astype(np.float32))
    assert rel_l2(y, ref) <= TOL


@pytest.mark.parametrize("R,Cc,K,s,M", [
    (37, 200, 64, 5, 1),     # ragged rows, edge strip of 8 columns, generic slot count
    (37, 200, 60, 5, 3),     # K not a multiple of 4
    (300, 64, 32, 8, 1),     # a single block column
    (513, 1000, 128, 3, 2),  # odd everything
    (64, 4096, 2048, 12, 1),
])
def test_ragged(gpu, R, Cc, K, s, M):
    stream = synth.hsdb_layer(R, Cc, K, s, seed_dict=3, seed_codes=4)
    x = synth.activations(Cc, M, seed=6)
    _, y = run(gpu, stream, x, np.float32)
    ref = oracle.hsdb_matmul(stream, x)
    assert rel_l2(y, ref) <= TOL


@pytest.mark.parametrize("key", ["hsdr1d", "hsdr1de"])
def test_reference_hsdr_streams_matmul(gpu, golden, key):
    # strategy-5 payloads written by the reference compressor, run unchanged (HK3)
    stream = golden[f"{key}_stream"].tobytes()
    x = golden[f"{key}_x"]
    _, y = run(gpu, stream, x, np.float32)
    assert rel_l2(y, golden[f"{key}_y"]) <= 1e-5
    # and the HSDB form of the same stream gives the same product
    _, yb = run(gpu, formats.hsdr_to_hsdb(stream), x, np.float32)
    assert rel_l2(yb, golden[f"{key}_y"]) <= 1e-5


@pytest.mark.parametrize("key", ["hsdr1d", "hsdr1de", "hsdr2d", "hsdr2db"])
def test_reference_hsdr_decompress_bitexact(gpu, golden, key):
    seg = seg_of(golden[f"{key}_stream"].tobytes())
    w = seg.decompress().cpu().numpy()
    assert np.array_equal(w.view(np.uint32), golden[f"{key}_w"].view(np.uint32))


def test_hsdb_decompress_and_codes_bitexact(gpu):
    stream = synth.hsdb_layer(96, 456, 256, 8, seed_dict=5, seed_codes=6)
    seg = seg_of(stream)
    w = seg.decompress().cpu().numpy()
    assert np.array_equal(w.view(np.uint32), oracle.hsdr_decompress(stream).view(np.uint32))
    packed, mag = seg.export_codes()
    idx, sign, mag_s, _ = formats.hsdb_unpack(stream)
    assert np.array_equal(packed & 0x7FFF, idx)
    assert np.array_equal(packed >> 15, sign)
    assert np.array_equal(mag, mag_s)


def test_config2_codes_layout_bitexact(gpu):
    stream = layer(4096, 11008, 1024, 8)
    packed, mag = seg_of(stream).export_codes()
    idx, sign, mag_s, _ = formats.hsdb_unpack(stream)
    assert np.array_equal(packed, (idx | (sign << 15)).astype(np.uint16))
    assert np.array_equal(mag, mag_s)


def test_workspace_reuse_across_batch_sizes(gpu):
    stream = layer(1024, 2048, 1024, 8)
    seg = seg_of(stream)
    ws = gpu.zeros(seg.workspace_bytes(16), dtype=gpu.uint8, device="cuda")
    outs = {}
    for M in (1, 16, 1, 5, 1):
        x = synth.activations(2048, M, seed=7 + M, dtype=np.float16)
        xd = gpu.from_numpy(x).cuda()
        y = seg.matmul(xd, workspace=ws).cpu().numpy()
        assert rel_l2(y, oracle.hsdb_matmul(stream, x.astype(np.float32))) <= TOL
        if M in outs:
            assert rel_l2(y, outs[M]) <= 1e-6
        outs[M] = y
    assert not ws[:24].cpu().numpy().any()


@pytest.mark.parametrize("M", [1, 3])
def test_group_launch(gpu, M):
    from cortexsdr_amd.hsdr import matmul_group

    shapes = [(4096, 11008, 1024, 8), (11008, 4096, 1024, 8), (896, 896, 1024, 8),
              (128, 896, 1024, 8)]
    segs = [seg_of(layer(*sh)) for sh in shapes]
    xs = [synth.activations(sh[1], M, seed=20 + i, dtype=np.float16)
          for i, sh in enumerate(shapes)]
    ys = matmul_group(segs, [gpu.from_numpy(x).cuda() for x in xs])
    for sh, x, y in zip(shapes, xs, ys):
        ref = oracle.hsdb_matmul(layer(*sh), x.astype(np.float32))
        assert rel_l2(y.cpu().numpy(), ref) <= TOL


def test_errors_are_reported(gpu, golden):
    from cortexsdr_amd.hsdr import CompressionError

    good = layer(64, 128, 32, 4)
    with pytest.raises(CompressionError) as e:
        seg_of(b"XXXX" + good[4:])
    assert e.value.code == -2
    with pytest.raises(CompressionError) as e:
        seg_of(good[:-10])
    assert e.value.code == -3
    bad = bytearray(good)
    off = 36 + 4 + 32 * 64 * 4  # first packed code
    bad[off:off + 2] = np.array([40], "<u2").tobytes()  # index 40 >= K = 32
    with pytest.raises(CompressionError) as e:
        seg_of(bytes(bad))
    assert e.value.code == -2
    # 2-D tiles: the fused matmul refuses them, as matmulRowMajor does (:1273-1276)
    seg2d = seg_of(golden["hsdr2d_stream"].tobytes())
    x = gpu.zeros((100, 1), dtype=gpu.float32, device="cuda")
    with pytest.raises(CompressionError) as e:
        seg2d.matmul(x)
    assert e.value.code == -2


@pytest.mark.parametrize("share", ["1", "0"])
def test_shared_dictionary_lifetime(gpu, monkeypatch, share):
    """Segments with the same dictionary bytes share one device copy (CSDR_HSDB_SHARE_DICT,
    default on): a segment keeps working after another user of its dictionary is freed, and
    segments with another dictionary are unaffected (M = 1 fp32 path and the fp16 batched
    path, which reads the fp16 copy)."""
    from cortexsdr_amd.hsdr import HsdbSegment

    monkeypatch.setenv("CSDR_HSDB_SHARE_DICT", share)
    st = {k: synth.hsdb_layer(96, 256, 64, 8, seed_dict=sd, seed_codes=sc)
          for k, (sd, sc) in {"a": (1, 2), "b": (1, 3), "c": (4, 5), "d": (1, 6)}.items()}
    segs = {k: HsdbSegment(v) for k, v in st.items() if k != "d"}

    def check(k, seg):
        for M in (1, 16):
            x = synth.activations(256, M, seed=ord(k) + M)
            y = seg.matmul(gpu.from_numpy(x).cuda()).cpu().numpy()
            assert rel_l2(y, oracle.hsdb_matmul(st[k], x)) < 1e-3, (k, M)

    segs["a"].free()
    check("b", segs["b"])
    check("c", segs["c"])
    segs["d"] = HsdbSegment(st["d"])
    segs["b"].free()
    check("d", segs["d"])
    check("c", segs["c"])
    segs["d"].free()
    segs["c"].free()


@pytest.mark.parametrize("dtype,shift", [(np.float16, 1), (np.float16, 3), (np.float32, 1),
                                         (np.float32, 2)])
def test_gemv_misaligned_x(gpu, dtype, shift):
    """M = 1 with 64-long blocks and an x that is not 16-byte aligned: the product takes the
    general dx kernel (the matrix-core one loads x as 16-byte pieces), with the same result."""
    torch = gpu
    R, Cc, K, s = 1024, 4096, 1024, 8
    stream = layer(R, Cc, K, s)
    x = synth.activations(Cc, 1, seed=9, dtype=dtype)
    buf = torch.zeros(Cc + 8, dtype=torch.float16 if dtype == np.float16 else torch.float32,
                      device="cuda")
    xd = buf[shift:shift + Cc].view(Cc, 1)
    xd.copy_(torch.from_numpy(np.ascontiguousarray(x)))
    assert xd.data_ptr() % 16 != 0
    seg = seg_of(stream)
    try:
        y = seg.matmul(xd).cpu().numpy()
        ref = oracle.hsdb_matmul(stream, x.astype(np.float32))
        assert rel_l2(y, ref) <= 1e-5
        # the aligned product agrees
        xa = torch.from_numpy(np.ascontiguousarray(x)).cuda()
        ya = seg.matmul(xa).cpu().numpy()
        assert rel_l2(y, ya) <= 1e-6
    finally:
        seg.free()
