"""GPU parity of the engine's GGUF block formats (csdr_gguf_dequant / csdr_gguf_linear, the
device form of SparseInferenceEngine.cpp decodeSupportedGGUFQuantized + linear_forward)
against the oracle (pinned in test_gguf_oracle.py), through the C-ABI.

Bars: dequant bit-exact; the products within 1e-3 relative L2 at M > 1 (the decoded values
rounded to fp16 once for the matrix cores, ~2e-4) and 1e-5 at M == 1 (exact decoded values and
products, fp32 accumulation).
"""
import numpy as np
import pytest

import oracle
from conftest import rel_l2

pytestmark = pytest.mark.gpu
F = oracle.GGUF_FORMATS
TOL = 1e-3
TOL_M1 = 1e-5   # M == 1: exact decoded values and products, fp32 accumulation


def blocks(fmt, n, rng, random_scale=False):
    """n random blocks of a format with finite, modest fp16 (or fp32) scales."""
    bb, _ = oracle.gguf_block(F[fmt])
    b = rng.integers(0, 256, (n, bb), dtype=np.uint8)
    if random_scale:
        return b   # the generic rule's scale sanitising is exercised too

    def put16(off):
        v = (rng.uniform(0.002, 0.03, n) * rng.choice([-1, 1], n)).astype(np.float16)
        b[:, off:off + 2] = v.view(np.uint8).reshape(n, 2)
    if fmt == "q8_1":
        b[:, 0:4] = rng.uniform(0.002, 0.03, n).astype("<f4").view(np.uint8).reshape(n, 4)
    elif fmt == "q6_k":
        put16(208)
    elif fmt in ("q4_1", "q5_1", "q4_k"):
        put16(0)
        put16(2)
    else:
        put16(0)
    return b


FORMATS = ["q4_0", "q4_1", "q5_0", "q5_1", "q8_0", "q8_1", "q8_k", "q6_k", "q4_k", "q2_k",
           "q3_k", "q5_k", "iq4_xs", "iq1_m", "q4_0_4_4"]


def _dev(gpu, a):
    return gpu.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("fmt", FORMATS)
def test_dequant_bitexact(gpu, fmt):
    from cortexsdr_amd import gguf

    rng = np.random.default_rng(F[fmt])
    for random_scale in (False, True):
        b = blocks(fmt, 37, rng, random_scale and fmt in ("q2_k", "q3_k", "q5_k", "iq4_xs",
                                                          "iq1_m", "q4_0_4_4"))
        want = oracle.gguf_dequant(b.ravel(), F[fmt])
        got = gguf.dequant(_dev(gpu, b.ravel()), F[fmt], b.shape[0]).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), fmt


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("R,nblk", [(37, 3), (256, 8)])
def test_linear_m1(gpu, fmt, R, nblk):
    from cortexsdr_amd import gguf

    rng = np.random.default_rng(100 + F[fmt])
    _, be = oracle.gguf_block(F[fmt])
    Cc = nblk * be
    w = blocks(fmt, R * nblk, rng)
    wd = _dev(gpu, w.ravel())
    x = rng.normal(size=(1, Cc)).astype(np.float32)
    ref = oracle.gguf_linear(w.ravel(), F[fmt], R, Cc, x)
    y = gguf.linear(wd, F[fmt], R, Cc, _dev(gpu, x)).cpu().numpy()
    xh = x.astype(np.float16)
    ref_h = oracle.gguf_linear(w.ravel(), F[fmt], R, Cc, xh.astype(np.float32))
    yh = gguf.linear(wd, F[fmt], R, Cc, _dev(gpu, xh)).cpu().numpy()
    print(f"{fmt} R={R} C={Cc}: rel_l2 {rel_l2(y, ref):.2e} (fp32 x), {rel_l2(yh, ref_h):.2e} "
          f"(fp16 x)", flush=True)
    assert rel_l2(y, ref) <= TOL_M1
    assert rel_l2(yh, ref_h) <= TOL_M1


@pytest.mark.parametrize("fmt,R,Cc", [("q6_k", 4100, 14336), ("q4_0", 9001, 4096),
                                      ("q8_0", 8500, 4096), ("q5_k", 8500, 8448),
                                      ("q8_0", 1031, 14336)])
def test_linear_m1_many_rows(gpu, fmt, R, Cc):
    """More rows than the chip holds at once (several rounds of workgroups), ragged counts."""
    from cortexsdr_amd import gguf

    rng = np.random.default_rng(400 + F[fmt])
    _, be = oracle.gguf_block(F[fmt])
    w = blocks(fmt, R * Cc // be, rng)
    wd = _dev(gpu, w.ravel())
    x = rng.normal(size=(1, Cc)).astype(np.float16)
    ref = oracle.gguf_linear(w.ravel(), F[fmt], R, Cc, x.astype(np.float32))
    y = gguf.linear(wd, F[fmt], R, Cc, _dev(gpu, x)).cpu().numpy()
    err = rel_l2(y, ref)
    print(f"{fmt} R={R} C={Cc} float16: rel_l2={err:.2e}", flush=True)
    assert err <= TOL_M1


@pytest.mark.parametrize("fmt", ["q4_0", "q4_1", "q6_k", "q5_k", "q2_k", "iq4_xs", "q8_0", "q8_k"])
def test_linear_m1_unaligned_x(gpu, fmt):
    """x not 16-byte aligned (one element into a buffer): the element-wise x reads."""
    from cortexsdr_amd import gguf

    rng = np.random.default_rng(200 + F[fmt])
    _, be = oracle.gguf_block(F[fmt])
    R, Cc = 45, 4 * 256
    w = blocks(fmt, R * Cc // be, rng)
    wd = _dev(gpu, w.ravel())
    for dt in (np.float32, np.float16):
        buf = rng.normal(size=(1, Cc + 1)).astype(dt)
        ref = oracle.gguf_linear(w.ravel(), F[fmt], R, Cc, buf[:, 1:].astype(np.float32))
        y = gguf.linear(wd, F[fmt], R, Cc, _dev(gpu, buf)[:, 1:]).cpu().numpy()
        assert rel_l2(y, ref) <= TOL_M1, np.dtype(dt).name


@pytest.mark.parametrize("fmt", ["q8_0", "q5_k"])
def test_linear_m1_pipelined_unaligned_x(gpu, fmt):
    """Rows of 8192 values and more in q8_0 / q5_k take the pipelined kernel (x staged in LDS):
    x one element into its buffer (the element-wise staging), a row count that leaves the last
    workgroup short, items that straddle 16-byte boundaries."""
    from cortexsdr_amd import gguf

    rng = np.random.default_rng(500 + F[fmt])
    _, be = oracle.gguf_block(F[fmt])
    R, Cc = 517, 8448
    w = blocks(fmt, R * Cc // be, rng)
    wd = _dev(gpu, w.ravel())
    for dt in (np.float32, np.float16):
        buf = rng.normal(size=(1, Cc + 1)).astype(dt)
        ref = oracle.gguf_linear(w.ravel(), F[fmt], R, Cc, buf[:, 1:].astype(np.float32))
        y = gguf.linear(wd, F[fmt], R, Cc, _dev(gpu, buf)[:, 1:]).cpu().numpy()
        err = rel_l2(y, ref)
        print(f"{fmt} R={R} C={Cc} {np.dtype(dt).name} unaligned: rel_l2={err:.2e}", flush=True)
        assert err <= TOL_M1


@pytest.mark.parametrize("fmt,R,Cc", [
    ("q6_k", 64, 24576),   # 20160-byte rows: two batches of row loads, over 64 KiB of LDS
    ("q4_0", 40, 4128),    # 2322-byte rows: rows start off 16-byte boundaries
    ("q8_0", 48, 14336),
    ("q5_k", 33, 14336),
])
def test_linear_m1_long_rows(gpu, fmt, R, Cc):
    from cortexsdr_amd import gguf

    rng = np.random.default_rng(300 + F[fmt])
    _, be = oracle.gguf_block(F[fmt])
    w = blocks(fmt, R * Cc // be, rng)
    wd = _dev(gpu, w.ravel())
    for dt in (np.float32, np.float16):
        x = rng.normal(size=(1, Cc)).astype(dt)
        ref = oracle.gguf_linear(w.ravel(), F[fmt], R, Cc, x.astype(np.float32))
        y = gguf.linear(wd, F[fmt], R, Cc, _dev(gpu, x)).cpu().numpy()
        err = rel_l2(y, ref)
        print(f"{fmt} R={R} C={Cc} {np.dtype(dt).name}: rel_l2={err:.2e}", flush=True)
        assert err <= TOL


@pytest.mark.parametrize("fmt", ["q4_0", "q5_1", "q8_0", "q6_k", "q4_k", "q3_k"])
@pytest.mark.parametrize("M", [3, 17, 64])
def test_linear_batched(gpu, fmt, M):
    from cortexsdr_amd import gguf

    rng = np.random.default_rng(200 + F[fmt] + M)
    _, be = oracle.gguf_block(F[fmt])
    R, Cc = 70, 4 * max(be, 64)
    w = blocks(fmt, R * Cc // be, rng)
    x = rng.normal(size=(M, Cc)).astype(np.float16)
    ref = oracle.gguf_linear(w.ravel(), F[fmt], R, Cc, x.astype(np.float32))
    y = gguf.linear(_dev(gpu, w.ravel()), F[fmt], R, Cc, _dev(gpu, x)).cpu().numpy()
    err = rel_l2(y, ref)
    print(f"{fmt} M={M}: rel_l2={err:.2e}", flush=True)
    assert err <= TOL


@pytest.mark.parametrize("fmt,R,nsteps,M", [
    ("q4_0", 300, 40, 32),    # 40 steps in 4 splits of 10 (one per pair of XCDs)
    ("q6_k", 96, 72, 70),     # 8 splits of 9, two column groups, padded row tiles
    ("q8_0", 1000, 12, 5),    # short rows: 4 splits of 3
    ("q4_k", 130, 33, 17),    # 33 steps in 4 splits of 9 (the last holds 6)
])
def test_linear_batched_split_k(gpu, fmt, R, nsteps, M):
    from cortexsdr_amd import gguf

    rng = np.random.default_rng(300 + F[fmt] + M)
    _, be = oracle.gguf_block(F[fmt])
    Cc = 256 * nsteps
    w = blocks(fmt, R * Cc // be, rng)
    x = rng.normal(size=(M, Cc)).astype(np.float16)
    ref = oracle.gguf_linear(w.ravel(), F[fmt], R, Cc, x.astype(np.float32))
    y = gguf.linear(_dev(gpu, w.ravel()), F[fmt], R, Cc, _dev(gpu, x)).cpu().numpy()
    err = rel_l2(y, ref)
    print(f"{fmt} R={R} C={Cc} M={M}: rel_l2={err:.2e}", flush=True)
    assert err <= TOL


def test_rejects_bad_use(gpu):
    from cortexsdr_amd import _lib, gguf

    lib = _lib.load()
    assert lib.csdr_gguf_format(b"Q6_K") == F["q6_k"]
    assert lib.csdr_gguf_format(b"bf16") == -1
    with pytest.raises(ValueError):
        gguf.format_id("f16")
    rng = np.random.default_rng(1)
    w = _dev(gpu, blocks("q8_0", 4, rng).ravel())
    x = _dev(gpu, np.zeros((1, 100), np.float32))
    with pytest.raises(_lib.CsdrError):
        gguf.linear(w, F["q8_0"], 1, 100, x)    # C not a multiple of 32
    with pytest.raises(_lib.CsdrError):
        gguf.linear(w, 99, 1, 128, _dev(gpu, np.zeros((1, 128), np.float32)))
    with pytest.raises(_lib.CsdrError):          # M > 1 takes fp16 x
        gguf.linear(w, F["q8_0"], 1, 64, _dev(gpu, np.zeros((2, 64), np.float32)))
