"""GPU parity of the batched (M >= 9) HSDB product on matrix cores against the CPU oracle's
fp32 fused product, through the C-ABI. Two kernels serve it: decoded 64-column weight tiles
times X (v_mfma_f32_16x16x32_f16, fp32 accumulation), and at M <= 16 with fp16 X and 4 or 8
slots the dictionary route (Q_b = D . X_b per 256-row strip and block column on the matrix
cores, stored in fp16, each row's slots gathered from it with fp32 multiply-adds).

Bar: relative L2 <= 1e-3 (the path's tolerance at fp32 accumulation). The kernels round the
dictionary to fp16 once, and each decoded weight (decoding kernel) or each Q value
(dictionary route) to fp16 (fp32 X is split into fp16 hi + lo), which puts them near 2e-4;
the printed errors show the margin."""
import ctypes as C
import functools
import os

import numpy as np
import pytest

import oracle
from conftest import rel_l2
from cortexsdr_amd import synth

pytestmark = pytest.mark.gpu
TOL = 1e-3


@functools.lru_cache(maxsize=None)
def layer(R, Cc, K, s, seed=2):
    return synth.hsdb_layer(R, Cc, K, s, seed_dict=1, seed_codes=seed)


def product(gpu, stream, x, dtype):
    from cortexsdr_amd.hsdr import HsdbSegment

    seg = HsdbSegment(stream)
    xd = gpu.from_numpy(np.ascontiguousarray(x.astype(dtype))).cuda()
    y = seg.matmul(xd).cpu().numpy()
    seg.free()
    return y


@pytest.mark.parametrize("R,Cc,M", [
    (4096, 11008, 16),   # config 2a
    (11008, 4096, 64),   # config 2b
    (4096, 11008, 256),
])
def test_config2_batched(gpu, R, Cc, M):
    stream = layer(R, Cc, 1024, 8)
    x = synth.activations(Cc, M, seed=3, dtype=np.float16)
    y = product(gpu, stream, x, np.float16)
    ref = oracle.hsdb_matmul(stream, x.astype(np.float32))
    err = rel_l2(y, ref)
    print(f"R={R} C={Cc} M={M} rel_l2={err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("R,Cc,K,s,M,dtype", [
    (300, 200, 64, 8, 17, np.float32),     # ragged rows, edge strip, fp32 X (hi/lo split)
    (129, 640, 1024, 4, 40, np.float16),   # one row past a 128-row strip
    (1000, 4096, 512, 16, 256, np.float32),  # fp32 X at M = 256: two 128-column tiles
    (64, 64, 32, 8, 16, np.float16),       # one block column, one strip
    (2048, 1024, 1024, 8, 100, np.float16),  # M not a multiple of 16
])
def test_batched_shapes(gpu, R, Cc, K, s, M, dtype):
    stream = synth.hsdb_layer(R, Cc, K, s, seed_dict=5, seed_codes=6)
    x = synth.activations(Cc, M, seed=7, dtype=dtype)
    y = product(gpu, stream, x, dtype)
    ref = oracle.hsdb_matmul(stream, x.astype(np.float32))
    err = rel_l2(y, ref)
    print(f"R={R} C={Cc} K={K} s={s} M={M} {np.dtype(dtype).name} rel_l2={err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("R,Cc,K,s,M", [
    (300, 896, 1024, 8, 9),      # ragged strip, a remainder chunk (14 block columns)
    (1000, 896, 256, 4, 16),     # 4 slots, a quarter of the waves holding atoms
    (513, 704, 1024, 8, 13),     # one row past two 256-row strips, 11 block columns
    (4096, 1024, 1024, 16, 16),  # 16 slots (the weight-decoding kernel)
])
def test_dictionary_route_shapes(gpu, R, Cc, K, s, M):
    # M <= 16 with fp16 X: Q_b = D . X_b per unit on the matrix cores, rows gathered from LDS
    stream = synth.hsdb_layer(R, Cc, K, s, seed_dict=12, seed_codes=13)
    x = synth.activations(Cc, M, seed=14, dtype=np.float16)
    y = product(gpu, stream, x, np.float16)
    ref = oracle.hsdb_matmul(stream, x.astype(np.float32))
    err = rel_l2(y, ref)
    print(f"R={R} C={Cc} K={K} s={s} M={M} rel_l2={err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("M", [12, 16])
def test_group_mixed_dictionaries(gpu, M):
    # matrices of different K, R and C in one call: workgroup unit ranges cross matrix
    # segments, and the dictionary route reloads its atoms per segment
    from cortexsdr_amd import _lib
    from cortexsdr_amd.hsdr import HsdbSegment, group_workspace

    shapes = [(300, 896, 256), (1000, 1024, 1024), (513, 640, 512)]
    streams = [synth.hsdb_layer(R, Cc, K, 8, seed_dict=30 + i, seed_codes=40 + i)
               for i, (R, Cc, K) in enumerate(shapes)]
    segs = [HsdbSegment(st) for st in streams]
    xs = [synth.activations(Cc, M, seed=50 + i, dtype=np.float16)
          for i, (_, Cc, _) in enumerate(shapes)]
    xd = [gpu.from_numpy(x).cuda() for x in xs]
    ys = [gpu.zeros((R, M), dtype=gpu.float32, device="cuda") for R, _, _ in shapes]
    ws = group_workspace(segs, M)
    n = len(segs)
    hs = (C.c_void_p * n)(*[sg._h.value for sg in segs])
    xp = (C.c_void_p * n)(*[x.data_ptr() for x in xd])
    yp = (C.c_void_p * n)(*[y.data_ptr() for y in ys])
    lib = _lib.load()
    sp = int(gpu.cuda.current_stream().cuda_stream)
    _lib.check(lib.csdr_hsdb_matmul_group_ex(n, hs, xp, 1, M, yp, None, 0, ws.data_ptr(),
                                             ws.numel(), sp))
    for st, x, y in zip(streams, xs, ys):
        err = rel_l2(y.cpu().numpy(), oracle.hsdb_matmul(st, x.astype(np.float32)))
        print(f"M={M} rel_l2={err:.3e}")
        assert err <= TOL
    for sg in segs:
        sg.free()


@pytest.mark.parametrize("M", [16, 24])
def test_group_bias_accumulate(gpu, M):
    from cortexsdr_amd import _lib
    from cortexsdr_amd.hsdr import HsdbSegment, group_workspace

    shapes = [(896, 896), (128, 896), (4864, 896)]
    streams = [synth.hsdb_layer(R, Cc, 1024, 8, seed_dict=1, seed_codes=20 + i)
               for i, (R, Cc) in enumerate(shapes)]
    segs = [HsdbSegment(s) for s in streams]
    x = synth.activations(896, M, seed=9, dtype=np.float16)
    xd = gpu.from_numpy(x).cuda()
    rng = np.random.default_rng(1)
    biases = [rng.normal(size=R).astype(np.float32) for R, _ in shapes]
    bd = [gpu.from_numpy(b).cuda() for b in biases]
    ys = [gpu.zeros((R, M), dtype=gpu.float32, device="cuda") for R, _ in shapes]
    ws = group_workspace(segs, M)
    n = len(segs)
    hs = (C.c_void_p * n)(*[s._h.value for s in segs])
    xp = (C.c_void_p * n)(*([xd.data_ptr()] * n))
    yp = (C.c_void_p * n)(*[y.data_ptr() for y in ys])
    bp = (C.c_void_p * n)(*[b.data_ptr() for b in bd])
    lib = _lib.load()
    sp = int(gpu.cuda.current_stream().cuda_stream)
    _lib.check(lib.csdr_hsdb_matmul_group_ex(n, hs, xp, 1, M, yp, bp, 0, ws.data_ptr(),
                                             ws.numel(), sp))
    wx = [oracle.hsdb_matmul(s, x.astype(np.float32)) for s in streams]
    for y, w, b in zip(ys, wx, biases):
        assert rel_l2(y.cpu().numpy(), w + b[:, None]) <= TOL
    _lib.check(lib.csdr_hsdb_matmul_group_ex(n, hs, xp, 1, M, yp, None, 1, ws.data_ptr(),
                                             ws.numel(), sp))
    for y, w, b in zip(ys, wx, biases):
        assert rel_l2(y.cpu().numpy(), 2 * w + b[:, None]) <= TOL
    for s in segs:
        s.free()


def test_mfma_and_p_path_agree(gpu):
    # the matrix-core path and the fp32 dictionary-product path on the same call
    stream = layer(1024, 2048, 1024, 8)
    x = synth.activations(2048, 32, seed=11, dtype=np.float16)
    y_mfma = product(gpu, stream, x, np.float16)
    os.environ["CSDR_HSDB_MFMA"] = "0"
    try:
        y_p = product(gpu, stream, x, np.float16)
    finally:
        del os.environ["CSDR_HSDB_MFMA"]
    ref = oracle.hsdb_matmul(stream, x.astype(np.float32))
    assert rel_l2(y_p, ref) <= 1e-5
    assert rel_l2(y_mfma, ref) <= TOL
