"""GPU parity of the 2 <= M <= 8 block-coded product (the streaming gather with M columns per
code read, fp32 accumulation) and of the token-major layout flag (CSDR_HSDB_TOKEN_MAJOR) on
every product path, against the CPU oracle's fused product (orc_hsdb_matmul, the research
closed form y = sum c * (D[idx] . x_b), pinned by fp64 brute force), through the C-ABI.

Bars: the fp32 gather paths within 1e-5 relative L2 (summation order only); the fp16 P option
at 5 <= M <= 8 (CSDR_HSDB_P16=1: the per-block products P = D . x_b rounded to fp16 once,
about 2e-4 per value) within 1e-3; the matrix-core path (M >= 16) within the path's 1e-3."""
import ctypes as C
import functools

import numpy as np
import pytest

import oracle
from conftest import rel_l2
from cortexsdr_amd import synth

pytestmark = pytest.mark.gpu
TOKEN_MAJOR = 2
ACCUMULATE = 1


@functools.lru_cache(maxsize=None)
def layer(R, Cc, K, s, seed):
    return synth.hsdb_layer(R, Cc, K, s, seed_dict=seed, seed_codes=seed + 1)


def run_group(gpu, streams, x_fm, dtype, M, flags=0, bias=None, y0=None):
    """Y_i = W_i . X through csdr_hsdb_matmul_group_ex with X given feature-major (C x M) or,
    with TOKEN_MAJOR, its transpose; returns Y_i feature-major (R x M) as numpy."""
    from cortexsdr_amd import _lib
    from cortexsdr_amd.hsdr import HsdbSegment, group_workspace

    segs = [HsdbSegment(s) for s in streams]
    tm = bool(flags & TOKEN_MAJOR)
    x = np.ascontiguousarray((x_fm.T if tm else x_fm).astype(dtype))
    xd = gpu.from_numpy(x).cuda()
    ys = []
    for i, sg in enumerate(segs):
        if y0 is None:
            ys.append(gpu.full((sg.rows * M,), float("nan"), dtype=gpu.float32, device="cuda"))
        else:
            y = y0[i].T if tm else y0[i]
            ys.append(gpu.from_numpy(np.ascontiguousarray(y, np.float32).ravel()).cuda())
    bd = [gpu.from_numpy(b).cuda() for b in bias] if bias is not None else None
    ws = group_workspace(segs, M)
    n = len(segs)
    lib = _lib.load()
    hs = (C.c_void_p * n)(*[s._h.value for s in segs])
    xp = (C.c_void_p * n)(*([xd.data_ptr()] * n))
    yp = (C.c_void_p * n)(*[y.data_ptr() for y in ys])
    bp = (C.c_void_p * n)(*[b.data_ptr() for b in bd]) if bd is not None else None
    _lib.check(lib.csdr_hsdb_matmul_group_ex(n, hs, xp, 1 if dtype == np.float16 else 0, M, yp,
                                             bp, flags, ws.data_ptr(), ws.numel(),
                                             int(gpu.cuda.current_stream().cuda_stream)))
    out = []
    for sg, y in zip(segs, ys):
        a = y.cpu().numpy()
        out.append(a.reshape(M, sg.rows).T if tm else a.reshape(sg.rows, M))
        sg.free()
    return out


def tol(M):
    """The bar at batch M on the default paths (see the module note)."""
    return 1e-5 if M <= 8 else 1e-3


@pytest.mark.parametrize("M", [2, 3, 4, 5, 8])
@pytest.mark.parametrize("flags", [0, TOKEN_MAJOR])
def test_config2_small_batch(gpu, M, flags):
    # configs[1] shapes (W 4096 x 11008 and 11008 x 4096, K = 1024, 8 nnz), fp16 activations
    streams = [layer(4096, 11008, 1024, 8, 1), layer(11008, 4096, 1024, 8, 1)]
    x = synth.activations(11008, M, seed=3, dtype=np.float16)
    (y,) = run_group(gpu, streams[:1], x, np.float16, M, flags)
    err = rel_l2(y, oracle.hsdb_matmul(streams[0], x.astype(np.float32)))
    print(f"4096x11008 M={M} flags={flags} rel_l2={err:.3e}")
    assert err <= tol(M)
    x2 = synth.activations(4096, M, seed=4, dtype=np.float16)
    (y2,) = run_group(gpu, streams[1:], x2, np.float16, M, flags)
    assert rel_l2(y2, oracle.hsdb_matmul(streams[1], x2.astype(np.float32))) <= tol(M)


@pytest.mark.parametrize("R,Cc,K,s,M,flags", [
    (4096, 11008, 1024, 8, 5, 0),            # configs[1] shape
    (4096, 11008, 1024, 8, 8, TOKEN_MAJOR),
    (1031, 4160, 512, 4, 6, 0),              # 4 slots, remainder chunks
    (77, 1000, 1024, 16, 7, TOKEN_MAJOR),    # 16 slots, 40-column edge
])
def test_fp16_p_option(gpu, R, Cc, K, s, M, flags):
    # CSDR_HSDB_P16=1 keeps P in fp16 at 5 <= M <= 8 (read per call: the same process runs
    # both): the default fp32 P within 1e-5, the fp16 one within 1e-3 and above the fp32 error
    import os
    stream = layer(R, Cc, K, s, 9)
    x = synth.activations(Cc, M, seed=11, dtype=np.float16)
    ref = oracle.hsdb_matmul(stream, x.astype(np.float32))
    (y32,) = run_group(gpu, [stream], x, np.float16, M, flags)
    os.environ["CSDR_HSDB_P16"] = "1"
    try:
        (y16,) = run_group(gpu, [stream], x, np.float16, M, flags)
    finally:
        del os.environ["CSDR_HSDB_P16"]
    e32, e16 = rel_l2(y32, ref), rel_l2(y16, ref)
    print(f"{R}x{Cc} M={M} fp32 P rel_l2={e32:.3e} fp16 P rel_l2={e16:.3e}")
    assert e32 <= 1e-5 and e16 <= 1e-3 and e16 > e32


@pytest.mark.parametrize("R,Cc,K,s,M", [
    (300, 200, 64, 8, 7),      # ragged rows, 8-column edge strip, fp32 X
    (1031, 4160, 512, 4, 6),   # 4 slots, many chunks incl. the remainder chunks
    (77, 1000, 1024, 16, 2),   # 16 slots, 40-column edge
    (77, 1000, 1024, 16, 7),   # the same at 7 columns (fp16 P, 16 slots)
    (4096, 64, 256, 8, 8),     # one block column
])
@pytest.mark.parametrize("flags", [0, TOKEN_MAJOR])
def test_small_batch_shapes(gpu, R, Cc, K, s, M, flags):
    stream = layer(R, Cc, K, s, 9)
    x = synth.activations(Cc, M, seed=7, dtype=np.float32)
    (y,) = run_group(gpu, [stream], x, np.float32, M, flags)
    assert rel_l2(y, oracle.hsdb_matmul(stream, x)) <= tol(M)


@pytest.mark.parametrize("M", [4, 8, 24])
@pytest.mark.parametrize("flags", [0, TOKEN_MAJOR])
def test_group_bias_accumulate_layouts(gpu, M, flags):
    # a decoder layer's q/k/v group with biases, then += (residual folding); M = 24 takes the
    # matrix-core path
    shapes = [(896, 896), (128, 896), (128, 896)]
    streams = [layer(R, Cc, 1024, 8, 20 + i) for i, (R, Cc) in enumerate(shapes)]
    x = synth.activations(896, M, seed=9, dtype=np.float32)
    rng = np.random.default_rng(M)
    biases = [rng.normal(size=R).astype(np.float32) for R, _ in shapes]
    wx = [oracle.hsdb_matmul(s, x) for s in streams]
    ys = run_group(gpu, streams, x, np.float32, M, flags, bias=biases)
    for y, w, b in zip(ys, wx, biases):
        assert rel_l2(y, w + b[:, None]) <= tol(M)
    y0 = [rng.normal(size=(R, M)).astype(np.float32) for R, _ in shapes]
    ys = run_group(gpu, streams, x, np.float32, M, flags | ACCUMULATE, bias=biases, y0=y0)
    for y, w, b, a in zip(ys, wx, biases, y0):
        assert rel_l2(y, a + w + b[:, None]) <= tol(M)


@pytest.mark.parametrize("M", [16, 40])
def test_matrix_core_path_token_major(gpu, M):
    stream = layer(2048, 1024, 1024, 8, 31)
    x = synth.activations(1024, M, seed=12, dtype=np.float16)
    ref = oracle.hsdb_matmul(stream, x.astype(np.float32))
    (y_fm,) = run_group(gpu, [stream], x, np.float16, M, 0)
    (y_tm,) = run_group(gpu, [stream], x, np.float16, M, TOKEN_MAJOR)
    assert rel_l2(y_fm, ref) <= 1e-3 and rel_l2(y_tm, ref) <= 1e-3
    assert rel_l2(y_tm, y_fm) <= 1e-6
