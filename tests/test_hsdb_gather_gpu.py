"""GPU parity of the M == 1 block-coded product (a dx launch writing P = D . x per block
column and Y's start value, then the gather launch of 1024-thread workgroups) against the CPU
oracle, through the C-ABI, over the chunk layouts the segment loader produces (full chunks
of 16 block columns, power-of-two remainders, edge strips, 4 / 8 / 16 slots, K not a
multiple of 4).

Bar: relative L2 <= 1e-3 at fp32 accumulation (P is computed in fp32, so the results agree
with the oracle to ~1e-6).
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from conftest import rel_l2
from cortexsdr_amd import synth

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _segs(streams):
    from cortexsdr_amd.hsdr import HsdbSegment

    return [HsdbSegment(s) for s in streams]


@pytest.mark.parametrize("R,Cc,K,s,dtype", [
    (4096, 11008, 1024, 8, np.float16),   # config 2 (chunks 10 x 16, then 8 and 4)
    (11008, 4096, 1024, 8, np.float16),   # config 2, tall
    (4096, 4096, 512, 4, np.float32),     # config 1 shape
    (896, 896, 1024, 8, np.float32),      # 14 block columns: chunks of 8, 4, 2
    (128, 896, 1024, 8, np.float32),
    (4864, 896, 1024, 8, np.float32),
    (896, 4864, 1024, 8, np.float32),     # 76 block columns: 4 x 16, then 8 and 4
    (300, 1000, 256, 16, np.float32),     # edge strip (40 columns), 16 slots: 64 pieces a row
    (37, 200, 64, 4, np.float32),         # ragged, edge strip, one short chunk
    (1, 512, 128, 8, np.float32),         # a single row
    (64, 4096, 2048, 8, np.float16),      # large dictionary: narrower chunks
    (130, 640, 60, 8, np.float32),        # K not a multiple of 4 or 16
])
def test_gather_parity(gpu, R, Cc, K, s, dtype):
    stream = synth.hsdb_layer(R, Cc, K, s, seed_dict=11, seed_codes=12)
    (seg,) = _segs([stream])
    ws = seg.workspace(1)
    for it in range(3):  # different x each call on one workspace
        x = synth.activations(Cc, 1, seed=20 + it, dtype=dtype)
        y = seg.matmul(gpu.from_numpy(np.ascontiguousarray(x)).cuda(), workspace=ws)
        ref = oracle.hsdb_matmul(stream, x.astype(np.float32))
        err = rel_l2(y.cpu().numpy(), ref)
        print(f"R={R} C={Cc} K={K} s={s} call {it}: rel_l2={err:.3e}", flush=True)
        assert err <= TOL
    seg.free()


def test_separate_launches_match_grouped(gpu):
    """csdr_hsdb_dx_group then csdr_hsdb_gather_group (the two launches issued separately,
    as bench.py times the gather) equal the grouped call."""
    from cortexsdr_amd import _lib
    from cortexsdr_amd.hsdr import group_workspace, matmul_group

    lib = _lib.load()
    streams = [synth.hsdb_layer(4096, 11008, 1024, 8, seed_dict=1, seed_codes=2),
               synth.hsdb_layer(11008, 4096, 1024, 8, seed_dict=1, seed_codes=3)]
    segs = _segs(streams)
    xs = [gpu.from_numpy(synth.activations(s.cols, 1, seed=4 + i, dtype=np.float16)).cuda()
          for i, s in enumerate(segs)]
    ws = group_workspace(segs, 1)
    yg = [y.cpu().numpy() for y in matmul_group(segs, xs, workspace=ws)]
    n = len(segs)
    ys = [gpu.empty((s.rows, 1), dtype=gpu.float32, device="cuda") for s in segs]
    hs = (C.c_void_p * n)(*[s._h.value for s in segs])
    xp = (C.c_void_p * n)(*[x.data_ptr() for x in xs])
    yp = (C.c_void_p * n)(*[y.data_ptr() for y in ys])
    sp = gpu.cuda.current_stream().cuda_stream
    _lib.check(lib.csdr_hsdb_dx_group(n, hs, xp, 1, 1, yp, ws.data_ptr(), ws.numel(), sp))
    _lib.check(lib.csdr_hsdb_gather_group(n, hs, xp, 1, 1, yp, ws.data_ptr(), ws.numel(), sp))
    for a, y, st, x in zip(yg, ys, streams, xs):
        b = y.cpu().numpy()
        assert rel_l2(a, b) <= 1e-6
        assert rel_l2(b, oracle.hsdb_matmul(st, x.cpu().numpy().astype(np.float32))) <= TOL
    for s in segs:
        s.free()


def test_group_bias_accumulate(gpu):
    from cortexsdr_amd import _lib

    lib = _lib.load()
    shapes = [(896, 896), (128, 896), (128, 896)]  # q / k / v of a 0.5B-shaped layer
    streams = [synth.hsdb_layer(r, c, 1024, 8, seed_dict=1, seed_codes=30 + i)
               for i, (r, c) in enumerate(shapes)]
    segs = _segs(streams)
    from cortexsdr_amd.hsdr import group_workspace

    x = synth.activations(896, 1, seed=40)
    xd = gpu.from_numpy(x).cuda()
    rng = np.random.default_rng(5)
    bias = [rng.standard_normal(r).astype(np.float32) for r, _ in shapes]
    y0 = [rng.standard_normal((r, 1)).astype(np.float32) for r, _ in shapes]
    bd = [gpu.from_numpy(b).cuda() for b in bias]
    ws = group_workspace(segs, 1)
    n = len(segs)
    hs = (C.c_void_p * n)(*[s._h.value for s in segs])
    xp = (C.c_void_p * n)(*[xd.data_ptr()] * n)
    bp = (C.c_void_p * n)(*[b.data_ptr() for b in bd])
    for flags in (0, 1):  # Y = W.x + b, then Y += W.x + b
        yd = [gpu.from_numpy(v.copy()).cuda() for v in y0]
        yp = (C.c_void_p * n)(*[y.data_ptr() for y in yd])
        _lib.check(lib.csdr_hsdb_matmul_group_ex(n, hs, xp, 0, 1, yp, bp, flags, ws.data_ptr(),
                                                  ws.numel(), None))
        for st, y, b, v in zip(streams, yd, bias, y0):
            ref = oracle.hsdb_matmul(st, x)[:, 0] + b + (v[:, 0] if flags else 0.0)
            assert rel_l2(y.cpu().numpy()[:, 0], ref) <= TOL
    for s in segs:
        s.free()


def test_graph_replays(gpu):
    """Captured once, replayed several times with eager work and synchronisations in
    between; every replay is checked against the eager result."""
    stream = synth.hsdb_layer(2048, 4096, 1024, 8, seed_dict=7, seed_codes=8)
    (seg,) = _segs([stream])
    ws = seg.workspace(1)
    x = gpu.from_numpy(synth.activations(4096, 1, seed=9, dtype=np.float16)).cuda()
    y = gpu.empty((2048, 1), dtype=gpu.float32, device="cuda")
    eager = seg.matmul(x, workspace=ws).cpu().numpy()
    s = gpu.cuda.Stream()
    with gpu.cuda.stream(s):
        seg.matmul(x, out=y, workspace=ws, stream=s)  # warm-up on the capture stream
        s.synchronize()
        g = gpu.cuda.CUDAGraph()
        with gpu.cuda.graph(g, stream=s):
            seg.matmul(x, out=y, workspace=ws, stream=s)
    for it in range(4):
        y.fill_(float("nan"))
        gpu.cuda.synchronize()
        g.replay()
        gpu.cuda.synchronize()
        assert rel_l2(y.cpu().numpy(), eager) <= 1e-6, it
        _ = (x.float() * 2).sum().item()  # eager work between replays
    ref = oracle.hsdb_matmul(stream, x.cpu().numpy().astype(np.float32))
    assert rel_l2(eager, ref) <= TOL
    seg.free()


@pytest.mark.parametrize("shapes,K", [
    ([(128, 128), (64, 128), (64, 128)], 128),      # tiny decoder q / k / v
    ([(192, 128), (192, 128)], 128),                # tiny gate / up
    ([(896, 896), (128, 896), (128, 896)], 1024),   # 0.5B-shaped q / k / v
])
def test_back_to_back(gpu, shapes, K):
    """Many calls queued back to back on one stream and workspace (as a decode loop issues
    them), each with a new x, each checked against the oracle."""
    from cortexsdr_amd.hsdr import group_workspace, matmul_group

    streams = [synth.hsdb_layer(r, c, K, 8, seed_dict=1, seed_codes=50 + i)
               for i, (r, c) in enumerate(shapes)]
    segs = _segs(streams)
    ws = group_workspace(segs, 1)
    rng = np.random.default_rng(3)
    n_calls = 32
    xs = [[rng.standard_normal((c, 1)).astype(np.float32) for _, c in shapes]
          for _ in range(n_calls)]
    outs = [matmul_group(segs, [gpu.from_numpy(v).cuda() for v in x], workspace=ws)
            for x in xs]
    gpu.cuda.synchronize()
    worst = 0.0
    for x, ys in zip(xs, outs):
        for st, v, y in zip(streams, x, ys):
            worst = max(worst, rel_l2(y.cpu().numpy(), oracle.hsdb_matmul(st, v)))
    print(f"worst rel_l2 over {n_calls} calls: {worst:.3e}")
    assert worst <= TOL
    for s in segs:
        s.free()


def test_groups_share_one_workspace(gpu):
    """Calls over different segment groups (different chunk counts, as a decoder layer's
    q/k/v, o, gate/up and down calls) alternate on one workspace."""
    from cortexsdr_amd.hsdr import group_workspace, matmul_group

    groups = [
        [(128, 128), (128, 128), (128, 128)],   # one chunk each
        [(128, 128)],
        [(300, 1000)],                          # 15 block columns: chunks 8, 4, 2, 1
        [(200, 640), (64, 640)],
    ]
    K = 128
    gs = [[synth.hsdb_layer(r, c, K, 8, seed_dict=1, seed_codes=70 + 10 * gi + i)
           for i, (r, c) in enumerate(g)] for gi, g in enumerate(groups)]
    segs = [_segs(st) for st in gs]
    nbytes = max(int(group_workspace(sg, 1).numel()) for sg in segs)
    ws = gpu.zeros(nbytes, dtype=gpu.uint8, device="cuda")
    rng = np.random.default_rng(8)
    for it in range(12):
        gi = it % len(groups)
        xs = [rng.standard_normal((c, 1)).astype(np.float32) for _, c in groups[gi]]
        ys = matmul_group(segs[gi], [gpu.from_numpy(x).cuda() for x in xs], workspace=ws)
        for st, x, y in zip(gs[gi], xs, ys):
            assert rel_l2(y.cpu().numpy(), oracle.hsdb_matmul(st, x)) <= TOL, (it, gi)
    for sg in segs:
        for s in sg:
            s.free()


@pytest.mark.parametrize("R,Cc,K,s", [
    (896, 4864, 1024, 8),   # the down projection of a 0.5B-shaped layer: 76 block columns
    (300, 1000, 256, 16),   # edge strip
    (40, 2048, 128, 4),
])
def test_accumulate_without_bias_wide(gpu, R, Cc, K, s):
    """Y += W.x (a residual add folded into the product, no bias): the gather workgroups add
    their row totals atomically into Y's existing values."""
    from cortexsdr_amd import _lib

    lib = _lib.load()
    stream = synth.hsdb_layer(R, Cc, K, s, seed_dict=4, seed_codes=5)
    (seg,) = _segs([stream])
    from cortexsdr_amd.hsdr import group_workspace

    ws = group_workspace([seg], 1)
    rng = np.random.default_rng(11)
    y0 = rng.standard_normal((R, 1)).astype(np.float32)
    hs = (C.c_void_p * 1)(seg._h.value)
    for it in range(2):
        x = synth.activations(Cc, 1, seed=60 + it)
        xd = gpu.from_numpy(x).cuda()
        yd = gpu.from_numpy(y0.copy()).cuda()
        xp = (C.c_void_p * 1)(xd.data_ptr())
        yp = (C.c_void_p * 1)(yd.data_ptr())
        _lib.check(lib.csdr_hsdb_matmul_group_ex(1, hs, xp, 0, 1, yp, None, 1, ws.data_ptr(),
                                                  ws.numel(), None))
        ref = y0 + oracle.hsdb_matmul(stream, x)
        assert rel_l2(yd.cpu().numpy(), ref) <= TOL
    seg.free()
