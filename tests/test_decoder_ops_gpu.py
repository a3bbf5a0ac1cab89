"""GPU parity of the decoder ops (HK6 attention, HK7 elementwise, HK8 token selection, tied
embedding row decode, bias/residual-folded HSDB products) against the CPU oracle, through
the C-ABI."""
import ctypes as C

import numpy as np
import pytest

import oracle
from conftest import rel_l2
from cortexsdr_amd import synth

pytestmark = pytest.mark.gpu


def lib():
    from cortexsdr_amd import _lib

    return _lib.load()


def sp(gpu):
    return int(gpu.cuda.current_stream().cuda_stream)


def chk(rc):
    from cortexsdr_amd import _lib

    _lib.check(rc)


def dev(gpu, a):
    return gpu.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("ntok,n", [(1, 896), (3, 4096), (2, 77)])
def test_rms_norm(gpu, ntok, n):
    rng = np.random.default_rng(1)
    x = rng.normal(size=(ntok, n)).astype(np.float32)
    w = rng.normal(size=n).astype(np.float32)
    xd, wd = dev(gpu, x), dev(gpu, w)
    y = gpu.empty_like(xd)
    chk(lib().csdr_rms_norm(xd.data_ptr(), wd.data_ptr(), ntok, n, 1e-5, y.data_ptr(), sp(gpu)))
    assert rel_l2(y.cpu().numpy(), oracle.rms_norm(x, w)) < 1e-6


def test_silu_mul(gpu):
    rng = np.random.default_rng(2)
    g = rng.normal(size=4864).astype(np.float32) * 4
    u = rng.normal(size=4864).astype(np.float32)
    gd, ud = dev(gpu, g), dev(gpu, u)
    y = gpu.empty_like(gd)
    chk(lib().csdr_silu_mul(gd.data_ptr(), ud.data_ptr(), g.size, y.data_ptr(), sp(gpu)))
    assert rel_l2(y.cpu().numpy(), oracle.silu_mul(g, u)) < 1e-6


@pytest.mark.parametrize("pos", [0, 5, 511, 639])
def test_rope_kv(gpu, pos):
    rng = np.random.default_rng(3 + pos)
    Hq, Hkv, hd, T = 14, 2, 64, 640
    q = rng.normal(size=(Hq, hd)).astype(np.float32)
    k = rng.normal(size=(Hkv, hd)).astype(np.float32)
    v = rng.normal(size=(Hkv, hd)).astype(np.float32)
    qd, kd, vd = dev(gpu, q), dev(gpu, k), dev(gpu, v)
    kc = gpu.zeros((T, Hkv, hd), dtype=gpu.float16, device="cuda")
    vc = gpu.zeros((T, Hkv, hd), dtype=gpu.float16, device="cuda")
    pd = gpu.tensor([pos], dtype=gpu.int32, device="cuda")
    chk(lib().csdr_rope_kv(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), 1, Hq, Hkv, hd,
                           pd.data_ptr(), 1e6, kc.data_ptr(), vc.data_ptr(), T, sp(gpu)))
    qr = oracle.rope(q[None], Hq, hd, 1e6, pos)[0]
    kr = oracle.rope(k[None], Hkv, hd, 1e6, pos)[0]
    # the angle pos * theta^(-i/hd) is an fp32 product: a 1-ulp difference between host and
    # device powf moves it by up to pos * 6e-8 rad, so the bound grows with the position
    tol = 1e-6 + pos * 1.2e-7
    assert rel_l2(qd.cpu().numpy(), qr) < tol
    assert rel_l2(kd.cpu().numpy(), kr) < tol
    assert np.array_equal(kc[pos].cpu().numpy(), kd.cpu().numpy().astype(np.float16))
    assert np.array_equal(vc[pos].cpu().numpy(), v.astype(np.float16))
    assert not kc[:pos].cpu().numpy().any()


@pytest.mark.parametrize("B,T,L,Hq,Hkv,hd", [
    (1, 640, 577, 14, 2, 64),     # config 4 shape
    (1, 640, 1, 14, 2, 64),
    (1, 4096, 4096, 32, 32, 128), # config 5 shape, batch 1
    (2, 300, None, 8, 2, 128),    # per-batch lengths
    (1, 256, 256, 4, 1, 64),      # exactly one split
    (1, 1280, 641, 14, 2, 64),    # two 640-position splits, the second holding one position
    (1, 2000, 1999, 32, 2, 128),  # 16 query heads per KV head, six splits
    (3, 700, None, 12, 4, 64),    # three query heads per KV head, ragged lengths
    (1, 48, 37, 6, 3, 128),       # a length that is not a multiple of 16
    (8, 4096, None, 32, 32, 128), # config 5 shape, batch 8 (several rounds of splits),
                                  # ragged lengths
    (6, 2000, None, 16, 16, 64),  # the same at head size 64
])
@pytest.mark.parametrize("mfma", ["1", "0"])
def test_attn_decode(gpu, B, T, L, Hq, Hkv, hd, mfma, monkeypatch):
    # CSDR_ATTN_MFMA=0 keeps the VALU kernels for grouped heads (attn_lds_kernel)
    monkeypatch.setenv("CSDR_ATTN_MFMA", mfma)
    rng = np.random.default_rng(4)
    q = rng.normal(size=(B, Hq, hd)).astype(np.float32)
    kc = rng.normal(size=(B, T, Hkv, hd)).astype(np.float16)
    vc = rng.normal(size=(B, T, Hkv, hd)).astype(np.float16)
    lens = np.array([T - 17 * b for b in range(B)], np.int32) if L is None else \
        np.full(B, L, np.int32)
    qd, kd, vd = dev(gpu, q), dev(gpu, kc), dev(gpu, vc)
    out = gpu.empty_like(qd)
    wsb = lib().csdr_attn_decode_workspace_bytes(B, Hq, hd, T)
    ws = gpu.zeros(max(wsb, 4), dtype=gpu.uint8, device="cuda")
    ld = dev(gpu, lens) if L is None else None
    chk(lib().csdr_attn_decode(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                               ld.data_ptr() if ld is not None else None, int(lens[0]), B, T, Hq,
                               Hkv, hd, 0.0, out.data_ptr(), ws.data_ptr(), ws.numel(), sp(gpu)))
    ref = oracle.attn_decode(q, kc.view(np.uint16), vc.view(np.uint16), lens, Hq, Hkv, hd)
    assert rel_l2(out.cpu().numpy(), ref) < 1e-5


@pytest.mark.parametrize("n", [151936, 1000, 7])
def test_select_best(gpu, n):
    rng = np.random.default_rng(5)
    lg = rng.normal(size=n).astype(np.float32)
    lg[n // 3] = lg[n // 2] = lg.max() + 1.0  # tie: the first index wins
    if n > 10:
        lg[3] = np.nan
        lg[4] = np.inf
    rep = (rng.random(n) < 0.1).astype(np.uint8)
    ld, rd = dev(gpu, lg), dev(gpu, rep)
    out = gpu.zeros(1, dtype=gpu.int32, device="cuda")
    pos = gpu.zeros(1, dtype=gpu.int32, device="cuda")
    upd = gpu.zeros(n, dtype=gpu.uint8, device="cuda")
    ws = gpu.zeros(lib().csdr_select_workspace_bytes(), dtype=gpu.uint8, device="cuda")
    for temp, pen, use_rep in ((0.0, 0.0, False), (0.8, 1.5, True)):
        chk(lib().csdr_select_best(ld.data_ptr(), n, rd.data_ptr() if use_rep else None, temp, pen,
                                   out.data_ptr(), pos.data_ptr(), upd.data_ptr(), ws.data_ptr(),
                                   ws.numel(), sp(gpu)))
        ref = oracle.select_best(lg, rep if use_rep else None, temp, pen)
        assert int(out.item()) == ref
    assert int(pos.item()) == 2
    assert upd.cpu().numpy().sum() >= 1


def test_decode_row_and_bias_accumulate(gpu):
    from cortexsdr_amd.hsdr import HsdbSegment, group_workspace

    R, Cc = 300, 200  # edge strip of 8 columns
    stream = synth.hsdb_layer(R, Cc, 64, 8, seed_dict=3, seed_codes=4)
    seg = HsdbSegment(stream)
    w = oracle.hsdr_decompress(stream)
    out = gpu.zeros(Cc, dtype=gpu.float32, device="cuda")
    row = gpu.tensor([123], dtype=gpu.int32, device="cuda")
    chk(lib().csdr_hsdb_decode_row(seg._h, row.data_ptr(), 0, out.data_ptr(), sp(gpu)))
    assert np.array_equal(out.cpu().numpy().view(np.uint32), w[123].view(np.uint32))
    chk(lib().csdr_hsdb_decode_row(seg._h, None, 299, out.data_ptr(), sp(gpu)))
    assert np.array_equal(out.cpu().numpy().view(np.uint32), w[299].view(np.uint32))
    # y = W x + bias, then y += W x (residual folding)
    x = synth.activations(Cc, 1, seed=5)
    bias = np.random.default_rng(6).normal(size=R).astype(np.float32)
    xd, bd = dev(gpu, x), dev(gpu, bias)
    y = gpu.zeros((R, 1), dtype=gpu.float32, device="cuda")
    ws = group_workspace([seg], 1)
    hs = (C.c_void_p * 1)(seg._h.value)
    xp = (C.c_void_p * 1)(xd.data_ptr())
    yp = (C.c_void_p * 1)(y.data_ptr())
    bp = (C.c_void_p * 1)(bd.data_ptr())
    chk(lib().csdr_hsdb_matmul_group_ex(1, hs, xp, 0, 1, yp, bp, 0, ws.data_ptr(), ws.numel(),
                                        sp(gpu)))
    wx = oracle.hsdb_matmul(stream, x)[:, 0]
    assert rel_l2(y.cpu().numpy()[:, 0], wx + bias) < 1e-5
    chk(lib().csdr_hsdb_matmul_group_ex(1, hs, xp, 0, 1, yp, None, 1, ws.data_ptr(), ws.numel(),
                                        sp(gpu)))
    assert rel_l2(y.cpu().numpy()[:, 0], 2 * wx + bias) < 1e-5


@pytest.mark.parametrize("M,p16", [(1, False), (3, False), (8, False), (8, True), (6, True),
                                   (12, False), (16, False)])
def test_matmul_xop_rmsnorm_and_silu(gpu, M, p16, monkeypatch):
    # p16: the fp16 P option of the 5 <= M <= 8 gather (CSDR_HSDB_P16=1), its x-op writes of P
    # included; one fp16 rounding per P value, so the bar is 1e-3 there
    from cortexsdr_amd.hsdr import HsdbSegment, group_workspace

    if p16:
        monkeypatch.setenv("CSDR_HSDB_P16", "1")
    tol = 1e-3 if p16 else 1e-5

    R, Cc = 300, 200  # 3 block columns + an 8-column edge strip (transformed too)
    stream = synth.hsdb_layer(R, Cc, 64, 8, seed_dict=3, seed_codes=9)
    seg = HsdbSegment(stream)
    rng = np.random.default_rng(7)
    x = rng.normal(size=(Cc, M)).astype(np.float32) * 3
    x2 = rng.normal(size=(Cc, M)).astype(np.float32)
    nw = rng.normal(size=Cc).astype(np.float32)
    bias = rng.normal(size=R).astype(np.float32)
    xd, x2d, nwd, bd = dev(gpu, x), dev(gpu, x2), dev(gpu, nw), dev(gpu, bias)
    y = gpu.zeros((R, M), dtype=gpu.float32, device="cuda")
    ws = group_workspace([seg], M)
    hs = (C.c_void_p * 1)(seg._h.value)
    xp = (C.c_void_p * 1)(xd.data_ptr())
    x2p = (C.c_void_p * 1)(x2d.data_ptr())
    yp = (C.c_void_p * 1)(y.data_ptr())
    bp = (C.c_void_p * 1)(bd.data_ptr())
    chk(lib().csdr_hsdb_matmul_group_xop(1, hs, xp, None, M, yp, bp, 0, 1, nwd.data_ptr(), 1e-5,
                                         0, 0, ws.data_ptr(), ws.numel(), sp(gpu)))
    xn = oracle.rms_norm(np.ascontiguousarray(x.T), nw).T   # per column
    ref = oracle.hsdb_matmul(stream, np.ascontiguousarray(xn)) + bias[:, None]
    assert rel_l2(y.cpu().numpy(), ref) < tol
    chk(lib().csdr_hsdb_matmul_group_xop(1, hs, xp, x2p, M, yp, None, 1, 2, None, 0.0, 0, 0,
                                         ws.data_ptr(), ws.numel(), sp(gpu)))
    xs = oracle.silu_mul(x, x2)
    ref2 = ref + oracle.hsdb_matmul(stream, xs)
    assert rel_l2(y.cpu().numpy(), ref2) < tol


@pytest.mark.parametrize("Hq,Hkv,hd,L,T", [(14, 2, 64, 300, 640), (32, 32, 128, 1000, 4096),
                                           (4, 4, 64, 1, 64), (32, 2, 128, 700, 1000),
                                           (14, 2, 64, 641, 1280), (8, 4, 64, 16, 640),
                                           # 67 splits x 32 heads: more partials than the
                                           # o projection's LDS weight table holds
                                           (32, 32, 64, 16999, 17000)])
def test_attn_rope_fused_matches_unfused(gpu, Hq, Hkv, hd, L, T):
    from cortexsdr_amd.hsdr import HsdbSegment, group_workspace

    rng = np.random.default_rng(11)
    q = rng.normal(size=(Hq, hd)).astype(np.float32)
    k = rng.normal(size=(Hkv, hd)).astype(np.float32)
    v = rng.normal(size=(Hkv, hd)).astype(np.float32)
    kc = rng.normal(size=(T, Hkv, hd)).astype(np.float16)
    vc = rng.normal(size=(T, Hkv, hd)).astype(np.float16)
    pos = L - 1
    # unfused: rope_kv then attention then the o projection
    qd, kd, vd = dev(gpu, q), dev(gpu, k), dev(gpu, v)
    kcd, vcd = dev(gpu, kc), dev(gpu, vc)
    pd = gpu.tensor([pos], dtype=gpu.int32, device="cuda")
    ld = gpu.tensor([L], dtype=gpu.int32, device="cuda")
    chk(lib().csdr_rope_kv(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), 1, Hq, Hkv, hd,
                           pd.data_ptr(), 1e6, kcd.data_ptr(), vcd.data_ptr(), T, sp(gpu)))
    out = gpu.empty((Hq, hd), dtype=gpu.float32, device="cuda")
    wsb = lib().csdr_attn_decode_workspace_bytes(1, Hq, hd, T)
    ws = gpu.zeros(max(wsb, 4), dtype=gpu.uint8, device="cuda")
    chk(lib().csdr_attn_decode(qd.data_ptr(), kcd.data_ptr(), vcd.data_ptr(), ld.data_ptr(), 0, 1,
                               T, Hq, Hkv, hd, 0.0, out.data_ptr(), ws.data_ptr(), ws.numel(),
                               sp(gpu)))
    # fused: rotation and append inside the attention, partials combined by the o projection
    q2, k2, v2 = dev(gpu, q), dev(gpu, k), dev(gpu, v)
    kc2, vc2 = dev(gpu, kc), dev(gpu, vc)
    ws2 = gpu.zeros(max(wsb, 4), dtype=gpu.uint8, device="cuda")
    out2 = gpu.empty((Hq, hd), dtype=gpu.float32, device="cuda")
    chk(lib().csdr_attn_decode_rope(q2.data_ptr(), k2.data_ptr(), v2.data_ptr(), kc2.data_ptr(),
                                    vc2.data_ptr(), ld.data_ptr(), 1, T, Hq, Hkv, hd, 1e6, 0.0,
                                    out2.data_ptr(), ws2.data_ptr(), ws2.numel(), sp(gpu)))
    assert rel_l2(out2.cpu().numpy(), out.cpu().numpy()) < 1e-6
    assert np.array_equal(kc2.cpu().numpy()[pos], kcd.cpu().numpy()[pos])
    assert np.array_equal(vc2.cpu().numpy()[pos], vcd.cpu().numpy()[pos])
    H = Hq * hd
    stream = synth.hsdb_layer(96, H, 64, 4, seed_dict=2, seed_codes=3)
    seg = HsdbSegment(stream)
    y = gpu.zeros((96, 1), dtype=gpu.float32, device="cuda")
    wsm = group_workspace([seg], 1)
    chk(lib().csdr_attn_decode_rope(q2.data_ptr(), k2.data_ptr(), v2.data_ptr(), kc2.data_ptr(),
                                    vc2.data_ptr(), ld.data_ptr(), 1, T, Hq, Hkv, hd, 1e6, 0.0,
                                    None, ws2.data_ptr(), ws2.numel(), sp(gpu)))
    nsplit = lib().csdr_attn_decode_splits(1, Hq, Hkv, hd, T)
    hs = (C.c_void_p * 1)(seg._h.value)
    xp = (C.c_void_p * 1)(ws2.data_ptr())
    yp = (C.c_void_p * 1)(y.data_ptr())
    chk(lib().csdr_hsdb_matmul_group_xop(1, hs, xp, None, 1, yp, None, 0, 3, None, 0.0, nsplit,
                                         hd, wsm.data_ptr(), wsm.numel(), sp(gpu)))
    ref = oracle.hsdb_matmul(stream, out.cpu().numpy().reshape(H, 1))
    assert rel_l2(y.cpu().numpy(), ref) < 1e-5
