"""The allocation-free product csdr_hsdb_matmul_noalloc against csdr_hsdb_matmul, through the
C-ABI: two calls in a row on the same device scratch, the second with a smaller input (fewer
columns, a smaller matrix), each to the parity bar of the caller-workspace entry point (same
kernels, fp32 accumulation with atomics: agreement to rounding); a product needing more
scratch than the entry point holds is refused with CSDR_E_WORKSPACE.
"""
import ctypes as C

import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu

CSDR_F32, CSDR_F16 = 0, 1
CSDR_E_WORKSPACE = -5
SCRATCH_BYTES = 8 << 20


def _noalloc(torch, seg, x, dt, M):
    from cortexsdr_amd import _lib

    y = torch.full((seg.rows, M), float("nan"), dtype=torch.float32, device="cuda")
    rc = _lib.load().csdr_hsdb_matmul_noalloc(seg._h, x.data_ptr(), dt, M, y.data_ptr(),
                                             int(torch.cuda.current_stream().cuda_stream))
    return rc, y


def _case(torch, R, C_, K, s, M, f16, seed):
    from cortexsdr_amd import synth
    from cortexsdr_amd.hsdr import HsdbSegment

    stream = synth.hsdb_layer(R, C_, K, s, seed_dict=seed, seed_codes=seed + 1)
    seg = HsdbSegment(stream)
    x = synth.activations(C_, M, seed=seed + 2, dtype=np.float16 if f16 else np.float32)
    return seg, torch.from_numpy(x).cuda()


@pytest.mark.parametrize("first,second", [
    ((4096, 11008, 1024, 8, 1, True), (1024, 4096, 1024, 8, 1, True)),   # M = 1 P path
    ((2048, 4096, 1024, 8, 16, True), (512, 2048, 512, 4, 4, False)),   # matrix-core path
    ((4096, 4096, 512, 4, 3, False), (300, 1000, 256, 4, 1, False)),    # any M, edge strips
])
def test_noalloc_matches_workspace_entry_point(gpu, first, second):
    torch = gpu
    for i, (R, C_, K, s, M, f16) in enumerate((first, second)):
        seg, x = _case(torch, R, C_, K, s, M, f16, seed=31 + 10 * i)
        assert seg.workspace_bytes(M) <= SCRATCH_BYTES
        want = seg.matmul(x).cpu().numpy()
        rc, y = _noalloc(torch, seg, x, CSDR_F16 if f16 else CSDR_F32, M)
        torch.cuda.synchronize()
        assert rc == 0
        got = y.cpu().numpy()
        assert np.isfinite(got).all()
        assert rel_l2(got, want) <= 1e-5, (i, rel_l2(got, want))
        seg.free()


def test_noalloc_sizes_scratch_for_the_path_taken(gpu):
    """cfg2's 4096 x 11008 at M = 16 takes the matrix-core path (under 1 MB of transposed X);
    the P path's 11 MB at that M, over the 8 MiB scratch, is not what it needs. Then a smaller
    product at M = 12 on the same scratch."""
    torch = gpu
    for i, (R, C_, K, s, M) in enumerate(((4096, 11008, 1024, 8, 16), (1024, 4096, 512, 8, 12))):
        seg, x = _case(torch, R, C_, K, s, M, True, seed=61 + 10 * i)
        if i == 0:
            # the caller-workspace size covers every path at this M (the P path's 11 MB)
            assert seg.workspace_bytes(M) > SCRATCH_BYTES
        want = seg.matmul(x).cpu().numpy()
        rc, y = _noalloc(torch, seg, x, CSDR_F16, M)
        torch.cuda.synchronize()
        assert rc == 0
        got = y.cpu().numpy()
        assert np.isfinite(got).all()
        assert rel_l2(got, want) <= 1e-5, (i, rel_l2(got, want))
        seg.free()


def test_noalloc_rejects_products_beyond_its_scratch(gpu):
    from cortexsdr_amd import _lib

    torch = gpu
    # P of 172 block columns x 1024 atoms x 16 columns = 11 MiB > 8 MiB (fp32 P path: the
    # matrix-core path is switched off for this matrix shape by its 2048 atoms)
    seg, x = _case(torch, 64, 11008, 2048, 8, 8, False, seed=5)
    assert seg.workspace_bytes(8) > SCRATCH_BYTES
    rc, _ = _noalloc(torch, seg, x, CSDR_F32, 8)
    assert rc == CSDR_E_WORKSPACE
    assert b"allocation-free" in _lib.load().csdr_last_error()
    seg.free()
