"""GPU parity of the Q4_K dequant-matmul (HK5) against the CPU oracle, through the C-ABI.

Bar: dequantised values bit-exact (same arithmetic order as the reference); products at
relative L2 <= 1e-5 (exact products of the quants with x, fp32 sums; M > 1 takes fp16 X)."""
import functools

import numpy as np
import pytest

import oracle
from conftest import rel_l2
from cortexsdr_amd import synth

pytestmark = pytest.mark.gpu


@functools.lru_cache(maxsize=None)
def weights(R, C, order, seed=7):
    return synth.q4k_matrix(R, C, seed=seed, order=order)


ORDERS = {"ggml": oracle.ORC_Q4K_GGML, "interleaved": oracle.ORC_Q4K_INTERLEAVED}


@pytest.mark.parametrize("order", ["ggml", "interleaved"])
def test_dequant_bitexact(gpu, order):
    from cortexsdr_amd import q4k

    blob = weights(64, 1024, order)
    wd = q4k.upload(blob)
    out = q4k.dequant(wd, len(blob) // 144, ORDERS[order]).cpu().numpy()
    ref = oracle.q4k_dequant(np.frombuffer(blob, np.uint8), ORDERS[order])
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("R,C,M,order,xdt", [
    (4096, 4096, 1, "ggml", np.float16),      # config 3, W 4096 x 4096
    (4096, 14336, 1, "ggml", np.float16),     # config 3, W 4096 x 14336
    (4096, 4096, 32, "ggml", np.float16),     # config 3, M = 32
    (4096, 14336, 32, "ggml", np.float16),
    (4096, 14336, 64, "ggml", np.float16),    # four 16-row tiles per wave, 16 super-blocks
    (4096, 4096, 64, "interleaved", np.float16),  # 64 columns, two row tiles per wave
    (300, 1024, 24, "interleaved", np.float16),   # two column tiles, ragged rows
    (300, 1024, 1, "interleaved", np.float32),
    (300, 1024, 5, "interleaved", np.float16),
    (37, 256, 1, "ggml", np.float32),
    (37, 512, 70, "ggml", np.float16),        # more than 64 columns: two column groups
    (4096, 4096, 1, "interleaved", np.float16),
    (8200, 2048, 1, "interleaved", np.float16),  # three rows per wave, ragged last workgroup
    (64, 18432, 1, "ggml", np.float16),       # two x staging batches, partial last wave step
    (96, 18432, 1, "interleaved", np.float32),  # fp32 x: more than 64 KiB of LDS
    (40, 4352, 1, "ggml", np.float32),        # 17 super-blocks: one block in the last step
    (8200, 512, 32, "interleaved", np.float16),  # 257 row tiles: one split, plain stores
    (37, 1280, 3, "ggml", np.float16),        # 5 super-blocks in 8 splits (three empty)
    (1000, 2816, 17, "ggml", np.float16),     # 11 super-blocks in 8 splits of 2; one live column
])
def test_linear(gpu, R, C, M, order, xdt):
    from cortexsdr_amd import q4k

    blob = weights(R, C, order)
    x = synth.activations(C, M, seed=11).T.copy().astype(xdt)  # (M, C)
    wd = q4k.upload(blob)
    y = q4k.linear(wd, R, C, gpu.from_numpy(x).cuda(), ORDERS[order]).cpu().numpy()
    ref = oracle.q4k_linear(blob, R, C, x.astype(np.float32), ORDERS[order])
    err = rel_l2(y, ref)
    print(f"R={R} C={C} M={M} {order} rel_l2={err:.3e}")
    assert err <= 1e-5


def test_kat_blocks_through_gpu(gpu):
    # the reference's known-answer block (test_hsdr_kquants.cpp:106-122) through the GPU
    # dequant in the interleaved order: 26, -4
    from cortexsdr_amd import q4k

    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([np.float16(2.0).view(np.uint16)], "<u2").view(np.uint8)
    b[2:4] = np.array([np.float16(1.0).view(np.uint16)], "<u2").view(np.uint8)
    b[4], b[8], b[16] = 3, 4, 0x05
    out = q4k.dequant(q4k.upload(b.tobytes()), 1, oracle.ORC_Q4K_INTERLEAVED).cpu().numpy()
    assert out[0] == 26.0 and out[1] == -4.0


def test_errors(gpu):
    from cortexsdr_amd import q4k
    from cortexsdr_amd.hsdr import CompressionError

    wd = q4k.upload(weights(4, 512, "ggml"))
    x = gpu.zeros((1, 500), dtype=gpu.float16, device="cuda")
    with pytest.raises(ValueError):
        q4k.linear(wd, 4, 512, x)
    with pytest.raises(CompressionError) as e:
        q4k.linear(wd, 4, 500, gpu.zeros((1, 500), dtype=gpu.float16, device="cuda"))
    assert e.value.code == -1
