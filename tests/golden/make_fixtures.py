"""Writes tests/golden/ref_fixtures.npz from the reference's own code.

Runs in the build container only (it needs oracle/_ref/libcsdr_ref.so, compiled by
`make -C oracle ref` from the reference sources). The .npz holds data only: the inputs
this script generates and the outputs the reference computed for them.

  hsdr1d_*   HierarchicalSDRStrategy::compress on a 64 x 256 fp32 matrix with 1-row tiles
             (K=32, 3 stages x 4), then decompress and matmulRowMajor (x: 256 x 4)
  hsdr1de_*  same with C = 200 (1-row tiles cover the whole row, no edge)
  hsdr2d_*   compress with 8 x 16 tiles on a 40 x 100 matrix (edge strip of 4 columns),
             then decompress
  hsdr2db_*  compress with 8 x 16 tiles on a 45 x 96 matrix (bottom edge of 5 rows)
  q4k/q5k/q6k_*  random super-blocks through dequantizeToFP32 (interleaved orders)
  mha_*      Kernels::multi_head_attention / flash_attention_forward, causal, B=2, T=9,
             hidden=32, heads=4

and tests/golden/hsda_fixtures.npz (`hsda` argument):

  hsda_bytes     SharedDictArchive::writeToStream of compressGroupedSegments over three
                 matrices (32/20/45 x 64, 1-row tiles, K=16, 2 stages x 2) named like GGUF
                 block tensors; hsda_x (64 x 3); per segment i: hsda_name_i, hsda_w_i
                 (HSDAReader::decompress), hsda_y_i (HSDAReader::matmul)

and, added to ref_fixtures.npz without touching its other arrays (`gguf` argument):

  q40/q80_*  random Q4_0 / Q8_0 blocks through dequantizeToFP32 (the compress side's decode,
             which equals the engine's decodeSupportedGGUFQuantized for these two formats)

and tests/golden/hsdr_encode_fixtures.npz (`encode` argument):

  enc_<i>_w, enc_<i>_stream, enc_<i>_cfg  HierarchicalSDRStrategy::compress with
             ksvd_iters = 0 (dictionary initialised from random tiles, then one pass of
             hierarchical matching pursuit) on: random matrices (1-row tiles, C = 48..256,
             and 8 x 16 / 8 x 8 tiles), and matrices whose rows are random rows A, their
             reversals, and reversal-symmetric rows, so that projections onto atom pairs
             (A, reversed A) tie in exact arithmetic and the float summation order decides the
             pick; and tile sizes that are not a multiple of 8 (60, 3 x 13, 100, 5, 9, 18,
             27, 30: the projection's scalar tail). cfg = (tile_rows, tile_cols, K, stages, k per
             stage). cpu_model: the CPU the reference ran on (its dictionary initialisation
             uses that CPU's approximate reciprocal square root).
  fit_<i>_w, fit_<i>_stream, fit_<i>_cfg  the same compress with ksvd_iters = 3..6 (atom
             updates and re-encodes); cfg = (tile_rows, tile_cols, K, stages, k, iters).
             Written with OMP_NUM_THREADS=1 (the tile-norm mean's reduction in tile order).

and tests/golden/sdr_fixtures.npz (`sdr` argument):

  sdr_<i>_bytes, sdr_<i>_listing  .sdr archives written by cortexsdr_amd.formats.write_sdr
             (version 2: a GGUF-named decoder's segments, raw segments with and without
             metadata, with scale / zero point / sorted flags, input / output shapes) and the
             reference's own index lister's output for them (src/tool_sdr_inspect.cpp --all,
             compiled by `make -C oracle inspect`)

and tests/golden/hsda_grouped_fixtures.npz (`hsda_grouped` argument): compressGroupedSegments
with a capped fit pool (reservoir sampling, max_tiles_for_fit), several 1-row tile widths (one
dictionary per width) and 2-D tiles with a skipped matrix, inputs included.

Usage: python tests/golden/make_fixtures.py [hsda | hsda_grouped | gguf | encode | sdr]
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

if sys.argv[1:] in (["encode"], ["hsda"], ["hsda_grouped"]):
    # one OpenMP thread: atomUpdateStep's tile-norm reduction (HierarchicalSDRStrategy.cpp
    # :376) then sums the tiles in order, which the library restates. Set before any library
    # that starts the OpenMP runtime is loaded (the oracle's is, at import).
    os.environ["OMP_NUM_THREADS"] = "1"

import oracle  # noqa: E402


def main() -> None:
    oracle.build(ref=True)
    if oracle.ref() is None:
        raise SystemExit("oracle/_ref/libcsdr_ref.so is not built")
    rng = np.random.default_rng(20261201)
    out = {}

    w = rng.normal(0, 0.05, (64, 256)).astype(np.float32)
    s = oracle.ref_hsdr_compress(w, 1, 256, 32, 3, 4, ksvd_iters=4)
    x = rng.normal(0, 1, (256, 4)).astype(np.float32)
    out["hsdr1d_stream"] = np.frombuffer(s, np.uint8)
    out["hsdr1d_x"] = x
    out["hsdr1d_w"] = oracle.ref_hsdr_decompress(s, 64, 256)
    out["hsdr1d_y"] = oracle.ref_hsdr_matmul_row_major(s, x, 64)

    w = rng.normal(0, 0.05, (48, 200)).astype(np.float32)
    s = oracle.ref_hsdr_compress(w, 1, 200, 16, 2, 3, ksvd_iters=3)
    x = rng.normal(0, 1, (200, 3)).astype(np.float32)
    out["hsdr1de_stream"] = np.frombuffer(s, np.uint8)
    out["hsdr1de_x"] = x
    out["hsdr1de_w"] = oracle.ref_hsdr_decompress(s, 48, 200)
    out["hsdr1de_y"] = oracle.ref_hsdr_matmul_row_major(s, x, 48)

    w = rng.normal(0, 0.05, (40, 100)).astype(np.float32)
    s = oracle.ref_hsdr_compress(w, 8, 16, 16, 3, 2, ksvd_iters=3)
    out["hsdr2d_stream"] = np.frombuffer(s, np.uint8)
    out["hsdr2d_w"] = oracle.ref_hsdr_decompress(s, 40, 100)

    w = rng.normal(0, 0.05, (45, 96)).astype(np.float32)
    s = oracle.ref_hsdr_compress(w, 8, 16, 16, 2, 3, ksvd_iters=3)
    out["hsdr2db_stream"] = np.frombuffer(s, np.uint8)
    out["hsdr2db_w"] = oracle.ref_hsdr_decompress(s, 45, 96)

    for name, nbytes in (("q4_k", 144), ("q5_k", 176), ("q6_k", 210)):
        blocks = rng.integers(0, 256, (6, nbytes), dtype=np.uint8)
        # keep the fp16 scales finite and modest: d (and dmin) from U(0.001, 0.05)
        d_off = 208 if name == "q6_k" else 0
        for i in range(6):
            for off in ((d_off,) if name == "q6_k" else (0, 2)):
                v = np.float16(rng.uniform(0.001, 0.05)).view(np.uint16)
                blocks[i, off:off + 2] = np.array([v], "<u2").view(np.uint8)
        key = name.replace("_", "")
        out[f"{key}_blocks"] = blocks
        out[f"{key}_ref"] = oracle.ref_dequant(blocks.ravel(), name, 6, 256)

    B, T, H, heads = 2, 9, 32, 4
    q = rng.normal(0, 1, (B, T, H)).astype(np.float32)
    k = rng.normal(0, 1, (B, T, H)).astype(np.float32)
    v = rng.normal(0, 1, (B, T, H)).astype(np.float32)
    out["mha_q"], out["mha_k"], out["mha_v"] = q, k, v
    out["mha_out"] = oracle.ref_mha(q, k, v, heads, causal=True)
    out["mha_flash_out"] = oracle.ref_mha(q, k, v, heads, causal=True, flash=True)

    path = os.path.join(HERE, "ref_fixtures.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


def gguf_main() -> None:
    oracle.build(ref=True)
    if oracle.ref() is None:
        raise SystemExit("oracle/_ref/libcsdr_ref.so is missing: run make -C oracle ref")
    path = os.path.join(HERE, "ref_fixtures.npz")
    with np.load(path) as z:
        out = {k: z[k] for k in z.files}
    rng = np.random.default_rng(20261203)
    for name, nbytes in (("q4_0", 18), ("q8_0", 34)):
        blocks = rng.integers(0, 256, (40, nbytes), dtype=np.uint8)
        for i in range(40):  # finite, modest fp16 scales
            v = np.float16(rng.uniform(0.001, 0.05) * rng.choice([-1, 1])).view(np.uint16)
            blocks[i, 0:2] = np.array([v], "<u2").view(np.uint8)
        key = name.replace("_", "")
        out[f"{key}_blocks"] = blocks
        out[f"{key}_ref"] = oracle.ref_dequant(blocks.ravel(), name, 5, 256)
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


def hsda_main() -> None:
    oracle.build(ref=True)
    if oracle.ref() is None:
        raise SystemExit("oracle/_ref/libcsdr_ref.so is not built")
    rng = np.random.default_rng(20261202)
    names = ["blk.0.attn_q.weight", "blk.0.attn_k.weight", "blk.1.ffn_up.weight"]
    mats = {n: rng.normal(0, 0.05, (R, 64)).astype(np.float32)
            for n, R in zip(names, (32, 20, 45))}
    data = oracle.ref_hsda_build(mats, 16, 2, 2, ksvd_iters=3)
    x = rng.normal(0, 1, (64, 3)).astype(np.float32)
    out = {"hsda_bytes": np.frombuffer(data, np.uint8), "hsda_x": x}
    for i, n in enumerate(names):
        R = mats[n].shape[0]
        out[f"hsda_name_{i}"] = np.frombuffer(n.encode(), np.uint8)
        out[f"hsda_w_{i}"] = oracle.ref_hsda_decompress(data, n, R, 64)
        out[f"hsda_y_{i}"] = oracle.ref_hsda_matmul(data, n, x, R)
    path = os.path.join(HERE, "hsda_fixtures.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


def hsda_grouped_main() -> None:
    """tests/golden/hsda_grouped_fixtures.npz: compressGroupedSegments cases with their
    inputs: g<i>_name_<j>, g<i>_w_<j> (inputs), g<i>_cfg (tile_rows, tile_cols, K, stages,
    k, ksvd_iters, max_tiles_for_fit), g<i>_bytes (the archive), g<i>_skipped."""
    oracle.build(ref=True)
    if oracle.ref() is None:
        raise SystemExit("oracle/_ref/libcsdr_ref.so is not built")
    rng = np.random.default_rng(20261203)
    cases = [
        # a capped fit pool: 97 tiles reservoir-sampled into 40
        (["blk.0.attn_q.weight", "blk.0.attn_k.weight", "blk.1.ffn_up.weight"],
         [(32, 64), (20, 64), (45, 64)], (1, 64, 16, 2, 2, 2, 40)),
        # 1-row tiles of different widths: one dictionary per width, in the bucket map's order;
        # a matrix whose rows are not a whole number of 2-row tiles is skipped in 2-D mode
        (["a.weight", "b.weight", "c.weight", "d.weight"],
         [(40, 64), (36, 32), (24, 64), (30, 48)], (1, 64, 8, 2, 2, 1, 0)),
        (["e.weight", "f.weight", "g.weight"],
         [(16, 32), (15, 32), (24, 32)], (2, 8, 8, 2, 2, 1, 0)),
    ]
    out = {}
    for i, (names, shapes, cfg) in enumerate(cases):
        mats = {n: rng.normal(0, 0.05, sh).astype(np.float32) for n, sh in zip(names, shapes)}
        tr, tc, K, S, k, it, cap = cfg
        data, skipped = oracle.ref_hsda_build_ex(mats, tr, tc, K, S, k, it, 0.5, cap)
        for j, n in enumerate(names):
            out[f"g{i}_name_{j}"] = np.frombuffer(n.encode(), np.uint8)
            out[f"g{i}_w_{j}"] = mats[n]
        out[f"g{i}_cfg"] = np.array(cfg, np.int64)
        out[f"g{i}_bytes"] = np.frombuffer(data, np.uint8)
        out[f"g{i}_skipped"] = skipped
    path = os.path.join(HERE, "hsda_grouped_fixtures.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


def cpu_model() -> str:
    """/proc/cpuinfo's model name: the reference's dictionary initialisation depends on the
    CPU's approximate reciprocal square root (its -ffast-math build)."""
    with open("/proc/cpuinfo") as f:
        for line in f:
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    return ""


def symmetric_pairs(C: int, seed: int) -> np.ndarray:
    """Rows: 24 random A, their reversals, 40 reversal-symmetric rows; shuffled."""
    rng = np.random.default_rng(seed)
    a = (rng.standard_normal((24, C)) * 0.02).astype(np.float32)
    sy = (rng.standard_normal((40, C)) * 0.02).astype(np.float32)
    sy = np.maximum(sy, sy[:, ::-1])
    w = np.concatenate([a, a[:, ::-1], sy])
    return np.ascontiguousarray(w[rng.permutation(w.shape[0])])


def encode_main() -> None:
    oracle.build(ref=True)
    if oracle.ref() is None:
        raise SystemExit("oracle/_ref/libcsdr_ref.so is not built")
    rng = np.random.default_rng(20261203)
    cases = []
    for (R, Cc, tr, tc, K, S, k) in [(64, 48, 1, 48, 16, 2, 3), (160, 256, 1, 256, 64, 3, 4),
                                     (96, 96, 8, 16, 32, 3, 2), (200, 72, 1, 72, 40, 2, 5),
                                     (130, 132, 8, 8, 24, 2, 3)]:
        cases.append(((rng.standard_normal((R, Cc)) * 0.02).astype(np.float32), (tr, tc, K, S, k)))
    for C, seed in [(48, 3), (48, 11), (48, 12), (64, 1), (72, 2), (80, 13)]:
        cases.append((symmetric_pairs(C, seed), (1, C, 48, 2, 2)))
    # tile sizes that are not a multiple of 8 (the projection's scalar tail, every length 1-7):
    # 60 = 3 x 16 + 8 + 4, 3 x 13 = 39 = 2 x 16 + 7, 100 = 6 x 16 + 4, 5, 9, 18, 27 = 16 + 8 +
    # 3, 30 = 16 + 8 + 6; own generator, so the cases above and the fit cases below keep their
    # inputs
    rng8 = np.random.default_rng(20261202)
    for (R, Cc, tr, tc, K, S, k) in [(64, 60, 1, 60, 16, 2, 3), (90, 41, 3, 13, 20, 2, 2),
                                     (48, 100, 1, 100, 32, 3, 2), (70, 5, 1, 5, 8, 2, 2),
                                     (60, 9, 1, 9, 8, 2, 2), (60, 18, 1, 18, 8, 2, 2),
                                     (60, 27, 1, 27, 12, 2, 2), (60, 30, 1, 30, 12, 2, 2)]:
        cases.append(((rng8.standard_normal((R, Cc)) * 0.02).astype(np.float32),
                      (tr, tc, K, S, k)))
    out = {}
    for i, (w, cfg) in enumerate(cases):
        tr, tc, K, S, k = cfg
        out[f"enc_{i}_w"] = w
        out[f"enc_{i}_stream"] = np.frombuffer(
            oracle.ref_hsdr_compress(w, tr, tc, K, S, k, ksvd_iters=0), np.uint8)
        out[f"enc_{i}_cfg"] = np.array(cfg, np.int32)
    for i, (R, Cc, tr, tc, K, S, k, it) in enumerate([(64, 256, 1, 256, 32, 3, 4, 4),
                                                       (200, 96, 1, 96, 48, 2, 3, 3),
                                                       (96, 96, 8, 16, 32, 3, 2, 3),
                                                       (256, 64, 1, 64, 64, 3, 5, 6)]):
        w = (rng.standard_normal((R, Cc)) * 0.02).astype(np.float32)
        out[f"fit_{i}_w"] = w
        out[f"fit_{i}_stream"] = np.frombuffer(
            oracle.ref_hsdr_compress(w, tr, tc, K, S, k, ksvd_iters=it), np.uint8)
        out[f"fit_{i}_cfg"] = np.array([tr, tc, K, S, k, it], np.int32)
    out["cpu_model"] = np.frombuffer(cpu_model().encode(), np.uint8)
    path = os.path.join(HERE, "hsdr_encode_fixtures.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


def sdr_archives():
    """The archives of sdr_fixtures.npz, as (name, entries) (deterministic)."""
    from cortexsdr_amd import formats
    from cortexsdr_amd.decoder import DecoderSpec, synthetic_weights

    spec = DecoderSpec(2, 64, 2, 1, 32, 128, 96, 16)
    w = synthetic_weights(spec, n_atoms=16, nnz=2, seed=4)
    dec = formats.decoder_entries(w)
    rng = np.random.default_rng(8)
    raw = [
        formats.SdrEntry(name="meta.json", payload=b'{"arch": "llama"}', data_format="json",
                         original_type=6),
        formats.SdrEntry(name="conv1.weight", payload=rng.standard_normal(24).astype(np.float32)
                         .tobytes(), dims=(2, 3, 4), sparsity=0.25, sorted_indices=True,
                         scale=0.125, zero_point=-3.0, layer_type="Conv", layer_name="conv1",
                         layer_index=7, input_shape=(1, 3, 8, 8), output_shape=(1, 2, 6, 6)),
        formats.SdrEntry(name="q.weight", payload=bytes(range(200)), strategy_id=4,
                         data_format="int8", original_size=800, dims=(10, 20), scale=0.02),
        formats.SdrEntry(name="bias", payload=b"", dims=(0,), zero_point=1.5),
        formats.SdrEntry(name="gguf_tokenizer_model", payload=b"gpt2", data_format="str",
                         original_type=6, input_shape=(4,)),
    ]
    return [("decoder", dec), ("raw", raw), ("mixed", raw[:2] + dec[:5] + raw[2:])]


def sdr_main() -> None:
    import subprocess
    import tempfile

    from cortexsdr_amd import formats

    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "inspect"], check=True)
    tool = os.path.join(ROOT, "oracle", "_ref", "sdr_inspect")
    out = {}
    with tempfile.TemporaryDirectory() as td:
        for i, (name, ents) in enumerate(sdr_archives()):
            path = os.path.join(td, f"{name}.sdr")
            formats.write_sdr(path, ents, version=2)
            listing = subprocess.run([tool, path, "--all"], check=True, capture_output=True,
                                     text=True).stdout
            out[f"sdr_{i}_bytes"] = np.frombuffer(open(path, "rb").read(), np.uint8)
            out[f"sdr_{i}_listing"] = np.frombuffer(listing.encode(), np.uint8)
    path = os.path.join(HERE, "sdr_fixtures.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    if sys.argv[1:] == ["sdr"]:
        sdr_main()
    elif sys.argv[1:] == ["encode"]:
        encode_main()
    elif sys.argv[1:] == ["hsda"]:
        hsda_main()
    elif sys.argv[1:] == ["hsda_grouped"]:
        hsda_grouped_main()
    elif sys.argv[1:] == ["gguf"]:
        gguf_main()
    else:
        main()
