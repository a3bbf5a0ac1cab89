"""GPU runs of the host tools: the text CLI (cortexsdr_text_cli, the reference's
cortexsdr_cli.cpp one-shot path) and the bench CLI's suite mode (the reference's
cortexsdr_bench runner), on a small decoder archive."""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

from conftest import ROOT
from cortexsdr_amd import formats
from cortexsdr_amd.decoder import DecoderSpec, synthetic_weights

pytestmark = pytest.mark.gpu
CLI = os.path.join(ROOT, "cortexsdr_amd", "bin", "cortexsdr_text_cli")


@pytest.fixture(scope="module")
def archive(tmp_path_factory):
    spec = DecoderSpec(2, 128, 2, 1, 64, 192, 300, 64)
    w = synthetic_weights(spec, n_atoms=128, nnz=8, seed=21, sigma=0.1, norm_jitter=0.1)
    path = str(tmp_path_factory.mktemp("cli") / "dec.sdr")
    formats.write_sdr(path, formats.decoder_entries(w))
    return path


def test_text_cli_profile(gpu, archive, tmp_path):
    from cortexsdr_amd.archive import InferenceEngine

    prof = str(tmp_path / "p.json")
    r = subprocess.run([CLI, "-p", "5 17 250 3 99 42", "-m", "8", "--profile", prof, archive],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    line = [l for l in r.stdout.splitlines() if l.startswith("Response: ")][0]
    toks = [int(t) for t in line[len("Response: "):].split()]
    eng = InferenceEngine(archive)
    try:
        assert toks == eng.generate([5, 17, 250, 3, 99, 42], 8)
    finally:
        eng.close()
    p = json.load(open(prof))
    assert p["tokens"] == 8 and p["tokens_per_sec"] > 0
    assert p["engine_stats"]["generated_tokens"] == 8
    bad = subprocess.run([CLI, "-p", "1 x", "-m", "2", archive], capture_output=True, text=True,
                         timeout=120)
    assert bad.returncode == 1 and "token ids" in bad.stderr


def test_bench_suite(gpu, archive, tmp_path):
    suite = {"project_root": str(tmp_path), "repeats": 2, "warmup_runs": 1,
             "tests": [{"name": "dec", "sdr_path": archive, "prompt": "1 2 3",
                        "max_length": 4, "run_inference": True}]}
    sp = str(tmp_path / "suite.json")
    json.dump(suite, open(sp, "w"))
    out = str(tmp_path / "summary.json")
    r = subprocess.run([sys.executable, "-m", "cortexsdr_amd.bench_cli", "--suite", sp, "--out",
                        out], capture_output=True, text=True, cwd=ROOT, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    res = json.load(open(out))
    t = res["tests"][0]
    assert t["ok"] and len(t["runs"]) == 2
    assert t["tokens_per_sec_p50"] > 0 and t["wall_ms_p95"] >= t["wall_ms_p50"]


@pytest.fixture(scope="module")
def lazy_archive(tmp_path_factory):
    """A decoder whose token embedding is a binary HSDR stream with 1-row tiles (the layout
    the reference CLI decodes lazily), the lm_head a separate output segment."""
    import dataclasses

    from cortexsdr_amd.encode import compress

    spec = DecoderSpec(2, 128, 2, 1, 64, 192, 300, 64)
    w = synthetic_weights(spec, n_atoms=128, nnz=8, seed=23, sigma=0.1, norm_jitter=0.1)
    table = np.random.default_rng(2).standard_normal((spec.vocab, spec.hidden)).astype(np.float32)
    w = dataclasses.replace(w, embedding=compress(table, 1, spec.hidden, 32, 2, 4))
    path = str(tmp_path_factory.mktemp("lazy") / "dec.sdr")
    formats.write_sdr(path, formats.decoder_entries(w))
    return path, w


def test_text_cli_lazy_hsdr(gpu, lazy_archive):
    """--lazy-hsdr: tokens chosen by the CLI's lazy HSDR scoring of the token embedding, the
    same tokens the decoder gives with that choice set directly."""
    from cortexsdr_amd.decoder import Decoder
    from cortexsdr_amd.hsdr import LazyHsdrEmbedding

    path, w = lazy_archive
    prompt = [5, 17, 250, 3, 99, 42]
    outs = {}
    for mode in ("packed", "cli"):
        r = subprocess.run([CLI, "-p", " ".join(map(str, prompt)), "-m", "6", "--lazy-hsdr",
                            mode, path], capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr
        line = [l for l in r.stdout.splitlines() if l.startswith("Response: ")][0]
        outs[mode] = [int(t) for t in line[len("Response: "):].split()]
        assert len(outs[mode]) == 6
    emb = LazyHsdrEmbedding(w.embedding)
    dec = Decoder(w)
    try:
        dec.set_lazy_selection(emb, 1.0)
        dec.prefill(np.array(prompt, np.int32), 0.8, 1.5)
        dec.decode(5, 0.8, 1.5)
        assert list(dec.tokens(len(prompt), 6)) == outs["packed"]
    finally:
        dec.close()
        emb.free()
    bad = subprocess.run([CLI, "-p", "1 2", "-m", "2", "--lazy-hsdr", "cli",
                          lazy_archive[0].replace("lazy", "nope")], capture_output=True,
                         text=True, timeout=120)
    assert bad.returncode != 0


def test_text_cli_lazy_needs_hsdr_embedding(gpu, archive):
    # the tied archive's token embedding is HSDB-coded: no lazy HSDR reading of it
    r = subprocess.run([CLI, "-p", "1 2 3", "-m", "2", "--lazy-hsdr", "packed", archive],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 1 and "HSDR" in r.stderr
