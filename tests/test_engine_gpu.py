"""GPU parity of the SDK surface: cortex_inference_engine_* over .sdr archives (run_layer
routing for strategy-5 HSDR/HSDB, uncoded fp32, q4_k and the other GGUF block segments;
memory options;
generate_text through the native decoder), HSDA/HSDC loads, against the CPU oracle and the
reference's own fixtures."""
import os

import numpy as np
import pytest

import oracle
from conftest import GOLDEN, rel_l2
from cortexsdr_amd import formats, synth
from cortexsdr_amd.archive import EngineError, HsdaArchive, InferenceEngine

pytestmark = pytest.mark.gpu


def q4k_entry(name, R, Cc, seed):
    blob = synth.q4k_matrix(R, Cc, seed=seed)
    return formats.SdrEntry(name=name, payload=blob, data_format="q4_k", original_type=3,
                            original_size=R * Cc * 4, dims=(R, Cc)), blob


def gguf_entry(name, fmt, R, Cc, seed):
    """Random blocks of a GGUF format with finite fp16 scales (q6_k's at byte 208)."""
    rng = np.random.default_rng(seed)
    bb, be = oracle.gguf_block(oracle.GGUF_FORMATS[fmt.lower()])
    b = rng.integers(0, 256, (R * Cc // be, bb), dtype=np.uint8)
    off = 208 if fmt.lower() == "q6_k" else 0
    b[:, off:off + 2] = rng.uniform(0.002, 0.03, b.shape[0]).astype(np.float16).view(
        np.uint8).reshape(-1, 2)
    blob = b.tobytes()
    return formats.SdrEntry(name=name, payload=blob, data_format=fmt, original_type=3,
                            original_size=R * Cc * 4, dims=(R, Cc)), blob


GGUF_ENTRIES = [("blk.0.attn_v.weight", "q6_k", 6, 512), ("blk.0.ffn_gate.weight", "q8_0", 9, 96),
                ("blk.0.attn_k.weight", "q5_k", 4, 256), ("blk.0.ffn_up.weight", "Q4_0", 5, 64)]


@pytest.fixture(scope="module")
def model(tmp_path_factory, golden):
    path = str(tmp_path_factory.mktemp("sdr") / "model.sdr")
    hsdb = synth.hsdb_layer(64, 256, 32, 4, seed_dict=1, seed_codes=2)
    hsdb_edge = synth.hsdb_layer(40, 200, 64, 8, seed_dict=3, seed_codes=4)
    dense = np.random.default_rng(0).normal(size=(5, 7)).astype(np.float32)
    q4e, q4blob = q4k_entry("blk.0.ffn_down.weight", 8, 512, 9)
    ents = [
        formats.hsdb_entry("blk.0.attn_q.weight", hsdb),
        formats.hsdb_entry("edge.weight", hsdb_edge),
        formats.SdrEntry(name="hsdr_ref", payload=golden["hsdr1d_stream"].tobytes(),
                         strategy_id=5, dims=(64, 256)),
        formats.SdrEntry(name="dense.weight", payload=dense.tobytes(), dims=(5, 7)),
        q4e,
        formats.SdrEntry(name="rle.weight", payload=b"\x00" * 16, strategy_id=2, dims=(2, 2)),
    ]
    gg = {}
    for i, (name, fmt, R, Cc) in enumerate(GGUF_ENTRIES):
        e, blob = gguf_entry(name, fmt, R, Cc, 20 + i)
        ents.append(e)
        gg[name] = blob
    formats.write_sdr(path, ents)
    return dict(path=path, hsdb=hsdb, hsdb_edge=hsdb_edge, dense=dense, q4=q4blob, gguf=gg)


def test_run_layer_routes(gpu, model, golden):
    eng = InferenceEngine(model["path"])
    try:
        x = synth.activations(256, 1, seed=5)[:, 0]
        y = eng.run_layer("blk.0.attn_q", x)                 # ".weight" fallback
        assert rel_l2(y, oracle.hsdb_matmul(model["hsdb"], x[:, None])[:, 0]) < 1e-5
        assert eng.stats()["path"] == "hsdb"
        X = synth.activations(200, 3, seed=6)                # (C, M) -> the API's (M, C)
        Y = eng.run_layer("edge.weight", X.T).reshape(3, 40)
        # batches of 2+ take the matrix-core path (fp16 dictionary/weights: ~3e-4)
        assert rel_l2(Y.T, oracle.hsdb_matmul(model["hsdb_edge"], X)) < 1e-3
        xr = golden["hsdr1d_x"]                              # reference HSDR payload, batch 4
        Y = eng.run_layer("hsdr_ref", xr.T).reshape(4, 64)
        assert rel_l2(Y.T, golden["hsdr1d_y"]) < 1e-5
        xd = np.random.default_rng(1).normal(size=(2, 7)).astype(np.float32)
        Y = eng.run_layer("dense.weight", xd).reshape(2, 5)
        assert rel_l2(Y, xd @ model["dense"].T) < 1e-6
        # Q4_K batches take the matrix-core form (x as exact fp16 hi + lo parts, weights
        # unrounded): fp32-level agreement at every batch
        for M in (1, 2, 32):
            xq = synth.activations(512, M, seed=7)
            Y = eng.run_layer("blk.0.ffn_down.weight", xq.T).reshape(M, 8)
            ref = oracle.q4k_linear(model["q4"], 8, 512, xq.T.copy())
            assert rel_l2(Y, ref) < 1e-5, M
        # inputs beyond fp16's range keep the fp32 GEMV form
        xb = (synth.activations(512, 2, seed=8) * 1e5).astype(np.float32)
        Y = eng.run_layer("blk.0.ffn_down.weight", xb.T).reshape(2, 8)
        assert rel_l2(Y, oracle.q4k_linear(model["q4"], 8, 512, xb.T.copy())) < 1e-5
        assert eng.memory_usage() > 0
    finally:
        eng.close()


def test_run_layer_gguf_formats(gpu, model):
    """Strategy-0 tensors in the other GGUF block formats route to csdr_gguf_linear with the
    reference engine's decode (its data_format names, any case)."""
    eng = InferenceEngine(model["path"])
    try:
        for name, fmt, R, Cc in GGUF_ENTRIES:
            # M = 1: the GEMV on fp32 x (1e-5); M > 1: the matrix-core form for the whole batch
            # (fp16 hi + lo parts of x, decoded values rounded to fp16 once: the path's 1e-3)
            for M, tol in ((1, 1e-5), (3, 1e-3)):
                x = np.random.default_rng(R + M).normal(size=(M, Cc)).astype(np.float32)
                Y = eng.run_layer(name, x).reshape(M, R)
                ref = oracle.gguf_linear(model["gguf"][name], oracle.GGUF_FORMATS[fmt.lower()],
                                         R, Cc, x)
                assert rel_l2(Y, ref) < tol, (fmt, M)
                assert eng.stats()["path"] == "gguf"
    finally:
        eng.close()


def test_run_layer_errors(gpu, model):
    eng = InferenceEngine(model["path"])
    try:
        with pytest.raises(EngineError) as e:
            eng.run_layer("missing", np.zeros(4, np.float32))
        assert e.value.code == -7
        with pytest.raises(EngineError) as e:
            eng.run_layer("blk.0.attn_q.weight", np.zeros(255, np.float32))
        assert e.value.code == -1
        with pytest.raises(EngineError) as e:                # too small: needs 64
            eng.run_layer("blk.0.attn_q.weight", np.zeros(256, np.float32), out_size=10)
        assert e.value.code == -3
        with pytest.raises(EngineError) as e:
            eng.run_layer("rle.weight", np.zeros(2, np.float32))
        assert e.value.code == -4
        import ctypes as C
        from cortexsdr_amd import _lib
        n = C.c_size_t()
        err = _lib.load().cortex_inference_engine_run(eng._h, None, 0, None, 0, C.byref(n))
        assert err.code == -1                                # null pointers (cortex_sdk.cpp:1860)
        # this archive's segments do not chain (widths differ from layer to layer)
        with pytest.raises(EngineError) as e:
            eng.run(np.zeros(256, np.float32))
        assert e.value.code in (-4, -7)
    finally:
        eng.close()
    with pytest.raises(EngineError):
        InferenceEngine(model["path"] + ".nope")


def test_memory_options(gpu, model):
    eng = InferenceEngine(model["path"])
    try:
        x = np.ones(256, np.float32)
        eng.run_layer("blk.0.attn_q.weight", x)
        one = eng.memory_usage()
        eng.run_layer("edge.weight", np.ones(200, np.float32))
        two = eng.memory_usage()
        assert two > one > 0
        eng.set_memory_pool(0)                               # unbounded: nothing released
        assert eng.memory_usage() == two
        eng.set_aggressive_memory(True)
        eng.run_layer("dense.weight", np.ones(7, np.float32))
        assert eng.memory_usage() == two                     # the dense segment went again
        eng.set_aggressive_memory(False)
        eng.set_memory_pool(1)                               # 1 MiB: LRU eviction
        assert eng.memory_usage() <= 1 << 20
        y = eng.run_layer("blk.0.attn_q.weight", x)          # reloads on demand
        assert rel_l2(y, oracle.hsdb_matmul(model["hsdb"], x[:, None])[:, 0]) < 1e-5
    finally:
        eng.close()


def test_matmul_device(gpu, model):
    eng = InferenceEngine(model["path"])
    try:
        X = synth.activations(256, 5, seed=8, dtype=np.float16)
        xd = gpu.from_numpy(X).cuda()
        yd = gpu.empty((64, 5), dtype=gpu.float32, device="cuda")
        eng.matmul_device("blk.0.attn_q.weight", xd, yd)
        gpu.cuda.synchronize()
        assert rel_l2(yd.cpu().numpy(), oracle.hsdb_matmul(model["hsdb"], X.astype(np.float32))) < 1e-3
        with pytest.raises(EngineError):
            eng.matmul_device("dense.weight", xd, yd)        # not strategy 5
    finally:
        eng.close()


def test_hsda_and_hsdc_loads(gpu):
    import ctypes as C
    from cortexsdr_amd import _lib
    from cortexsdr_amd.hsdr import HsdbSegment

    f = np.load(os.path.join(GOLDEN, "hsda_fixtures.npz"), allow_pickle=False)
    data = f["hsda_bytes"].tobytes()
    a = HsdaArchive(data=data)
    x = gpu.from_numpy(f["hsda_x"]).cuda()
    for i in range(3):
        name = f[f"hsda_name_{i}"].tobytes().decode()
        seg = a.load(name)
        y = seg.matmul(x).cpu().numpy()         # batch 3: matrix-core path (fp16 operands)
        assert rel_l2(y, f[f"hsda_y_{i}"]) < 1e-3
        os.environ["CSDR_HSDB_MFMA"] = "0"      # the fp32 path agrees to rounding
        try:
            y32 = seg.matmul(x).cpu().numpy()
        finally:
            del os.environ["CSDR_HSDB_MFMA"]
        assert rel_l2(y32, f[f"hsda_y_{i}"]) < 1e-6
        w = seg.decompress().cpu().numpy()
        assert np.array_equal(w.view(np.uint32), f[f"hsda_w_{i}"].view(np.uint32))
        seg.free()
    # the same codes through csdr_hsdb_load_codes with the dictionary passed explicitly
    dicts, segs = oracle.hsda_parse(data)
    d = dicts[0]
    sc = np.ascontiguousarray(d["stage_scales"], np.float32)
    at = np.ascontiguousarray(d["atoms"], np.float32)
    cd = _lib.Dictionary(d["tile_rows"], d["tile_cols"], d["n_atoms"], d["n_stages"], d["k"],
                         d["stage_decay"], sc.ctypes.data, sc.size, at.ctypes.data, at.size)
    codes = segs[2][4]
    h = C.c_void_p()
    _lib.check(_lib.load().csdr_hsdb_load_codes(codes, len(codes), C.byref(cd), None,
                                                C.byref(h)))
    seg = HsdbSegment.from_handle(h)
    w = seg.decompress().cpu().numpy()
    assert np.array_equal(w.view(np.uint32), f["hsda_w_2"].view(np.uint32))
    seg.free()
    bad = _lib.Dictionary(d["tile_rows"], d["tile_cols"], d["n_atoms"] + 1, d["n_stages"], d["k"],
                          d["stage_decay"], sc.ctypes.data, sc.size, at.ctypes.data, at.size)
    assert _lib.load().csdr_hsdb_load_codes(codes, len(codes), C.byref(bad), None,
                                            C.byref(h)) == -2  # geometry mismatch
    with pytest.raises(_lib.CsdrError):
        a.load("no.such.segment")


def test_generate_text_matches_oracle(gpu, tmp_path):
    from oracle import decoder as odec
    from cortexsdr_amd.decoder import DecoderSpec, synthetic_weights

    spec = DecoderSpec(2, 128, 2, 1, 64, 192, 300, 64)
    w = synthetic_weights(spec, n_atoms=128, nnz=8, seed=21, sigma=0.1, norm_jitter=0.1)
    path = str(tmp_path / "dec.sdr")
    formats.write_sdr(path, formats.decoder_entries(w))
    eng = InferenceEngine(path)
    try:
        prompt = [5, 17, 250, 3, 99, 42]
        toks = eng.generate(prompt, 8)
        st = eng.stats()
        assert st["prompt_tokens"] == 6 and st["generated_tokens"] == 8
        assert len(toks) == 8
        _, scores = odec.generate(w, prompt, 8, 0.8, 1.5, forced=np.array(toks, np.int32))
        for i, lg in enumerate(scores):
            pen = lg / np.float32(0.8)
            pen[np.asarray(toks[:i], np.int64)] -= 1.5
            top = np.sort(pen)[-2:]
            if top[1] - top[0] > 2e-3 * max(1.0, abs(top[1])):
                assert toks[i] == int(np.argmax(pen)), f"step {i}"
        assert eng.generate(prompt, 8) == toks                # deterministic, state reset
        with pytest.raises(EngineError):
            eng.generate([1, 2, 300], 2)                      # id beyond the vocabulary
    finally:
        eng.close()


def test_run_chains_linear_layers(gpu, tmp_path):
    """cortex_inference_engine_run (SDRInferenceEngine::run -> runLayersOnDemand): the
    archive's weight segments in getExecutionOrder's order (layer_index first, then names),
    each output the next input: a strategy-5 layer (no bias, the reference's HSDR stub), an
    fp32 layer plus its .bias segment, a Q4_K layer; a token embedding is skipped. Checked
    against the oracle layer by layer; a chain with a mismatched width and one with a non-linear
    segment are refused."""
    hs = synth.hsdb_layer(128, 256, 64, 4, seed_dict=5, seed_codes=6)
    rng = np.random.default_rng(3)
    dense = (rng.standard_normal((256, 128)) * 0.05).astype(np.float32)
    bias = rng.standard_normal(256).astype(np.float32)
    q4e, q4 = q4k_entry("head.weight", 48, 256, 12)
    q4e.layer_name, q4e.layer_index = "head", 2
    ents = [
        q4e,
        formats.SdrEntry(name="mid.weight", payload=dense.tobytes(), dims=(256, 128),
                         layer_name="mid", layer_index=1),
        formats.SdrEntry(name="mid.bias", payload=bias.tobytes(), dims=(256,),
                         layer_name="mid", layer_index=1),
        formats.hsdb_entry("first.weight", hs, layer_name="first", layer_index=0),
        formats.hsdb_entry("token_embd.weight", hs, original_type=13),
    ]
    path = str(tmp_path / "chain.sdr")
    formats.write_sdr(path, ents)
    eng = InferenceEngine(path)
    try:
        for M in (1, 3):
            x = rng.standard_normal((M, 256)).astype(np.float32)
            y = eng.run(x).reshape(M, 48)
            h1 = oracle.hsdb_matmul(hs, x.T.copy()).T
            h2 = h1 @ dense.T + bias[None, :]
            ref = oracle.q4k_linear(q4, 48, 256, h2.astype(np.float32))
            # batches through the matrix-core HSDB product (fp16 weights): the path's 1e-3
            assert rel_l2(y, ref) < (1e-5 if M == 1 else 1e-3), M
            st = eng.stats()
            assert [l["name"] for l in st["layers"]] == ["first", "mid", "head"]
            assert [l["path"] for l in st["layers"]] == ["hsdb", "dense_f32", "q4_k"]
        with pytest.raises(EngineError):
            eng.run(np.ones(100, np.float32))        # not a multiple of the first layer's width
    finally:
        eng.close()
    # a layer-norm vector in the chain is not a linear layer of the device path
    path2 = str(tmp_path / "chain2.sdr")
    formats.write_sdr(path2, [formats.hsdb_entry("first.weight", hs, layer_name="first"),
                              formats.vector_entry("norm.weight", np.ones(128, np.float32))])
    eng = InferenceEngine(path2)
    try:
        with pytest.raises(EngineError) as ei:
            eng.run(np.ones(256, np.float32))
        assert ei.value.code == -4
    finally:
        eng.close()
