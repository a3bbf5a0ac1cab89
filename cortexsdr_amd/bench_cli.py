"""Bench CLI for the compressed-weight path: every BASELINE.json configuration on one GPU.

    python -m cortexsdr_amd.bench_cli [--configs cfg1,cfg2,cfg3,gguf,cfg4,cfg5,strategy5]
        [--steps 50] [--out f.json]
    python -m cortexsdr_amd.bench_cli --suite suite.json [--out summary.json]

The role of the reference's `cortexsdr_bench` suite runner (src/cortexsdr_bench.cpp:52-79,
160-181: run each workload, collect times, write a summary JSON), for the device path:
each workload is timed as `steps` calls captured in a HIP graph and replayed between two HIP
events, inputs resident in HBM, over rotating weight copies larger than the 256 MiB
Infinity Cache. Reported per workload: microseconds per call, algorithmic GB/s (compressed
weights + dictionary + x + y, each once), the fraction of the 8 TB/s HBM peak and, for the
batched cases, dense-equivalent TFLOP/s (2*R*C*M per call).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import sys
import time

import numpy as np

from . import synth

HBM_PEAK = 8.0e12
MALL = 256 * 1024 * 1024


def _copies(nbytes: int, cap: int = 24) -> int:
    return max(2, min(cap, math.ceil(3 * MALL / max(1, nbytes)) + 1))


def time_graph(torch, fn, n_copies: int, steps: int) -> float:
    """Microseconds per call of fn(i) (i = copy index), `steps` calls in one graph replay."""
    for i in range(3):
        fn(i % n_copies)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            fn(i % n_copies)
    g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    best = float("inf")
    for _ in range(3):
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e3 / steps)
    return best


def bench_hsdb(torch, R, Cc, K, s, M, xdtype, steps, seed=2):
    from . import _lib
    from .hsdr import HsdbSegment, group_workspace

    stream = synth.hsdb_layer(R, Cc, K, s, seed_dict=1, seed_codes=seed)
    codes = R * (Cc // 64) * s * 4
    ncp = _copies(codes)
    segs = [HsdbSegment(stream) for _ in range(ncp)]
    x = torch.from_numpy(synth.activations(Cc, M, seed=3, dtype=xdtype)).cuda()
    y = torch.empty((R, M), dtype=torch.float32, device="cuda")
    ws = group_workspace([segs[0]], M)
    lib = _lib.load()
    xt = 1 if xdtype == np.float16 else 0
    xp = (C.c_void_p * 1)(x.data_ptr())
    yp = (C.c_void_p * 1)(y.data_ptr())
    hs = [(C.c_void_p * 1)(sg._h.value) for sg in segs]

    def fn(i):
        sp = int(torch.cuda.current_stream().cuda_stream)
        _lib.check(lib.csdr_hsdb_matmul_group(1, hs[i], xp, xt, M, yp, ws.data_ptr(),
                                              ws.numel(), sp))

    us = time_graph(torch, fn, ncp, steps)
    alg = codes + K * 64 * 4 + Cc * M * np.dtype(xdtype).itemsize + R * M * 4
    for sg in segs:
        sg.free()
    return {"R": R, "C": Cc, "K": K, "nnz": s, "M": M, "us": round(us, 3),
            "GBps": round(alg / us / 1e3, 1), "hbm_frac": round(alg / us / 1e-6 / HBM_PEAK, 4),
            "dense_equiv_TFLOPs": round(2.0 * R * Cc * M / us / 1e6, 2), "copies": ncp}


STRATEGY5_SHAPES = (("attn 896x896", 896, 896, 256, 3, 5), ("mlp 4864x896", 4864, 896, 512, 3, 8))


def strategy5_stream(R, Cc, K, S, k, seed=9):
    """An HSDR v2 stream in the reference's own strategy-5 geometry (one tile per row,
    tile_cols = C, a K x C dictionary; configFor's 1-row mode, HierarchicalSDRStrategy.cpp:
    1024-1062) from this package's encoder with no refinement passes."""
    from . import encode

    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((R, Cc)) * 0.02).astype(np.float32)
    return encode.compress(w, 1, Cc, K, S, k, ksvd_iters=0)


def strategy5_alg_bytes(R, Cc, K, S, k, M):
    """The stream's own bytes a product reads and writes: u16 codes, the fp32 dictionary, x
    (fp32) and y."""
    return R * S * k * 2 + K * Cc * 4 + Cc * M * 4 + R * M * 4


def bench_strategy5(torch, steps, Ms=(1, 8)):
    """matmulRowMajor on the reference's strategy-5 geometry (HK3): Qwen2-0.5B-shaped attention
    (K = 256, 3 x 5 picks) and MLP (K = 512, 3 x 8) matrices, x fp32 feature-major."""
    from .hsdr import HsdbSegment

    out = []
    for name, R, Cc, K, S, k in STRATEGY5_SHAPES:
        stream = strategy5_stream(R, Cc, K, S, k)
        for M in Ms:
            seg = HsdbSegment(stream)
            x = torch.from_numpy(synth.activations(Cc, M, seed=3)).cuda()
            ws = seg.workspace(M)
            y = seg.matmul(x, workspace=ws)

            def fn(i, seg=seg, x=x, y=y, ws=ws):
                seg.matmul(x, out=y, workspace=ws)

            us = time_graph(torch, fn, 1, steps)
            alg = strategy5_alg_bytes(R, Cc, K, S, k, M)
            out.append({"matrix": name, "R": R, "C": Cc, "K": K, "slots": S * k, "M": M,
                        "us": round(us, 3), "GBps": round(alg / us / 1e3, 1),
                        "hbm_frac": round(alg / us / 1e-6 / HBM_PEAK, 4)})
            seg.free()
    return out


def bench_hsdb_layers(torch, R, Cc, K, s, G, xdtype, steps, seed=2):
    """G independent layers of one shape in one grouped call (csdr_hsdb_matmul_group, one dx
    and one gather launch for all G): microseconds per call and per layer."""
    from . import _lib
    from .hsdr import HsdbSegment, group_workspace

    streams = [synth.hsdb_layer(R, Cc, K, s, seed_dict=1, seed_codes=seed + g) for g in range(G)]
    codes = R * (Cc // 64) * s * 4
    ncp = max(2, _copies(codes * G))
    segs = [[HsdbSegment(st) for st in streams] for _ in range(ncp)]
    xs = [torch.from_numpy(synth.activations(Cc, 1, seed=3 + g, dtype=xdtype)).cuda()
          for g in range(G)]
    ys = [torch.empty((R, 1), dtype=torch.float32, device="cuda") for _ in range(G)]
    ws = group_workspace(segs[0], 1)
    lib = _lib.load()
    xt = 1 if xdtype == np.float16 else 0
    xp = (C.c_void_p * G)(*[x.data_ptr() for x in xs])
    yp = (C.c_void_p * G)(*[y.data_ptr() for y in ys])
    hs = [(C.c_void_p * G)(*[sg._h.value for sg in cp]) for cp in segs]

    def fn(i):
        sp = int(torch.cuda.current_stream().cuda_stream)
        _lib.check(lib.csdr_hsdb_matmul_group(G, hs[i], xp, xt, 1, yp, ws.data_ptr(),
                                              ws.numel(), sp))

    us = time_graph(torch, fn, ncp, steps)
    alg = G * (codes + K * 64 * 4 + Cc * np.dtype(xdtype).itemsize + R * 4)
    for cp in segs:
        for sg in cp:
            sg.free()
    return {"R": R, "C": Cc, "K": K, "nnz": s, "layers": G, "us": round(us, 3),
            "us_per_layer": round(us / G, 3), "GBps": round(alg / us / 1e3, 1),
            "hbm_frac": round(alg / us / 1e-6 / HBM_PEAK, 4), "copies": ncp}


def bench_q4k(torch, R, Cc, M, steps, order=0):
    from . import _lib, q4k

    blob = synth.q4k_matrix(R, Cc, seed=7)
    ncp = _copies(len(blob))
    ws = [q4k.upload(blob) for _ in range(ncp)]
    x = torch.from_numpy(synth.activations(Cc, M, seed=11).T.copy().astype(np.float16)).cuda()
    y = torch.empty((M, R), dtype=torch.float32, device="cuda")
    lib = _lib.load()

    def fn(i):
        sp = int(torch.cuda.current_stream().cuda_stream)
        _lib.check(lib.csdr_q4k_linear(ws[i].data_ptr(), R, Cc, order, x.data_ptr(), 1, M,
                                       y.data_ptr(), sp))

    us = time_graph(torch, fn, ncp, steps)
    alg = len(blob) + Cc * M * 2 + R * M * 4
    return {"R": R, "C": Cc, "M": M, "us": round(us, 3), "GBps": round(alg / us / 1e3, 1),
            "hbm_frac": round(alg / us / 1e-6 / HBM_PEAK, 4),
            "dense_equiv_TFLOPs": round(2.0 * R * Cc * M / us / 1e6, 2), "copies": ncp}


def gguf_matrix(fmt: int, R: int, Cc: int, seed: int) -> bytes:
    """Random blocks of a GGUF format with fp16 scales ~U(0.001, 0.05) (q6_k's at byte 208,
    q8_1's fp32), like synth.q4k_matrix for Q4_K."""
    from . import gguf

    bb, be = gguf.block(fmt)
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (R * Cc // be, bb), dtype=np.uint8)
    off = 208 if fmt == 14 else 0
    b[:, off:off + 2] = rng.uniform(0.001, 0.05, b.shape[0]).astype(np.float16).view(
        np.uint8).reshape(-1, 2)
    return b.tobytes()


def bench_gguf(torch, fmt_name, R, Cc, M, steps):
    """The engine's other GGUF formats at cfg3's shapes (csdr_gguf_linear)."""
    from . import _lib, gguf

    fmt = gguf.format_id(fmt_name)
    blob = gguf_matrix(fmt, R, Cc, seed=7)
    ncp = _copies(len(blob))
    ws = [gguf.upload(blob) for _ in range(ncp)]
    x = torch.from_numpy(synth.activations(Cc, M, seed=11).T.copy().astype(np.float16)).cuda()
    y = torch.empty((M, R), dtype=torch.float32, device="cuda")
    lib = _lib.load()

    def fn(i):
        sp = int(torch.cuda.current_stream().cuda_stream)
        _lib.check(lib.csdr_gguf_linear(ws[i].data_ptr(), fmt, R, Cc, x.data_ptr(), 1, M,
                                        y.data_ptr(), sp))

    us = time_graph(torch, fn, ncp, steps)
    alg = len(blob) + Cc * M * 2 + R * M * 4
    return {"format": fmt_name, "R": R, "C": Cc, "M": M, "us": round(us, 3),
            "GBps": round(alg / us / 1e3, 1), "hbm_frac": round(alg / us / 1e-6 / HBM_PEAK, 4),
            "dense_equiv_TFLOPs": round(2.0 * R * Cc * M / us / 1e6, 2), "copies": ncp}


def cfg4_workload(n_prompt=512, seed=0):
    """Config 4's model and prompt: the Qwen2-0.5B-shaped decoder with every linear
    HSDB-coded against one shared 1024 x 64 dictionary (8 nnz per block) and a prompt of
    n_prompt uniform random token ids. bench.py, this CLI and the GPU parity test of the
    benchmarked run share it."""
    from .decoder import QWEN2_0_5B, synthetic_weights

    w = synthetic_weights(QWEN2_0_5B, seed=seed)
    prompt = (synth.uniform(seed + 77, n_prompt, stream=61) * QWEN2_0_5B.vocab).astype(np.int32)
    return w, prompt


def cfg4_run(dec, prompt, n_new):
    """The benchmarked greedy run on a decoder: a warm-up over the first 8 prompt tokens
    (captures both step graphs), then the prompt (multi-token prefill, its last token through
    the step graph, which picks new token 1) and n_new - 1 decode steps in one call.
    Returns (prefill seconds, decode seconds, the n_new new tokens)."""
    dec.prefill(prompt[:8], 0.0, 0.0)
    dec.decode(8, 0.0, 0.0)
    t0 = time.perf_counter()
    dec.prefill(prompt, 0.0, 0.0)       # greedy: temperature 0 (scale 1), no penalty
    t_prefill = time.perf_counter() - t0
    t0 = time.perf_counter()
    dec.decode(n_new - 1, 0.0, 0.0)
    t_decode = time.perf_counter() - t0
    return t_prefill, t_decode, dec.tokens(len(prompt), n_new)


def bench_decoder(torch, n_prompt=512, n_new=128, seed=0):
    """Config 4: Qwen2-0.5B-shaped decoder, all linears HSDB-coded (1024 x 64 shared
    dictionary, 8 nnz per block), prompt of uniform random ids, greedy (plain argmax)."""
    from .decoder import QWEN2_0_5B, Decoder

    t0 = time.time()
    w, prompt = cfg4_workload(n_prompt, seed)
    t_build = time.time() - t0
    dec = Decoder(w)
    try:
        t_prefill, t_decode, toks = cfg4_run(dec, prompt, n_new)
        per_tok = t_decode / (n_new - 1)
        code = w.code_bytes()
        kv = 2 * QWEN2_0_5B.n_layers * QWEN2_0_5B.n_kv_heads * QWEN2_0_5B.head_dim * 4  # fp32 cache
        alg = code + kv * (n_prompt + n_new // 2)
        return {"n_prompt": n_prompt, "n_new": n_new,
                "decode_tokens_per_s": round(1.0 / per_tok, 1),
                "ms_per_token": round(per_tok * 1e3, 4),
                "prefill_tokens_per_s": round(n_prompt / t_prefill, 1),
                "code_MB_per_token": round(code / 1e6, 2),
                "alg_GBps": round(alg / per_tok / 1e9, 1),
                "hbm_frac": round(alg / per_tok / HBM_PEAK, 4),
                "device_MB": round(dec.device_bytes() / 1e6, 1),
                "host_build_s": round(t_build, 1), "first_tokens": toks[:8].tolist()}
    finally:
        dec.close()


def cfg5_weights(max_ctx: int, seed: int = 5):
    """Config 5's model: Llama-7B shape (32 layers, hidden 4096, 32 heads of 128, SwiGLU
    11008, vocab 32000, fp16 K/V cache), every linear HSDB-coded (1024 x 64 dictionary, 8 nnz
    per block). Two distinct coded layers are generated and used 16 times each (the decoder
    loads a device copy per layer, so a step still streams 32 layers' codes)."""
    import dataclasses

    from .decoder import DecoderSpec, DecoderWeights, synthetic_weights

    spec = DecoderSpec(32, 4096, 32, 32, 128, 11008, 32000, max_ctx, kv_dtype="f16")
    w2 = synthetic_weights(dataclasses.replace(spec, n_layers=2), seed=seed)
    return DecoderWeights(spec, [w2.layers[l % 2] for l in range(32)], w2.lm_head,
                          w2.final_norm)


def bench_decoder_7b(torch, ctx=4096, steps=16, seed=5, batch=1, stream_layers=False,
                     prefetch=True):
    """Config 5: Llama-7B-shaped decode step (32 layers, hidden 4096, 32 heads of 128, SwiGLU
    11008, vocab 32000, all linears HSDB-coded: 1024 x 64 dictionary, 8 nnz per block) at
    context `ctx` with the fp16 KV cache (as configs[4] states) filled with N(0,1), `batch`
    sequences, weights resident.
    Two distinct coded layers are generated and loaded 16 times each: every layer has its own
    device copy, so HBM traffic per step is that of 32 distinct layers."""
    from .decoder import Decoder

    t0 = time.time()
    w = cfg5_weights(ctx + steps + 8, seed)
    spec = w.spec
    t_build = time.time() - t0
    dec = Decoder(w, batch=batch, stream_layers=stream_layers, prefetch=prefetch)
    try:
        for l in range(spec.n_layers):
            k = torch.randn((batch, ctx, spec.n_kv_heads, spec.head_dim), device="cuda").half()
            v = torch.randn((batch, ctx, spec.n_kv_heads, spec.head_dim), device="cuda").half()
            dec.load_kv(l, k, v, ctx)
            del k, v
        torch.cuda.synchronize()
        dec.set_position(ctx, 1)
        dec.decode(3, 0.0, 0.0)                      # captures the step graph
        dec.set_position(ctx, 1)
        t0 = time.perf_counter()
        dec.decode(steps, 0.0, 0.0)
        dt = (time.perf_counter() - t0) / steps
        code = w.code_bytes()
        kv = 2 * spec.n_layers * (ctx + steps // 2) * spec.n_kv_heads * spec.head_dim * 2 * batch
        return {"layers": 32, "hidden": 4096, "heads": 32, "head_dim": 128, "ffn": 11008,
                "vocab": 32000, "context": ctx, "batch": batch, "steps": steps,
                "ms_per_step": round(dt * 1e3, 3), "tokens_per_s": round(batch / dt, 1),
                "code_GB_per_step": round(code / 1e9, 3), "kv_GB_per_step": round(kv / 1e9, 3),
                "alg_GBps": round((code + kv) / dt / 1e9, 1),
                "hbm_frac": round((code + kv) / dt / HBM_PEAK, 4),
                "device_GB": round(dec.device_bytes() / 1e9, 2),
                "host_build_s": round(t_build, 1),
                **({"streamed": True, "prefetch": bool(prefetch),
                    "streamed_GB_per_step": round(dec.streamed_bytes() / 1e9, 3),
                    "pcie_GBps": round(dec.streamed_bytes() / dt / 1e9, 2)}
                   if stream_layers else {})}
    finally:
        dec.close()


def _percentile(v, q):
    """Linear-interpolated percentile of the sorted samples (cortexsdr_bench.cpp:160-181)."""
    v = sorted(v)
    if not v:
        return None
    pos = (len(v) - 1) * q / 100.0
    lo = int(pos)
    hi = min(lo + 1, len(v) - 1)
    return v[lo] + (v[hi] - v[lo]) * (pos - lo)


def run_suite(path: str) -> dict:
    """The reference bench suite runner's inference leg (cortexsdr_bench.cpp:52-79,
    435-462) over a suite JSON of the reference's shape: "repeats", "warmup_runs",
    "binaries.text_cli" (default: this package's cortexsdr_text_cli) and "tests" entries
    with "sdr_path", "prompt" (token ids here), "max_length", "run_inference". Each run
    spawns the text CLI with --profile and records wall time and the profile."""
    import os
    import subprocess
    import tempfile

    with open(path) as f:
        suite = json.load(f)
    root = suite.get("project_root", ".")
    here = os.path.dirname(os.path.abspath(__file__))
    cli = suite.get("binaries", {}).get("text_cli") or os.path.join(here, "bin",
                                                                      "cortexsdr_text_cli")
    if not os.path.isabs(cli) and not os.path.exists(cli):
        cli = os.path.join(root, cli)
    repeats = int(suite.get("repeats", 1))
    warm = int(suite.get("warmup_runs", 0))
    out = {"suite": path, "text_cli": cli, "tests": []}
    for t in suite.get("tests", []):
        if not t.get("run_inference", True):
            continue
        sdr = t["sdr_path"] if os.path.isabs(t["sdr_path"]) else os.path.join(root, t["sdr_path"])
        runs = []
        for i in range(warm + repeats):
            with tempfile.TemporaryDirectory() as td:
                prof = os.path.join(td, "profile.json")
                cmd = [cli, "-p", str(t["prompt"]), "-m", str(t.get("max_length", 64)),
                       "--profile", prof, sdr]
                t0 = time.perf_counter()
                r = subprocess.run(cmd, capture_output=True, text=True)
                ms = (time.perf_counter() - t0) * 1e3
                rec = {"exit_code": r.returncode, "elapsed_ms_wall": round(ms, 3),
                       "command": " ".join(cmd)}
                if os.path.exists(prof):
                    with open(prof) as pf:
                        rec["profile"] = json.load(pf)
                    tps = rec["profile"].get("tokens_per_sec")
                    if tps is not None:
                        rec["tokens_per_min"] = tps * 60.0
                elif r.returncode:
                    rec["stderr"] = r.stderr[-2000:]
            if i >= warm:
                runs.append(rec)
        walls = [r["elapsed_ms_wall"] for r in runs if r["exit_code"] == 0]
        tps = [r["profile"]["tokens_per_sec"] for r in runs
               if r["exit_code"] == 0 and "profile" in r]
        out["tests"].append({
            "name": t.get("name", sdr), "runs": runs,
            "wall_ms_p50": _percentile(walls, 50), "wall_ms_p95": _percentile(walls, 95),
            "tokens_per_sec_p50": _percentile(tps, 50), "tokens_per_sec_p95": _percentile(tps, 95),
            "ok": all(r["exit_code"] == 0 for r in runs),
        })
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--configs", default="cfg1,cfg2,cfg3,cfg4")
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--out", default=None)
    ap.add_argument("--cfg2-batches", default="1,16,64,256")
    ap.add_argument("--cfg5-batches", default="1,8")
    ap.add_argument("--cfg5-stream", action="store_true",
                    help="cfg5 also with on-demand layer streaming (host-resident blocks)")
    ap.add_argument("--suite", default=None, help="run a bench suite JSON through the text CLI")
    args = ap.parse_args(argv)
    if args.suite:
        res = run_suite(args.suite)
        text = json.dumps(res)
        print(text, flush=True)
        if args.out:
            with open(args.out, "w") as f:
                f.write(text + "\n")
        return 0 if all(t["ok"] for t in res["tests"]) else 1
    import torch

    if not torch.cuda.is_available():
        print("bench_cli: no HIP device", file=sys.stderr)
        return 1
    cfgs = set(args.configs.split(","))
    res = {"device": torch.cuda.get_device_name(0), "steps": args.steps, "results": {}}
    t0 = time.time()
    if "cfg1" in cfgs:
        res["results"]["cfg1"] = [bench_hsdb(torch, 4096, 4096, 512, 4, 1, np.float32,
                                             args.steps),
                                  bench_hsdb_layers(torch, 4096, 4096, 512, 4, 8, np.float32,
                                                    args.steps)]
    if "cfg2" in cfgs:
        ms = [int(v) for v in args.cfg2_batches.split(",")]
        out = []
        for (R, Cc) in ((4096, 11008), (11008, 4096)):
            for M in ms:
                out.append(bench_hsdb(torch, R, Cc, 1024, 8, M, np.float16, args.steps))
                print(json.dumps(out[-1]), flush=True)
        res["results"]["cfg2"] = out
    if "cfg3" in cfgs:
        out = []
        for (R, Cc) in ((4096, 4096), (4096, 14336)):
            for M in (1, 32):
                out.append(bench_q4k(torch, R, Cc, M, args.steps))
                print(json.dumps(out[-1]), flush=True)
        res["results"]["cfg3"] = out
    if "gguf" in cfgs:  # the engine's other block formats at cfg3's shapes
        out = []
        for fmt in ("q6_k", "q8_0", "q4_0", "q5_k"):
            for (R, Cc) in ((4096, 4096), (4096, 14336)):
                for M in (1, 32):
                    out.append(bench_gguf(torch, fmt, R, Cc, M, args.steps))
                    print(json.dumps(out[-1]), flush=True)
        res["results"]["gguf"] = out
    if "strategy5" in cfgs:  # the reference's own strategy-5 geometry (HK3)
        res["results"]["strategy5"] = bench_strategy5(torch, args.steps)
        for r in res["results"]["strategy5"]:
            print(json.dumps(r), flush=True)
    if "cfg5" in cfgs:
        out = []
        for B in (int(v) for v in args.cfg5_batches.split(",")):
            out.append(bench_decoder_7b(torch, batch=B))
            print(json.dumps(out[-1]), flush=True)
            torch.cuda.empty_cache()
            if args.cfg5_stream:
                for pf in (True, False):
                    out.append(bench_decoder_7b(torch, batch=B, stream_layers=True, prefetch=pf))
                    print(json.dumps(out[-1]), flush=True)
                    torch.cuda.empty_cache()
        res["results"]["cfg5"] = out
    if "cfg4" in cfgs:
        res["results"]["cfg4"] = bench_decoder(torch)
        print(json.dumps(res["results"]["cfg4"]), flush=True)
    res["wall_s"] = round(time.time() - t0, 1)
    text = json.dumps(res)
    print(text, flush=True)
    if args.out:
        with open(args.out, "w") as f:
            f.write(text + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
