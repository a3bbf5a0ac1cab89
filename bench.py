#!/usr/bin/env python3
"""Benchmark of the compressed-weight inference hot path on one MI355X.

Headline (BASELINE.json metric "fused decode-GEMV HBM GB/s"): configs[1] at M = 1, i.e.
one step = Y_a = W_a . x_a and Y_b = W_b . x_b for the two dictionary-coded matrices
W_a 4096 x 11008 and W_b 11008 x 4096 (1 x 64 blocks, shared-format dictionary of
1024 unit-norm fp32 atoms, 8 nonzeros per block, fp16 coefficients, x fp16, fp32
accumulation). value = algorithmic bytes of a step / step time, where algorithmic bytes
= compressed codes + dictionary + x + y of both matrices, each counted once.

Inputs are resident in HBM before timing. Each step uses a different copy of the coded
matrices (a rotation over > 3 x 256 MiB) so the Infinity Cache cannot serve them.

Timing: the K steps are captured once into a HIP graph; the timed region is one replay
(exactly K steps, bracketed by synchronize) and gives `value` / `ms_per_step`; `replays`
adds the median, min and max per-step time over 100 further replays of the same graph,
each bracketed by HIP events.

The JSON line carries:
  roofline      the dominant kernel (the gather launch over both matrices): median over 100
                replays of a graph of K back-to-back gather launches, HIP events on the
                launch stream; `traffic` = HBM bytes per launch from the committed rocprofv3
                --pmc measurement (profiles/hsdb_gather_cfg2_traffic.json), null unless it
                was made from the kernel sources in this tree
  cpu_baseline  the CPU restatement of the reference algorithm (oracle/, OpenMP) on a
                bounded sample of the same workload, on this host's cores, with the CPU
                model, its physical cores and a single-thread time (the reference's fused
                path is single-threaded)
  decode        the metric's second half, configs[3]: Qwen2-0.5B-shaped decoder (24 layers,
                hidden 896, 14/2 heads of 64, FFN 4864, vocab 151936, every linear
                HSDB-coded against one shared 1024 x 64 dictionary), 512-token prompt of
                uniform random ids, then greedy decode of 128 tokens; tokens/s of the decode
                phase next to a KV-cached CPU decode step of the same model (oracle/)
  decode_7b     configs[4]: the Llama-7B-shaped decode step (32 layers, hidden 4096, 32 heads
                of 128, SwiGLU 11008, vocab 32000, HSDB-coded linears) over an fp16 KV
                context of 4096 positions, batch 1 and 8, weights and KV resident
  decode_7b_streaming  the same step with on-demand layer streaming: blocks in pinned host
                memory, copied to the device per step (prefetch on at batch 1 and 8, off at
                batch 1), ms per step and the host-to-device GB/s of the streamed codes
  cfg1          configs[0] (the reference CPU path's configuration): W 4096x4096, K=512, 4
                nnz, x fp32, M=1, one matrix and 8 layers per call, next to the CPU
                restatement (OpenMP and one thread)
  cfg3          configs[2]: Q4_K 4096x4096 / 4096x14336 at M = 1 and 32, next to the
                reference engine's dequantize + fp32 linear restated on the CPU
  encode        the compress side: GPU matching pursuit (rows/s, TFLOP/s against the fp32
                vector peak) and compress wall time on Qwen2-0.5B-shaped attention / MLP
                matrices, next to the reference's own compress (oracle/_ref)
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 * 1024 * 1024

# HBM bytes per gather launch (cfg2, M = 1, both matrices): two rocprofv3 --pmc runs of this
# script (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each scaled by what the same counter
# reads for a plain 256 MiB device copy in the same run (--calibrate-copy), written by
# cortexsdr_amd/traffic.py with the digest of the kernel's sources; reported only when that
# digest is the current tree's (a measurement of an older kernel is not this kernel's).
TRAFFIC_JSON = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "hsdb_gather_cfg2_traffic.json")


def gather_traffic():
    """(bytes per launch, the measurement's record) from the committed PMC measurement of the
    current sources, or (None, reason)."""
    from cortexsdr_amd import traffic

    t, why = traffic.load_current(TRAFFIC_JSON)
    if t is None:
        return None, why
    return int(t["traffic_bytes"]), t


def cpu_info():
    """CPU model name, physical cores (distinct (package, core) pairs) and logical CPUs."""
    model, pairs, logical = None, set(), 0
    phys = core = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "processor":
                    logical += 1
                elif k == "model name" and model is None:
                    model = v
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    core = v
                elif not k and phys is not None:
                    pairs.add((phys, core))
                    phys = core = None
        if phys is not None:
            pairs.add((phys, core))
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count()
    return {"cpu_model": model, "physical_cores": len(pairs) or None,
            "logical_cpus": logical or os.cpu_count(), "usable_cpus": usable}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--config", default="cfg2", choices=["cfg1", "cfg2"])
    ap.add_argument("--no-decode", action="store_true", help="skip the config-4 decode leg")
    ap.add_argument("--decode-cpu-seconds", type=float, default=5.0)
    ap.add_argument("--no-encode", action="store_true", help="skip the HSDR encoder leg")
    ap.add_argument("--no-7b", action="store_true", help="skip the config-5 decode-step leg")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the config-1 and config-3 legs")
    ap.add_argument("--replays", type=int, default=100,
                    help="graph replays for the median / min / max statistics")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 256 MiB device copy 5 times (the reference dispatch "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    return ap.parse_args()


def workloads(cfg: str):
    if cfg == "cfg1":
        return [dict(name="W 4096x4096", R=4096, C=4096, K=512, s=4, xdtype=np.float32)]
    return [
        dict(name="W 4096x11008", R=4096, C=11008, K=1024, s=8, xdtype=np.float16),
        dict(name="W 11008x4096", R=11008, C=4096, K=1024, s=8, xdtype=np.float16),
    ]


def alg_bytes(w, M=1):
    NB = w["C"] // 64
    codes = w["R"] * NB * w["s"] * 4
    dict_b = w["K"] * 64 * 4
    xb = w["C"] * M * np.dtype(w["xdtype"]).itemsize
    yb = w["R"] * M * 4
    P = NB * w["K"] * M * 4
    return dict(op=codes + dict_b + xb + yb, gather=codes + P + yb, codes=codes)


def cpu_baseline(streams, xs, seconds, threads=None):
    """Seconds per step of the CPU restatement, `threads` OpenMP threads (default: the
    OMP_NUM_THREADS / CPU count the run was given)."""
    import oracle

    if threads is None:
        threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count()
    prev = oracle.set_threads(threads)
    try:
        xs32 = [x.astype(np.float32) for x in xs]
        for s, x in zip(streams, xs32):  # warm-up
            oracle.hsdb_matmul(s, x)
        n = 0
        t0 = time.perf_counter()
        while True:
            for s, x in zip(streams, xs32):
                oracle.hsdb_matmul(s, x)
            n += 1
            if time.perf_counter() - t0 >= seconds and n >= 2:
                break
        dt = (time.perf_counter() - t0) / n
    finally:
        oracle.set_threads(prev)
    return dt, n, threads


def cpu_decode_step(w, ctx: int, seconds: float):
    """Seconds per KV-cached decode step of the same model on the CPU restatement (oracle/):
    per layer RMSNorm, the seven HSDB linears (orc_hsdb_matmul, OpenMP), RoPE, GQA attention
    over `ctx` fp16 cached positions, SwiGLU; then output norm, lm_head scores, argmax."""
    import oracle

    s = w.spec
    rng = np.random.default_rng(0)
    kc = rng.standard_normal((1, ctx, s.n_kv_heads, s.head_dim)).astype(np.float16)
    vc = rng.standard_normal((1, ctx, s.n_kv_heads, s.head_dim)).astype(np.float16)
    kc, vc = kc.view(np.uint16), vc.view(np.uint16)
    lens = np.array([ctx], np.int32)
    x0 = rng.standard_normal(s.hidden).astype(np.float32)

    def one():
        x = x0.copy()
        for L in w.layers:
            h = oracle.rms_norm(x, L["attn_norm"]).reshape(-1, 1)
            q = oracle.hsdb_matmul(L["q"], h)[:, 0]
            k = oracle.hsdb_matmul(L["k"], h)[:, 0]
            oracle.hsdb_matmul(L["v"], h)
            q = oracle.rope(q, s.n_heads, s.head_dim, s.rope_theta, ctx - 1)
            oracle.rope(k, s.n_kv_heads, s.head_dim, s.rope_theta, ctx - 1)
            a = oracle.attn_decode(q.reshape(1, s.n_heads, s.head_dim), kc, vc, lens,
                                   s.n_heads, s.n_kv_heads, s.head_dim)
            x = x + oracle.hsdb_matmul(L["o"], a.reshape(-1, 1))[:, 0]
            h = oracle.rms_norm(x, L["ffn_norm"]).reshape(-1, 1)
            f = oracle.silu_mul(oracle.hsdb_matmul(L["gate"], h), oracle.hsdb_matmul(L["up"], h))
            x = x + oracle.hsdb_matmul(L["down"], f)[:, 0]
        h = oracle.rms_norm(x, w.final_norm).reshape(-1, 1)
        oracle.select_best(oracle.hsdb_matmul(w.lm_head, h)[:, 0], None, 0.0, 0.0)

    one()
    n, t0 = 0, time.perf_counter()
    while True:
        one()
        n += 1
        if time.perf_counter() - t0 >= seconds and n >= 2:
            break
    return (time.perf_counter() - t0) / n, n


def _threads():
    return int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count()


def _cpu_time(fn, seconds, min_runs=2):
    """Seconds per call of fn after one warm-up call: at least min_runs calls and `seconds`."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        if time.perf_counter() - t0 >= seconds and n >= min_runs:
            break
    return (time.perf_counter() - t0) / n, n


def cfg1_leg(torch, args):
    """configs[0], the configuration the reference CPU path runs: W 4096x4096 (64-blocks,
    K=512 unit-norm fp32 atoms, 4 nnz, fp16 coefficients), x fp32, M=1. GPU: one matrix per
    call, and 8 independent layers per grouped call (bench_cli); CPU: the restated fused
    product (oracle orc_hsdb_matmul) on the same matrix and x, OpenMP and one thread."""
    from cortexsdr_amd import bench_cli, synth

    one = bench_cli.bench_hsdb(torch, 4096, 4096, 512, 4, 1, np.float32, 50)
    eight = bench_cli.bench_hsdb_layers(torch, 4096, 4096, 512, 4, 8, np.float32, 50)
    alg = 4096 * 64 * 4 * 4 + 512 * 64 * 4 + 4096 * 4 + 4096 * 4
    out = {"workload": "cfg1: W 4096x4096, K=512, 4 nnz/block, x fp32, M=1",
           "algorithmic_bytes": alg,
           "us_per_call": one["us"], "GBps": one["GBps"], "hbm_frac": one["hbm_frac"],
           "eight_layers_per_call": {"us_per_layer": eight["us_per_layer"],
                                     "GBps": eight["GBps"], "hbm_frac": eight["hbm_frac"]},
           "cpu_baseline": None}
    if not args.no_cpu:
        import oracle

        stream = synth.hsdb_layer(4096, 4096, 512, 4, seed_dict=1, seed_codes=2)
        x = synth.activations(4096, 1, seed=3)
        th = _threads()
        prev = oracle.set_threads(th)
        try:
            dt, n = _cpu_time(lambda: oracle.hsdb_matmul(stream, x), args.cpu_seconds / 2)
            oracle.set_threads(1)
            dt1, n1 = _cpu_time(lambda: oracle.hsdb_matmul(stream, x), args.cpu_seconds / 4)
        finally:
            oracle.set_threads(prev)
        out["cpu_baseline"] = {
            "value": round(alg / dt / 1e9, 3), "unit": "GB/s", "cores": th, "kind": "port",
            "sample": f"{n} products of the same matrix and x through oracle/csdr_oracle.c "
                      f"orc_hsdb_matmul, {th} OpenMP threads, {dt * 1e3:.2f} ms each",
            "single_thread": {"value": round(alg / dt1 / 1e9, 3), "unit": "GB/s", "cores": 1,
                              "sample": f"{n1} products on one thread, {dt1 * 1e3:.2f} ms each"}}
    return out


def strategy5_leg(torch, args):
    """The reference's own strategy-5 geometry (one tile per row, tile_cols = C, a K x C
    dictionary: what its compressor writes in 1-row mode, HierarchicalSDRStrategy.cpp:
    1024-1062): Qwen2-0.5B-shaped attention (896 x 896, K = 256, 3 x 5 picks) and MLP
    (4864 x 896, K = 512, 3 x 8) streams from this package's encoder, matmulRowMajor at M = 1
    and 8 (bench_cli.bench_strategy5). CPU: the restated matmulRowMajor (oracle
    orc_hsdr_matmul_row_major, one thread, as the reference's loop) on the same streams at
    M = 1."""
    from cortexsdr_amd import bench_cli, synth

    gpu = bench_cli.bench_strategy5(torch, 50, Ms=(1, 8))
    out = {"workload": "strategy-5 geometry (1-row tiles of C features), x fp32",
           "gpu": gpu, "cpu_baseline": None}
    if not args.no_cpu:
        import oracle

        rows = []
        for name, R, Cc, K, S, k in bench_cli.STRATEGY5_SHAPES:
            stream = bench_cli.strategy5_stream(R, Cc, K, S, k)
            x = synth.activations(Cc, 1, seed=3)
            dt, n = _cpu_time(lambda: oracle.hsdr_matmul_row_major(stream, x),
                              args.cpu_seconds / 4)
            alg = bench_cli.strategy5_alg_bytes(R, Cc, K, S, k, 1)
            rows.append({"matrix": name, "M": 1, "us": round(dt * 1e6, 1),
                         "GBps": round(alg / dt / 1e9, 3), "calls": n})
        out["cpu_baseline"] = {
            "value": rows[-1]["GBps"], "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": "the MLP stream at M=1 (and the attention stream, rows) through "
                      "oracle/csdr_oracle.c orc_hsdr_matmul_row_major on one thread",
            "rows": rows}
    return out


def cfg3_leg(torch, args):
    """Q4_K dequant-matmul, W 4096x4096 and 4096x14336, x fp16, M = 1 and 32
    (bench_cli.bench_q4k: ggml element order, HIP graph replays); CPU: the reference engine's
    path restated (oracle orc_q4k_linear: dequantize each row to fp32 as
    decodeSupportedGGUFQuantized does, then the fp32 row dot products of linear_forward),
    OpenMP, on the same matrix and x."""
    from cortexsdr_amd import bench_cli, synth

    rows = []
    for (R, Cc) in ((4096, 4096), (4096, 14336)):
        for M in (1, 32):
            r = bench_cli.bench_q4k(torch, R, Cc, M, 50)
            rows.append({k: r[k] for k in ("R", "C", "M", "us", "GBps", "hbm_frac",
                                           "dense_equiv_TFLOPs")})
    out = {"workload": "cfg3: Q4_K 4096x4096 / 4096x14336, x fp16, M=1/32", "gpu": rows,
           "cpu_baseline": None}
    if not args.no_cpu:
        import oracle

        th = _threads()
        prev = oracle.set_threads(th)
        cpu = []
        try:
            R, Cc = 4096, 14336
            blob = synth.q4k_matrix(R, Cc, seed=7)
            for M in (1, 32):
                x = synth.activations(Cc, M, seed=11).T.copy().astype(np.float16).astype(np.float32)
                dt, n = _cpu_time(lambda: oracle.q4k_linear(blob, R, Cc, x), args.cpu_seconds / 4)
                alg = len(blob) + Cc * M * 2 + R * M * 4
                cpu.append({"R": R, "C": Cc, "M": M, "us": round(dt * 1e6, 1),
                            "GBps": round(alg / dt / 1e9, 3), "calls": n})
        finally:
            oracle.set_threads(prev)
        out["cpu_baseline"] = {
            "value": cpu[0]["GBps"], "unit": "GB/s", "cores": th, "kind": "port",
            "sample": "W 4096x14336 at M=1 (and M=32 below) through oracle/csdr_oracle.c "
                      "orc_q4k_linear (per-row dequantize + fp32 dot), "
                      f"{th} OpenMP threads", "rows": cpu}
    return out


def decode_leg(args):
    """tokens/s of graph-replayed decode steps after a 512-token prefill."""
    from cortexsdr_amd import bench_cli
    from cortexsdr_amd.decoder import Decoder

    n_prompt, n_new = 512, 128
    # the workload and call sequence tests/test_full_depth_gpu.py checks against the oracle
    w, prompt = bench_cli.cfg4_workload(n_prompt, seed=0)
    dec = Decoder(w)
    try:
        t_pre, t_dec, toks = bench_cli.cfg4_run(dec, prompt, n_new)
    finally:
        dec.close()
    per_tok = t_dec / (n_new - 1)
    out = {
        "metric": "Qwen2-0.5B-shape decode tokens/sec",
        "value": round(1.0 / per_tok, 1),
        "unit": "tokens/s",
        "ms_per_token": round(per_tok * 1e3, 4),
        "prefill_tokens_per_s": round(n_prompt / t_pre, 1),
        "workload": "cfg4: 512-token prompt, greedy decode of 128 tokens, batch 1",
        "code_bytes_per_token": w.code_bytes(),
        "first_tokens": toks[:4].tolist(),
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        dt, n = cpu_decode_step(w, n_prompt + n_new // 2, args.decode_cpu_seconds)
        threads = _threads()
        out["cpu_baseline"] = {
            "value": round(1.0 / dt, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": (f"{n} KV-cached decode steps at context {n_prompt + n_new // 2} through "
                       f"oracle/ (orc_hsdb_matmul OpenMP linears), {dt * 1e3:.0f} ms/token")}
        out["cpu_full_recompute"] = cpu_recompute_steps(w, prompt, toks, args)
    return out


def cpu_recompute_steps(w, prompt, toks, args, steps=2):
    """The reference's own decode loop, labelled: run_transformer_decode recomputes the whole
    context for every generated token (api/cortex_sdk.cpp:1995-2006, 1543-1696) over weights
    decompressed to dense fp32 at load. Restated with the oracle (every weight decoded once,
    fp32 BLAS products, whole-context causal attention); `steps` tokens after the 512-token
    prompt, seconds per token (not extrapolated to the 128-token run)."""
    from oracle import decoder as odec

    th = _threads()
    t0 = time.perf_counter()
    dense = odec.DenseWeights()
    for L in w.layers:
        for name in ("q", "k", "v", "o", "gate", "up", "down"):
            dense.get(L[name])
    dense.get(w.lm_head)
    t_load = time.perf_counter() - t0
    per = []
    for i in range(steps):
        ctx = np.concatenate([prompt, toks[:i]]).astype(np.int32)
        t0 = time.perf_counter()
        odec.prompt_state(w, ctx, dense)
        per.append(time.perf_counter() - t0)
    dt = float(np.median(per))
    return {"value": round(1.0 / dt, 4), "unit": "tokens/s", "cores": th, "kind": "port",
            "sample": (f"{steps} tokens at context {len(prompt)}..{len(prompt) + steps - 1}, each "
                       f"recomputing the whole context (dense fp32 weights decoded once in "
                       f"{t_load:.1f} s, numpy BLAS products, OpenMP attention), "
                       f"{dt:.2f} s/token")}


def decode_7b_leg(torch, args):
    """ms per decode step of the Llama-7B-shaped model at context 4096, batch 1 and
    8 (bench_cli.bench_decoder_7b: HIP-graph steps, weights and the N(0,1) fp16 KV context
    resident); HBM fraction from codes + KV bytes per step."""
    from cortexsdr_amd import bench_cli

    out = []
    for B in (1, 8):
        r = bench_cli.bench_decoder_7b(torch, batch=B)
        out.append({k: r[k] for k in ("batch", "context", "ms_per_step", "tokens_per_s",
                                      "code_GB_per_step", "kv_GB_per_step", "alg_GBps",
                                      "hbm_frac")})
        torch.cuda.empty_cache()
    if not args.no_cpu:
        out[0]["cpu_baseline"] = cpu_7b_step()
    return out


def cpu_7b_step(ctx=4096):
    """One configs[4] decode step at batch 1 on the CPU restatement (oracle.decoder
    .step_cached: orc_hsdb_matmul OpenMP linears over the same 32 coded layers, RoPE, cached
    attention over a 4096-position fp16 context of N(0,1) values, SwiGLU, lm_head)."""
    from cortexsdr_amd import bench_cli
    from oracle import decoder as odec

    w = bench_cli.cfg5_weights(ctx + 8)
    s = w.spec
    rng = np.random.default_rng(5)
    kv = []
    for _ in range(s.n_layers):
        k = rng.standard_normal((1, ctx + 1, s.n_kv_heads, s.head_dim), np.float32)
        v = rng.standard_normal((1, ctx + 1, s.n_kv_heads, s.head_dim), np.float32)
        kv.append((k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16)))
    t0 = time.perf_counter()
    odec.step_cached(w, [1], kv, ctx)
    dt = time.perf_counter() - t0
    th = _threads()
    return {"value": round(1.0 / dt, 3), "unit": "tokens/s", "cores": th, "kind": "port",
            "ms_per_step": round(dt * 1e3, 1),
            "sample": (f"one batch-1 step at context {ctx} through "
                       f"oracle.decoder.step_cached, {th} OpenMP threads")}


def decode_7b_streaming_leg(torch):
    """configs[4] "with on-demand layer streaming": the same step with every block's codes in
    pinned host memory, copied to the device when the block runs (the next block's copy under
    the current block's kernels with prefetch); ms per step and the host-to-device rate of the
    streamed code bytes (PCIe-bound, reported apart from the resident headline)."""
    from cortexsdr_amd import bench_cli

    out = []
    for B, pf in ((1, True), (8, True), (1, False)):
        r = bench_cli.bench_decoder_7b(torch, batch=B, stream_layers=True, prefetch=pf)
        out.append({k: r[k] for k in ("batch", "prefetch", "context", "ms_per_step",
                                      "tokens_per_s", "streamed_GB_per_step", "pcie_GBps")})
        torch.cuda.empty_cache()
    return out


# fp32 vector FMA peak without packed-FP32 instructions (this build disables them):
# 256 CUs x 64 FMA lanes x 2 FLOP x 2.4 GHz
VALU_FP32_PEAK_TFLOPS = 78.6


def encode_leg(args):
    """The compress side (HSDR encoder): matching pursuit of every row of a Qwen2-0.5B-shaped
    attention (896 x 896, the reference's default K=256, 3 x 5 picks) and MLP (4864 x 896,
    forMLP: K=512, 3 x 8) matrix, 1-row tiles, on the GPU (csdr_hsdr_encode), and compress with
    the reference's default refinement passes (8 / 12); next to the reference's own compress
    (oracle/_ref, its OpenMP build) with no refinement on the same matrices."""
    import ctypes as C

    import torch

    import oracle
    from cortexsdr_amd import _lib, encode

    lib = _lib.load()
    rng = np.random.default_rng(9)
    out = []
    for name, R, Cc, K, S, k, iters in (("attn 896x896", 896, 896, 256, 3, 5, 8),
                                        ("mlp 4864x896", 4864, 896, 512, 3, 8, 12)):
        w = (rng.standard_normal((R, Cc)) * 0.02).astype(np.float32)
        D = encode.init_dictionary(w, K, S, k)
        g = (0.5 ** np.arange(S)).astype(np.float32)
        td = torch.from_numpy(w).cuda()
        Dd = torch.from_numpy(D).cuda()
        codes = torch.empty((R, S * k), dtype=torch.int16, device="cuda")
        st = torch.cuda.current_stream()
        args_ = (td.data_ptr(), R, Cc, Dd.data_ptr(), K, S, k, g.ctypes.data, codes.data_ptr(),
                 st.cuda_stream)
        _lib.check(lib.csdr_hsdr_encode(*args_))
        reps = 20
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(st)
        for _ in range(reps):
            _lib.check(lib.csdr_hsdr_encode(*args_))
        e1.record(st)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        flops = 2.0 * R * S * k * K * Cc
        encode.compress(w, 1, Cc, K, S, k, ksvd_iters=0)   # warm
        t0 = time.perf_counter()
        encode.compress(w, 1, Cc, K, S, k, ksvd_iters=0)
        gpu_c0 = time.perf_counter() - t0
        t0 = time.perf_counter()
        encode.compress(w, 1, Cc, K, S, k, ksvd_iters=iters)
        gpu_fit = time.perf_counter() - t0
        row = {"matrix": name, "K": K, "stages": S, "k_per_stage": k,
               "encode_us": round(us, 1), "rows_per_s": round(R / (us * 1e-6), 1),
               "encode_TFLOPs": round(flops / (us * 1e-6) / 1e12, 2),
               "valu_frac": round(flops / (us * 1e-6) / 1e12 / VALU_FP32_PEAK_TFLOPS, 4),
               "compress_s": round(gpu_c0, 4), "ksvd_iters": iters,
               "compress_fit_s": round(gpu_fit, 4), "cpu_reference": None}
        if not args.no_cpu and oracle.ref() is not None:
            oracle.ref_hsdr_compress(w[:64], 1, Cc, min(K, 64), S, k, ksvd_iters=0)
            t0 = time.perf_counter()
            oracle.ref_hsdr_compress(w, 1, Cc, K, S, k, ksvd_iters=0)
            dt = time.perf_counter() - t0
            threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count()
            row["cpu_reference"] = {
                "compress_s": round(dt, 4), "cores": threads, "kind": "reference",
                "sample": "HierarchicalSDRStrategy::compress, ksvd_iters = 0, same matrix"}
        out.append(row)
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the path shards by output rows across GPUs, which is not built here)",
              file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py: no HIP device", file=sys.stderr)
        sys.exit(1)
    from cortexsdr_amd import synth
    from cortexsdr_amd.hsdr import HsdbSegment

    wl = workloads(args.config)
    t_gen = time.time()
    streams = [synth.hsdb_layer(w["R"], w["C"], w["K"], w["s"], seed_dict=1, seed_codes=2 + i)
               for i, w in enumerate(wl)]
    xs = [synth.activations(w["C"], 1, seed=3 + i, dtype=w["xdtype"]) for i, w in enumerate(wl)]
    print(f"# generated {len(wl)} coded matrices in {time.time() - t_gen:.1f}s", flush=True)

    step_codes = sum(alg_bytes(w)["codes"] for w in wl)
    copies = max(2, math.ceil(3 * MALL_BYTES / step_codes) + 1)
    segs = [[HsdbSegment(s) for s in streams] for _ in range(copies)]
    xd = [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in xs]
    yd = [torch.empty((w["R"], 1), dtype=torch.float32, device="cuda") for w in wl]
    print(f"# {copies} rotating copies, {copies * step_codes / 2**20:.0f} MiB of codes resident",
          flush=True)

    from cortexsdr_amd import _lib

    lib = _lib.load()
    stream = torch.cuda.current_stream()
    sp = int(stream.cuda_stream)
    xt = [1 if w["xdtype"] == np.float16 else 0 for w in wl]

    from cortexsdr_amd.hsdr import group_workspace
    import ctypes as C

    ws = group_workspace(segs[0], 1)
    n = len(wl)
    hs = [(C.c_void_p * n)(*[s._h.value for s in segs[c]]) for c in range(copies)]
    xp = (C.c_void_p * n)(*[x.data_ptr() for x in xd])
    yp = (C.c_void_p * n)(*[y.data_ptr() for y in yd])
    xtype = xt[0]

    def step(it, sp_=None):
        # one grouped call for both coded matrices of the step: a dx launch, then the gather
        _lib.check(lib.csdr_hsdb_matmul_group(n, hs[it % copies], xp, xtype, 1, yp,
                                              ws.data_ptr(), ws.numel(), sp_ or sp))

    for it in range(args.warmup):
        step(it)
    torch.cuda.synchronize()

    # Timed region: the K steps are captured once into a HIP graph (launches through ctypes
    # are host-bound otherwise) and replayed, bracketed by synchronize.
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        sp_cap = int(torch.cuda.current_stream().cuda_stream)
        for it in range(args.steps):
            step(it, sp_cap)
    graph.replay()  # untimed first replay
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    graph.replay()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_total = start.elapsed_time(end)
    ms_step = ms_total / args.steps

    def replay_stats(g, per):
        """Per-unit ms over args.replays replays of graph g (per units each), HIP events on
        the launch stream around every replay: (median, min, max)."""
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(args.replays)]
        torch.cuda.synchronize()
        for e0, e1 in ev:
            e0.record(stream)
            g.replay()
            e1.record(stream)
        torch.cuda.synchronize()
        t = sorted(e0.elapsed_time(e1) / per for e0, e1 in ev)
        return t[len(t) // 2], t[0], t[-1]

    rep_med, rep_min, rep_max = replay_stats(graph, args.steps)

    # Dominant-kernel duration: the gather launch (both matrices), K launches back to back
    # over the rotating copies captured in one graph (after one dx; repeated gathers only
    # accumulate into y), the median over the replays.
    _lib.check(lib.csdr_hsdb_dx_group(n, hs[0], xp, xtype, 1, yp, ws.data_ptr(), ws.numel(), sp))
    ggraph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(ggraph):
        sp_cap = int(torch.cuda.current_stream().cuda_stream)
        for it in range(args.steps):
            _lib.check(lib.csdr_hsdb_gather_group(n, hs[it % copies], xp, xtype, 1, yp,
                                                  ws.data_ptr(), ws.numel(), sp_cap))
    ggraph.replay()
    kern_ms, kern_min, kern_max = replay_stats(ggraph, args.steps)

    op_bytes = sum(alg_bytes(w)["op"] for w in wl)
    value = op_bytes / (ms_step * 1e-3) / 1e9
    # dominant kernel: the gather launch (codes + P + y of both matrices); its algorithmic
    # bytes count the compressed codes, each block column's P (K floats) once, and y
    g_bytes = sum(alg_bytes(w)["gather"] for w in wl)
    achieved = g_bytes / (kern_ms * 1e-3) / 1e9

    traffic, trec = gather_traffic() if args.config == "cfg2" else (None, "not measured")
    out = {
        "metric": "fused decode-GEMV HBM GB/s",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded SplitMix64/Box-Muller; BASELINE.json configs[1])",
        "config": {
            "workload": ("cfg2 M=1: Y=W.x for W 4096x11008 and W 11008x4096, 1x64 blocks, "
                         "K=1024 unit-norm fp32 atoms, 8 nnz/block, fp16 coef, x fp16, "
                         "fp32 accumulate") if args.config == "cfg2" else
                        "cfg1 M=1: W 4096x4096, K=512, 4 nnz/block, x fp32",
            "M": 1,
            "algorithmic_bytes_per_step": op_bytes,
            "rotating_copies": copies,
            "percent_hbm_roofline": round(100.0 * value / HBM_PEAK_GBS, 2),
            "wall_s_timed": round(wall, 4),
            "gather_kernel_ms_events": round(kern_ms, 6),
        },
        "replays": {
            "count": args.replays, "steps_per_replay": args.steps,
            "median_ms_per_step": round(rep_med, 6), "min_ms_per_step": round(rep_min, 6),
            "max_ms_per_step": round(rep_max, 6),
            "median_value": round(op_bytes / (rep_med * 1e-3) / 1e9, 2),
            "gather_median_ms": round(kern_ms, 6), "gather_min_ms": round(kern_min, 6),
            "gather_max_ms": round(kern_max, 6),
        },
        "roofline": {
            "kernel": "gatherw_kernel<8,4,true> (csdr_hsdb_gather_group, both matrices)",
            "timing": f"median of {args.replays} graph replays of {args.steps} launches",
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": ("profiles/hsdb_gather_cfg2_traffic.json (sources "
                               f"{trec['source_digest']}, commit {trec.get('git_head')})"
                               if traffic else trec),
            "algorithmic_bytes_per_launch": g_bytes,
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        dt, n, threads = cpu_baseline(streams, xs, args.cpu_seconds)
        dt1, n1, _ = cpu_baseline(streams, xs, args.cpu_seconds / 2, threads=1)
        info = cpu_info()
        out["cpu_baseline"] = {
            "value": round(op_bytes / dt / 1e9, 3),
            "unit": "GB/s",
            "cores": threads,
            "kind": "port",
            "sample": (f"{n} full steps of the same workload (both matrices, M=1) through "
                       f"oracle/csdr_oracle.c orc_hsdb_matmul with {threads} OpenMP threads, "
                       f"{dt * 1e3:.1f} ms/step"),
            **info,
            "single_thread": {
                "value": round(op_bytes / dt1 / 1e9, 3), "unit": "GB/s", "cores": 1,
                "sample": f"{n1} steps on one thread, {dt1 * 1e3:.1f} ms/step (the reference's "
                          "fused HSDR path is single-threaded)"},
        }
    if not args.no_configs:
        out["cfg1"] = cfg1_leg(torch, args)
        out["cfg3"] = cfg3_leg(torch, args)
        out["strategy5"] = strategy5_leg(torch, args)
    if not args.no_decode:
        out["decode"] = decode_leg(args)
    if not args.no_7b:
        out["decode_7b"] = decode_7b_leg(torch, args)
        out["decode_7b_streaming"] = decode_7b_streaming_leg(torch)
    if not args.no_encode:
        out["encode"] = encode_leg(args)
    if args.calibrate_copy:
        a = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        del a, b
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
