"""GPU parity at the depth and length the benchmarks run.

* configs[3], the run bench.py times: the Qwen2-0.5B-shaped model (24 layers, hidden 896,
  vocab 151,936, every linear HSDB-coded against one 1024 x 64 dictionary), the 512-token
  prompt of uniform random ids and 128 greedy tokens, through the same call sequence
  (bench_cli.cfg4_run). Against the oracle: the prompt's full-context forward (the reference's
  recompute, api/cortex_sdk.cpp:1543-1696), then one cached fp32 step per new token forced
  along the device's tokens. Per step the lm_head scores are within 1e-3 relative L2 and the
  token is the oracle's argmax unless the oracle's top two are within 2e-3 (a near-tie that
  float summation order may flip).
* configs[4], the step bench.py times: the Llama-7B-shaped model at all 32 layers
  (bench_cli.cfg5_weights), fp16 K/V context of 4096 positions with N(0,1) values, batch 1
  and 8, one decode step against oracle.decoder.step_cached.
  At this depth the random-init model amplifies fp32 rounding: two fp32 orderings of the
  oracle itself (the fused product and decode-then-dense) differ by 1e-5 to 1.2e-3 in these
  scores over the 8 sequences, and the device's batch-8 step agrees with the same sequences
  decoded alone at batch 1 within 1.3e-4 (both measured on MI355X with these inputs). The
  residual against the oracle is that conditioning (transcendentals and the fp16 rounding of
  the new K/V row differ in their last bits), not the batched path, so the bar here is 2e-3
  per sequence and 1e-3 on the batch mean; the test measures and prints the oracle's own
  spread beside the device's error.
"""
import numpy as np
import pytest

from oracle import decoder as odec
from cortexsdr_amd import bench_cli
from cortexsdr_amd.decoder import Decoder
from conftest import rel_l2

pytestmark = pytest.mark.gpu


def _check_token(scores, tok, what):
    top = np.sort(scores)[-2:]
    if top[1] - top[0] > 2e-3 * max(1.0, abs(float(top[1]))):
        assert tok == int(np.argmax(scores)), what


def test_cfg4_benchmarked_run_matches_oracle(gpu):
    n_prompt, n_new = 512, 128
    print(f"cfg4 benchmarked run: prompt {n_prompt}, {n_new} greedy tokens", flush=True)
    w, prompt = bench_cli.cfg4_workload(n_prompt, seed=0)
    s = w.spec
    dec = Decoder(w)
    try:
        # the bench's own sequence (one decode call for the 127 steps) ...
        _, _, bench_toks = bench_cli.cfg4_run(dec, prompt, n_new)
        # ... and the same run step by step, reading the scores of every step
        dec.prefill(prompt, 0.0, 0.0)
        scores = [dec.logits()]
        for _ in range(n_new - 1):
            dec.decode(1, 0.0, 0.0)
            scores.append(dec.logits())
        toks = dec.tokens(n_prompt, n_new)
    finally:
        dec.close()
    assert np.array_equal(toks, bench_toks)
    print(f"device tokens {toks[:8].tolist()} ...", flush=True)
    dense = odec.DenseWeights()
    want, kvs = odec.prompt_state(w, prompt, dense)
    cap = n_prompt + n_new
    kv = []
    for k, v in kvs:
        kb = np.zeros((1, cap, s.n_kv_heads, s.head_dim), np.float32)
        vb = np.zeros_like(kb)
        kb[0, :n_prompt], vb[0, :n_prompt] = k, v
        kv.append((kb, vb))
    worst = 0.0
    for i in range(n_new):
        if i:
            want = odec.step_cached(w, toks[i - 1:i], kv, n_prompt + i - 1, dense)[0][0]
        err = rel_l2(scores[i], want)
        worst = max(worst, err)
        assert err < 1e-3, f"step {i}: scores rel L2 {err:.2e}"
        _check_token(want, int(toks[i]), f"step {i}")
    print(f"cfg4: {n_new} steps, worst scores rel L2 {worst:.2e}", flush=True)


@pytest.mark.parametrize("B", [1, 8])
def test_cfg5_full_depth_step_matches_oracle(gpu, B):
    torch = gpu
    n = 4096
    w = bench_cli.cfg5_weights(n + 8)
    s = w.spec
    print(f"cfg5 full depth: B={B} layers={s.n_layers} context={n}", flush=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(1000 + B)
    rng = np.random.default_rng(200 + B)
    tokens = rng.integers(0, s.vocab, size=B).astype(np.int32)
    dec = Decoder(w, batch=B)
    try:
        kv = []
        shape = (B, n, s.n_kv_heads, s.head_dim)
        for layer in range(s.n_layers):
            k = torch.randn(shape, device="cuda", generator=g).half()
            v = torch.randn(shape, device="cuda", generator=g).half()
            dec.load_kv(layer, k, v, n)
            # host copies with room for the step's row (written in place by the oracle)
            kh = np.empty((B, n + 1, s.n_kv_heads, s.head_dim), np.uint16)
            vh = np.empty_like(kh)
            kh[:, :n] = k.cpu().numpy().view(np.uint16)
            vh[:, :n] = v.cpu().numpy().view(np.uint16)
            kv.append((kh, vh))
            del k, v
        dec.set_position(n, tokens)
        dec.decode(1, 0.0, 0.0)
        got = dec.logits().reshape(B, s.vocab)
        nxt = dec.tokens(n + 1, 1).reshape(B)
        assert dec.position() == n + 1
    finally:
        dec.close()
    want, _ = odec.step_cached(w, tokens, kv, n)
    # the oracle's own spread: the same step with decode-then-dense products
    other, _ = odec.step_cached(w, tokens, kv, n, odec.DenseWeights())
    errs = []
    for b in range(B):
        err = rel_l2(got[b], want[b])
        errs.append(err)
        print(f"cfg5 B={B} seq {b}: device rel L2 {err:.2e}, oracle orderings "
              f"{rel_l2(other[b], want[b]):.2e}", flush=True)
        assert err < 2e-3, f"B={B} seq {b}: rel L2 {err:.2e}"
        _check_token(want[b], int(nxt[b]), f"B={B} seq {b}")
    assert float(np.mean(errs)) < 1e-3, errs
