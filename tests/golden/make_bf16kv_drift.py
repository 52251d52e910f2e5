"""Writes tests/golden/c4_bf16kv_drift.npz: how far two correct fp32
implementations of the Llama-3-8B-shaped greedy decode drift apart, with a
bf16 KV cache (the configuration the benchmark measures) and with the
reference's fp32 cache, measured with the oracle against itself.

The model is the C4 fixture's (32 layers, dim 4096, 32 q / 8 kv heads of
128, SwiGLU hidden 14336, vocab 128256, RoPE theta 500000, bf16 weights N(0,
0.02) from weight seed 1003, RMSNorm weights 1, cache sized 8192).  The
16-token prompt is drawn with seed 1004 -- the C4 fixture's prompt, taken
by rule (the first seed of its range), with no screening.

Run A is the oracle as it restates the reference (every GEMV row summed
with j ascending, src/kernels.rs:54-73).  Run B is the same oracle with one
valid change of fp32 summation order: every GEMV row summed with j
descending.  Both runs decode greedily from the same prompt, each feeding
back its own choice (reference src/generate.rs:43-91), in lockstep; per step
the study records both tokens, run A's top-2 logit margin, and the normwise
relative difference of the two logit vectors (max |a - b| / max |a|).  It
stops at the first step whose tokens differ (after that the two runs decode
different sequences) or after max_new_tokens 528 (527 steps).

Stored per cache dtype (prefix "bf16_" and "f32_"): tokens_a, tokens_b,
margins_a [steps], drift [steps], first_divergent (-1 if none), and the
config, weight seed and prompt.  About 16 GB of host memory; at 8 threads
about 0.4 s per step per run.

Run: python tests/golden/make_bf16kv_drift.py
"""
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle  # noqa: E402

C4 = dict(dim=4096, n_layers=32, n_heads=32, n_kv_heads=8, hidden=14336, vocab=128256,
          max_seq=8192, theta=500000.0, eps=1e-5)
WEIGHT_SEED = 1003
PROMPT_SEED = 1004
PROMPT_LEN = 16
MAX_NEW_TOKENS = 528
PATH = os.path.join(HERE, "c4_bf16kv_drift.npz")


def prompt_tokens():
    rng = np.random.default_rng(PROMPT_SEED)
    return rng.integers(1, C4["vocab"], size=PROMPT_LEN).astype(np.int32)


def top2_margin(logits):
    i = int(oracle.sample_argmax(logits))
    rest = logits.copy()
    rest[i] = -np.inf
    return float(logits[i]) - float(np.max(rest))


def drift_run(weights, kv_dtype, prompt, log):
    cfg = oracle.LlamaConfig(**C4, w_dtype=oracle.BF16, kv_dtype=kv_dtype)
    a, b = oracle.Model(cfg, weights), oracle.Model(cfg, weights)
    limit = min(MAX_NEW_TOKENS, cfg.max_seq)
    ta, tb, margins, drift = [], [], [], []
    tok_a = tok_b = int(prompt[0])
    first = -1
    t0 = time.time()
    try:
        for pos in range(limit - 1):
            oracle.set_gemv_order(False)
            la = a.step(tok_a, pos)
            oracle.set_gemv_order(True)
            lb = b.step(tok_b, pos)
            oracle.set_gemv_order(False)
            forced = pos < len(prompt) - 1
            na = int(prompt[pos + 1]) if forced else int(oracle.sample_argmax(la))
            nb = int(prompt[pos + 1]) if forced else int(oracle.sample_argmax(lb))
            ta.append(na)
            tb.append(nb)
            margins.append(top2_margin(la))
            drift.append(float(np.max(np.abs(la.astype(np.float64) - lb)) /
                               np.max(np.abs(la.astype(np.float64)))))
            if pos % 32 == 0:
                log(f"  kv {'bf16' if kv_dtype == oracle.BF16 else 'f32'} pos {pos}: drift "
                    f"{drift[-1]:.2e}, margin {margins[-1]:.2e} ({(pos + 1) / (time.time() - t0):.2f} "
                    f"steps/s)")
            if na != nb:
                first = pos
                log(f"  first divergent step {pos}: run A {na}, run B {nb}, run A's top-2 margin "
                    f"{margins[-1]:.3e}, drift {drift[-1]:.2e}")
                break
            tok_a, tok_b = na, nb
    finally:
        oracle.set_gemv_order(False)
        a.close()
        b.close()
    return (np.array(ta, np.int32), np.array(tb, np.int32), np.array(margins, np.float32),
            np.array(drift, np.float64), first)


def main():
    log = lambda m: print(m, flush=True)
    t0 = time.time()
    cfg = oracle.LlamaConfig(**C4, w_dtype=oracle.BF16, kv_dtype=oracle.BF16)
    weights = oracle.random_weights(cfg, seed=WEIGHT_SEED, std=0.02)
    log(f"weights in {time.time() - t0:.0f} s")
    prompt = prompt_tokens()
    out = dict(config=json.dumps(C4), weight_seed=WEIGHT_SEED, prompt_seed=PROMPT_SEED,
               prompt=prompt, max_new_tokens=MAX_NEW_TOKENS)
    for name, kv in (("bf16", oracle.BF16), ("f32", oracle.F32)):
        ta, tb, m, d, first = drift_run(weights, kv, prompt, log)
        out.update({f"{name}_tokens_a": ta, f"{name}_tokens_b": tb, f"{name}_margins_a": m,
                    f"{name}_drift": d, f"{name}_first_divergent": first})
        log(f"kv {name}: {len(ta)} steps, first divergent step {first}, max drift "
            f"{d.max():.2e}, drift at steps 15/63/127: "
            f"{[float(d[i]) if i < len(d) else None for i in (15, 63, 127)]}")
    np.savez_compressed(PATH, **out)
    log(f"wrote {PATH}")


if __name__ == "__main__":
    main()
