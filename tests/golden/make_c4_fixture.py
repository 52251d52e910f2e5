"""Writes tests/golden/c4_greedy.npz: the Llama-3-8B-shaped greedy decode
(32 layers, dim 4096, 32 q / 8 kv heads of 128, SwiGLU hidden 14336, vocab
128256, RoPE theta 500000, bf16 weights N(0, 0.02) from the oracle's seeded
generator, RMSNorm weights 1, KV cache sized 8192) run through the oracle
from a seeded 16-token prompt with max_new_tokens 528: 527 steps, 15 forced
prompt tokens then 512 greedy picks (reference src/generate.rs:43-91).

The KV cache is fp32, as in the reference (src/modules.rs:53-54).  (With a
bf16 cache a free-running comparison of two correct implementations parts
after a few hundred steps: tests/golden/c4_bf16kv_drift.npz.)  The prompt
is drawn with seed 1004, taken by rule (the first seed of the range the
earlier fixtures drew from), not chosen for its margins; the test stops its
token comparison at the first step whose top-2 margin the logits'
tolerance could close, so that margins are stored per step with the
step's logit scale.

Stored:
  inputs   config, weight seed, prompt, max_new_tokens, and per weight tensor
           two 64-bit checksums of its storage words (wrapping sum and xor of
           the little-endian uint64 words), so a test that generates the
           weights elsewhere can prove they are the oracle's, bit for bit;
  outputs  the 527 chosen tokens, the last step's logits [128256], and for
           every step the gap between the largest and the second-largest
           logit (top-2 margin), the runner-up's index and the largest
           |logit| (the scale of the normwise tolerance), so a mismatch can
           be told apart from a near tie.

The oracle (C, OpenMP over output rows, each row in its serial order) is
bit-identical for any thread count.  About 16 GB of host memory for the
weights; at 8 threads about half a second per step.

Run: python tests/golden/make_c4_fixture.py
"""
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle  # noqa: E402

C4 = dict(dim=4096, n_layers=32, n_heads=32, n_kv_heads=8, hidden=14336, vocab=128256,
          max_seq=8192, theta=500000.0, eps=1e-5)
WEIGHT_SEED = 1003
PROMPT_SEED = 1004
PROMPT_LEN = 16
MAX_NEW_TOKENS = 528
PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c4_greedy.npz")


def config():
    return oracle.LlamaConfig(**C4, w_dtype=oracle.BF16, kv_dtype=oracle.F32)


def c4_prompt():
    # 16 ids uniform in [1, 128256)
    rng = np.random.default_rng(PROMPT_SEED)
    return rng.integers(1, C4["vocab"], size=PROMPT_LEN).astype(np.int32)


def checksum(a: np.ndarray):
    """(wrapping sum, xor) of the array's storage as little-endian uint64 words."""
    w = np.ascontiguousarray(a).reshape(-1).view(np.uint64)
    return int(np.sum(w, dtype=np.uint64)), int(np.bitwise_xor.reduce(w))


def top2(logits: np.ndarray):
    """(margin between the two largest logits, index of the runner-up)."""
    i = int(oracle.sample_argmax(logits))
    rest = logits.copy()
    rest[i] = -np.inf
    j = int(np.argmax(rest))
    return float(logits[i]) - float(logits[j]), j


def log(msg):
    print(msg, flush=True)


def run():
    cfg = config()
    t0 = time.time()
    weights = oracle.random_weights(cfg, seed=WEIGHT_SEED, std=0.02)
    sums = {name: checksum(a) for name, a in weights.items()}
    log(f"weights generated in {time.time() - t0:.0f} s")
    prompt = c4_prompt()
    m = oracle.Model(cfg, weights)
    limit = min(MAX_NEW_TOKENS, cfg.max_seq)
    tokens, margins, runners, scales = [], [], [], []
    token = int(prompt[0])
    logits = None
    t1 = time.time()
    for pos in range(limit - 1):
        logits = m.step(token, pos)
        margin, runner = top2(logits)
        nxt = int(prompt[pos + 1]) if pos < len(prompt) - 1 else int(oracle.sample_argmax(logits))
        tokens.append(nxt)
        margins.append(margin)
        runners.append(runner)
        scales.append(float(np.max(np.abs(logits))))
        token = nxt
        if pos % 16 == 0:
            rate = (pos + 1) / (time.time() - t1)
            log(f"pos {pos}: next {nxt}, top-2 margin {margin:.3e}, {rate:.2f} steps/s")
    m.close()
    return prompt, np.array(tokens, np.int32), logits, np.array(margins, np.float32), \
        np.array(runners, np.int32), np.array(scales, np.float32), sums


if __name__ == "__main__":
    prompt, tokens, logits, margins, runners, scales, sums = run()
    np.savez_compressed(PATH, prompt=prompt, tokens=tokens, logits=logits, margins=margins,
                        runners=runners, scales=scales, config=json.dumps(C4),
                        weight_seed=WEIGHT_SEED,
                        w_dtype=oracle.BF16, kv_dtype=oracle.F32,
                        max_new_tokens=MAX_NEW_TOKENS,
                        checksums=json.dumps({k: [str(s), str(x)] for k, (s, x) in sums.items()}))
    gen = margins[PROMPT_LEN - 1:]
    log(f"wrote {PATH}: {len(tokens)} tokens, first generated {tokens[PROMPT_LEN - 1:][:8].tolist()}, "
        f"smallest generated-step margin {float(gen.min()):.3e} at step {int(gen.argmin())}")
