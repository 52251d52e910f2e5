"""Writes tests/golden/c1_greedy.npz: the tiny llama-style decoder (dim 288,
6 layers, 6 heads of 48, SwiGLU hidden 768, vocab 32000, max_seq 256, fp32,
weights N(0, 0.02) from the oracle's seeded generator, RMSNorm weights 1,
RoPE theta 10000) run through the oracle's greedy loop from a seeded 8-token
prompt for 255 steps (7 forced, 248 generated).

Stored: the inputs (weight seed, prompt, config) and the expected outputs
(token sequence, final-step logits).  The reference cannot be run here (Rust,
absent Goldy crate), so the fixture comes from the oracle; tests/test_golden.py
regenerates it to pin the oracle's determinism, and the GPU tests compare the
HIP path against it.

Run: python tests/golden/make_c1_fixture.py
"""
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle  # noqa: E402

C1 = dict(dim=288, n_layers=6, n_heads=6, n_kv_heads=6, hidden=768, vocab=32000, max_seq=256,
          theta=10000.0)
WEIGHT_SEED = 1000
PROMPT_SEED = 1001
MAX_NEW_TOKENS = 256
PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c1_greedy.npz")


def c1_prompt():
    # 8 ids uniform in [1, 32000) from the reference tests' xorshift generator.
    u = oracle.pseudo_random(8, PROMPT_SEED).astype(np.float64)  # in [-1, 1]
    return (1 + np.floor((u + 1.0) / 2.0001 * 31999)).astype(np.int32)


def run():
    cfg = oracle.LlamaConfig(**C1)
    weights = oracle.random_weights(cfg, seed=WEIGHT_SEED, std=0.02)
    prompt = c1_prompt()
    tokens, logits = oracle.Model(cfg, weights).generate_tokens(prompt, MAX_NEW_TOKENS)
    return cfg, prompt, tokens, logits


if __name__ == "__main__":
    cfg, prompt, tokens, logits = run()
    np.savez_compressed(PATH, prompt=prompt, tokens=tokens, logits=logits,
                        config=json.dumps(C1), weight_seed=WEIGHT_SEED,
                        max_new_tokens=MAX_NEW_TOKENS)
    print(f"wrote {PATH}: {len(tokens)} tokens, first {tokens[:12].tolist()}")
