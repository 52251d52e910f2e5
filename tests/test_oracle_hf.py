"""The oracle's whole model against an independent implementation: Hugging
Face transformers' LlamaForCausalLM (CPU, fp32) with random weights, its
parameters converted as llama2.c's export.py converts Hugging Face
checkpoints (tests/hf_reference.py).  Logits at every prompt position within
1e-5 (normwise, the fp32 bar) and the greedy continuation identical while
the top-2 margin is not a near-tie.  This pins the RoPE pairing and the
q/k row permutation, GQA head sharing, the RMSNorm placement and the
gate/up/down roles with code this repository did not write."""
import numpy as np
import pytest

import oracle

pytest.importorskip("transformers")
import hf_reference as hf  # noqa: E402

# (dim, layers, heads, kv heads, hidden, vocab, RoPE base): GQA 2:1 at head
# 64, no GQA at head 64 with odd widths elsewhere, and Llama-3-style heads
# (128 wide, GQA 4:1, base 5e5)
SHAPES = [(256, 2, 4, 2, 520, 611, 10000.0), (192, 2, 3, 3, 300, 257, 10000.0),
          (1024, 2, 8, 2, 2816, 1000, 500000.0)]


def rel(got, want):
    return float(np.max(np.abs(np.asarray(got, np.float64) - want)) / np.max(np.abs(want)))


@pytest.mark.parametrize("shape", SHAPES)
def test_oracle_model_matches_hf_llama(shape):
    dim, layers, heads, kv_heads, hidden, vocab, theta = shape
    cfg = oracle.LlamaConfig(dim=dim, n_layers=layers, n_heads=heads, n_kv_heads=kv_heads,
                             hidden=hidden, vocab=vocab, max_seq=48, theta=theta)
    m = hf.hf_model(cfg, seed=3)
    om = oracle.Model(cfg, hf.to_arrays(m, cfg))
    try:
        prompt = [1, vocab - 1, 37, 37, 5, 200, 42, 7]
        want = hf.logits(m, prompt)
        got = None
        for pos, tok in enumerate(prompt):
            got = om.step(tok, pos)
            assert rel(got, want[pos]) <= 1e-5, pos
        want_toks, margins = hf.greedy(m, prompt, 12)
        tok = int(oracle.sample_argmax(got))
        for i, (w, margin) in enumerate(zip(want_toks, margins)):
            if margin < 1e-4:
                break  # a near-tie: either token is the fp32 model's answer
            assert tok == w, i
            got = om.step(tok, len(prompt) + i)
            tok = int(oracle.sample_argmax(got))
    finally:
        om.close()
