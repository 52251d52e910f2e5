"""GPU test of text generation (reference src/generate.rs:93-118): the
library's tokenizer + model loops against the oracle model and the oracle's
tokenizer restatement -- identical prompt ids, generated ids and text."""
import json
import os
import random

import numpy as np
import pytest

import oracle
from ammon_amd import BpeTokenizer, LlamaModel
from oracle import bpe

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def c1_tokenizer(vocab_size):
    """llama2.c layout: <unk> <s> </s>, 256 byte pieces, then pieces over a
    small alphabet with seeded scores."""
    rng = random.Random(2718)
    vocab = ["<unk>", "<s>", "</s>"] + [f"<0x{b:02X}>" for b in range(256)]
    alphabet = list("etaoin shrdlu")
    seen = set(vocab)
    for ch in alphabet:
        vocab.append(ch)
        seen.add(ch)
    vocab.append(" once")
    seen.add(" once")
    while len(vocab) < vocab_size:
        piece = "".join(rng.choice(alphabet) for _ in range(rng.randint(2, 6)))
        if piece not in seen:
            seen.add(piece)
            vocab.append(piece)
    scores = [0.0] * 259 + [round(rng.uniform(-30, 30), 3) for _ in range(vocab_size - 259)]
    return vocab, scores


@pytest.fixture(scope="module")
def c1_model_and_tokenizer():
    f = np.load(os.path.join(HERE, "golden", "c1_greedy.npz"))
    cfg = oracle.LlamaConfig(**json.loads(str(f["config"])))
    weights = oracle.random_weights(cfg, seed=int(f["weight_seed"]), std=0.02)
    vocab, scores = c1_tokenizer(cfg.vocab)
    return cfg, weights, vocab, scores


@pytest.mark.parametrize("loop", ["host", "device", "prefill"])
def test_generate_text_matches_oracle(rt, c1_model_and_tokenizer, loop):
    cfg, weights, vocab, scores = c1_model_and_tokenizer
    prompt = "once upon a time, there was a tiny shard"
    tok = BpeTokenizer.from_parts(vocab, scores, 6)
    otok = bpe.Bpe(vocab, scores, 6)
    ids = otok.encode(prompt.encode(), True, False)
    assert tok.encode(prompt, True, False) == ids
    om = oracle.Model(cfg, dict(weights))
    want_tokens, _ = om.generate_tokens(ids, 48)
    om.close()
    want_text = bpe.decode_text(otok, ids[0], want_tokens)
    m = LlamaModel.from_host(rt, cfg, weights)
    text, tokens, tps = m.generate_text(tok, prompt, 48, loop=loop)
    np.testing.assert_array_equal(tokens, want_tokens)
    assert text.encode() == want_text
    assert text.startswith("once upon a time")  # the prompt after the first token, then generation
    assert tps > 0
    m.close()
