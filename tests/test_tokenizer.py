"""CPU tests of the BPE tokenizer (host code in libammon_amd.so, reference
src/tokenizer.rs:18-177) against the oracle's restatement (oracle/bpe.py).

The oracle is pinned first: the reference's own tokenizer tests
(src/tokenizer.rs:197-235), the Unicode standard's worked example of
replacing maximal invalid subparts (the reference's from_utf8_lossy on
load), the lossless property of the byte fallback, the merge loop's
termination condition, and decode's round trip.  The product must then give
identical ids and identical decoded bytes to the oracle on random
llama2.c-style vocabularies and texts, and load tokenizer.bin files alike.
"""
import os
import random

import pytest

from ammon_amd import AmmonError, BpeTokenizer
from oracle import bpe

TOY = (["<unk>", "<s>", "</s>", "a", "b", "ab", " "], [0.0, 0.0, 0.0, 1.0, 1.0, 10.0, 0.0])


def both(vocab, scores, max_len=8):
    return bpe.Bpe(vocab, scores, max_len), BpeTokenizer.from_parts(vocab, scores, max_len)


# ---- the reference's own tests, on the oracle and the product ----------------------------
@pytest.mark.parametrize("which", ["oracle", "product"])
def test_reference_tokenizer_tests(which):
    o, p = both(*TOY)
    tok = o if which == "oracle" else p
    dec = (lambda a, b: tok.decode(a, b)) if which == "oracle" else tok.decode_bytes
    ids = tok.encode(b"ab" if which == "oracle" else "ab", True, False)
    assert ids[0] == 1 and ids[1] == 6 and ids[2] == 5  # src/tokenizer.rs:208-214
    assert dec(1, 6) == b"" and dec(0, 6) == b" "        # :216-221
    vocab = ["<unk>", "<s>", "</s>", "<0x41>"]            # :228-234
    o2, p2 = both(vocab, [0.0] * 4)
    assert (o2.decode(0, 3) if which == "oracle" else p2.decode_bytes(0, 3)) == b"A"


# ---- pinning the oracle ---------------------------------------------------------------------
def test_lossy_utf8_matches_the_unicode_standard_example():
    # Unicode 15, section 3.9, table 3-8: 61 F1 80 80 E1 80 C2 62 80 63 80 BF 64
    raw = bytes.fromhex("61F18080E180C2628063" "80BF64")
    want = "a���b�c��d".encode()
    assert bpe.lossy_utf8(raw) == want


def llama2c_vocab(rng, n_merges, alphabet="ab cdé→xyz", dup=False):
    """<unk> <s> </s>, the 256 byte pieces <0x00>..<0xFF> (ids 3..258), then
    random merged pieces with random scores."""
    vocab = ["<unk>", "<s>", "</s>"] + [f"<0x{b:02X}>" for b in range(256)]
    scores = [0.0, 0.0, 0.0] + [0.0] * 256
    seen = set(vocab)
    singles = list(dict.fromkeys(alphabet))
    for ch in singles:  # every code point of the alphabet as a piece
        vocab.append(ch)
        scores.append(rng.uniform(-5, 0))
        seen.add(ch)
    while len(vocab) < 259 + len(singles) + n_merges:
        piece = "".join(rng.choice(singles) for _ in range(rng.randint(2, 5)))
        if piece in seen and not dup:
            continue
        seen.add(piece)
        vocab.append(piece)
        scores.append(round(rng.uniform(-20, 20), 2))
    return vocab, scores


def token_bytes(tok, t):
    if 3 <= t < 259:
        return bytes([t - 3])
    return tok.vocab[t]


def test_oracle_encoding_is_lossless_and_fully_merged():
    rng = random.Random(5)
    vocab, scores = llama2c_vocab(rng, 300)
    tok = bpe.Bpe(vocab, scores)
    for _ in range(60):
        text = "".join(rng.choice("ab cdé→xyzQé") for _ in range(rng.randint(0, 40))).encode()
        ids = tok.encode(text, False, False)
        joined = b"".join(token_bytes(tok, t) for t in ids)
        assert joined == (b" " + text if text else b"")  # dummy prefix + the text, byte for byte
        for a, b in zip(ids, ids[1:]):  # the merge loop stopped: no mergeable pair is left
            pid = tok.lookup(tok.vocab[a] + tok.vocab[b])
            assert pid is None or tok.scores[pid] <= -1e10


def test_oracle_decode_round_trip():
    rng = random.Random(6)
    vocab, scores = llama2c_vocab(rng, 200, alphabet="ab cd")
    tok = bpe.Bpe(vocab, scores)
    for _ in range(40):
        text = "".join(rng.choice("ab cdQZ!") for _ in range(rng.randint(1, 30))).encode()
        ids = tok.encode(text, True, False)
        assert bpe.decode_text(tok, ids[0], ids[1:]) == text  # space dropped after BOS


def test_oracle_binary_search_settles_on_the_last_duplicate():
    tok = bpe.Bpe(["<unk>", "<s>", "</s>", "x", "y", "x", "x"], [0] * 7)
    assert tok.lookup(b"x") == 6 and tok.lookup(b"y") == 4 and tok.lookup(b"z") is None


# ---- product vs oracle ----------------------------------------------------------------------
@pytest.mark.parametrize("seed", range(4))
def test_encode_matches_oracle_on_random_vocabularies(seed):
    rng = random.Random(100 + seed)
    vocab, scores = llama2c_vocab(rng, rng.choice([50, 400, 1500]), dup=seed == 3)
    o, p = both(vocab, scores)
    for _ in range(80):
        text = "".join(rng.choice("ab cdé→xyzQé\U0001F600\n") for _ in range(rng.randint(0, 60)))
        for bos, eos in ((True, False), (False, False), (True, True)):
            assert p.encode(text, bos, eos) == o.encode(text.encode(), bos, eos), text


def test_decode_matches_oracle_including_edge_pieces():
    rng = random.Random(7)
    vocab, scores = llama2c_vocab(rng, 100)
    vocab += [" lead", "<0x+41>", "<0x100>", "<0x>", "<0xZZ>", "<0x0a>", "<0xe9>", " <0x41>"]
    scores += [0.0] * 8
    o, p = both(vocab, scores)
    for prev in (0, 1, 2, 5):
        for t in list(range(len(vocab))) + [-1, len(vocab), 1 << 30]:
            assert p.decode_bytes(prev, t) == o.decode(prev, t), (prev, t, vocab[t] if 0 <= t < len(vocab) else t)


def test_tokenizer_bin_load_matches_oracle(tmp_path):
    rng = random.Random(8)
    vocab, scores = llama2c_vocab(rng, 300)
    # pieces that are not valid UTF-8 are read lossily, as the reference
    raw = [v.encode() for v in vocab] + [b"\xf1\x80\x80z", b"\xc0\xaf", b"ok\xe2\x82"]
    scores = scores + [1.0, 2.0, 3.0]
    path = tmp_path / "tokenizer.bin"
    path.write_bytes(bpe.tokenizer_bin(raw, scores, 27))
    o = bpe.Bpe.from_bytes(path.read_bytes(), len(raw))
    p = BpeTokenizer.from_file(str(path), len(raw))
    assert p.vocab_size == len(raw) and p.max_token_length == 27
    for t in range(len(raw)):
        assert p.decode_bytes(0, t) == o.decode(0, t)
    for text in ("ab cd", "zzé→", "", "QQ ab"):
        assert p.encode(text, True, False) == o.encode(text.encode(), True, False)


def test_tokenizer_bin_errors(tmp_path):
    with pytest.raises(AmmonError, match="open tokenizer"):
        BpeTokenizer.from_file(str(tmp_path / "missing.bin"), 3)
    path = tmp_path / "neg.bin"
    path.write_bytes(bpe.tokenizer_bin(["a"], [0.0], 4)[:8] + (-2).to_bytes(4, "little", signed=True))
    with pytest.raises(AmmonError, match="negative length"):
        BpeTokenizer.from_file(str(path), 1)
    path.write_bytes(bpe.tokenizer_bin(["a", "b"], [0.0, 0.0], 4))
    with pytest.raises(AmmonError, match="read tokenizer score 2"):
        BpeTokenizer.from_file(str(path), 3)


def test_byte_fallback_outside_the_vocabulary_is_an_error():
    # the reference indexes its vocabulary with the fallback id and would panic
    p = BpeTokenizer.from_parts(*TOY, 8)
    with pytest.raises(AmmonError, match="outside the vocabulary"):
        p.encode("c", True, False)
