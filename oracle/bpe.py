"""CPU oracle for the reference's BPE tokenizer and text generation -- TEST
INFRASTRUCTURE.

A pure-Python restatement (small vocabularies and texts only) of
``src/tokenizer.rs:18-177`` (llama2.c tokenizer.bin loading, encode,
decode) and of the text assembly of ``generate`` (``src/generate.rs:93-118``),
citing file:line per function.  Strings are handled as UTF-8 ``bytes``, as
the reference's ``String``s hold them.

Only ``tests/`` may import this module, to check results; the product
(``libammon_amd.so``'s C++ tokenizer) never calls it.

Points where the reference's behaviour comes from Rust's standard library
rather than its own code, restated here from the library's documented
semantics:
- ``String::from_utf8_lossy`` replaces each maximal invalid UTF-8 subpart
  with U+FFFD (Python's ``bytes.decode("utf-8", "replace")`` follows the same
  Unicode recommendation);
- ``<[T]>::binary_search_by`` with duplicate keys: the loop of the current
  standard library settles on the last equal element (parity for duplicate
  pieces follows that implementation; older releases could return another
  of the equals -- unpinned by the reference's tests);
- ``u8::from_str_radix(s, 16)`` accepts an optional leading '+';
- ``byte as char`` maps byte b to the code point U+00b.
"""
from __future__ import annotations

import struct

BOS_ID = 1  # src/tokenizer.rs:8
EOS_ID = 2  # src/tokenizer.rs:9


def lossy_utf8(raw: bytes) -> bytes:
    """String::from_utf8_lossy (used at src/tokenizer.rs:53)."""
    return raw.decode("utf-8", "replace").encode("utf-8")


def _is_utf8(raw: bytes) -> bool:
    try:
        raw.decode("utf-8")
        return True
    except UnicodeDecodeError:
        return False


class Bpe:
    """BpeTokenizer (src/tokenizer.rs:18-94)."""

    def __init__(self, vocab, scores, max_token_length: int = 0):
        # from_parts, src/tokenizer.rs:59-73
        self.vocab = [v.encode() if isinstance(v, str) else bytes(v) for v in vocab]
        self.scores = [float(s) for s in scores]
        assert len(self.vocab) == len(self.scores)
        self.max_token_length = max_token_length
        # stable sort by bytes: equal pieces keep id order
        self.sorted = sorted(((p, i) for i, p in enumerate(self.vocab)), key=lambda e: e[0])

    @classmethod
    def from_bytes(cls, data: bytes, vocab_size: int) -> "Bpe":
        """from_path (src/tokenizer.rs:28-57) on the file's bytes."""
        (max_len,) = struct.unpack_from("<I", data, 0)
        off = 4
        vocab, scores = [], []
        for i in range(vocab_size):
            score, n = struct.unpack_from("<fi", data, off)
            off += 8
            if n < 0:
                raise ValueError(f"tokenizer piece {i} has negative length {n}")
            raw = data[off:off + n]
            if len(raw) < n:
                raise ValueError(f"read tokenizer piece {i}")
            off += n
            scores.append(score)
            vocab.append(lossy_utf8(raw))
        return cls(vocab, scores, max_len)

    def lookup(self, s: bytes):
        """lookup (src/tokenizer.rs:87-92): the standard library's slice
        binary search over the sorted pieces."""
        size = len(self.sorted)
        if size == 0:
            return None
        base = 0
        while size > 1:
            half = size // 2
            mid = base + half
            if not (self.sorted[mid][0] > s):  # Less or Equal
                base = mid
            size -= half
        return self.sorted[base][1] if self.sorted[base][0] == s else None

    def encode(self, text: bytes, bos: bool, eos: bool) -> list:
        """Tokenizer::encode (src/tokenizer.rs:104-159)."""
        tokens = []
        if bos:
            tokens.append(BOS_ID)
        if text:
            dummy = self.lookup(b" ")
            if dummy is not None:
                tokens.append(dummy)
        i = 0
        while i < len(text):
            start = i
            i += 1
            while i < len(text) and (text[i] & 0xC0) == 0x80 and i - start < 4:
                i += 1
            piece = text[start:i]
            if _is_utf8(piece):
                pid = self.lookup(piece)
                if pid is not None:
                    tokens.append(pid)
                    continue
            tokens.extend(b + 3 for b in piece)
        while True:
            best_score, best_id, best_idx = -1e10, -1, None
            for j in range(len(tokens) - 1):
                pid = self.lookup(self.vocab[tokens[j]] + self.vocab[tokens[j + 1]])
                if pid is not None and self.scores[pid] > best_score:
                    best_score, best_id, best_idx = self.scores[pid], pid, j
            if best_idx is None:
                break
            tokens[best_idx] = best_id
            del tokens[best_idx + 1]
        if eos:
            tokens.append(EOS_ID)
        return tokens

    def decode(self, prev_token: int, token: int) -> bytes:
        """Tokenizer::decode (src/tokenizer.rs:161-170) with parse_byte_token
        (:173-176)."""
        piece = self.vocab[token] if 0 <= token < len(self.vocab) else b""
        if prev_token == BOS_ID and piece.startswith(b" "):
            piece = piece[1:]
        if piece.startswith(b"<0x") and piece.endswith(b">") and len(piece) >= 4:
            rest = piece[3:-1]
            digits = rest[1:] if rest.startswith(b"+") else rest
            if digits and all(c in b"0123456789abcdefABCDEF" for c in digits):
                value = int(digits, 16)
                if value <= 255:
                    return chr(value).encode("utf-8")
        return piece


def decode_text(tok: Bpe, first: int, tokens) -> bytes:
    """The text assembly of generate (src/generate.rs:106-113)."""
    out, prev = b"", first
    for t in tokens:
        out += tok.decode(prev, int(t))
        prev = int(t)
    return out


def tokenizer_bin(vocab, scores, max_token_length: int) -> bytes:
    """A llama2.c tokenizer.bin image (the layout src/tokenizer.rs:28-57
    reads)."""
    out = struct.pack("<I", max_token_length)
    for piece, score in zip(vocab, scores):
        raw = piece.encode() if isinstance(piece, str) else bytes(piece)
        out += struct.pack("<fi", float(score), len(raw)) + raw
    return out
