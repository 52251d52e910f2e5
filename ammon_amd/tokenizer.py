"""ctypes handle on the library's BPE tokenizer (include/ammon/ammon_tokenizer.h):
the reference's ``BpeTokenizer`` (src/tokenizer.rs:18-177) implemented in C++."""
from __future__ import annotations

import ctypes

import numpy as np

from . import _abi
from ._abi import call


class BpeTokenizer:
    """llama2.c-compatible BPE: ``from_file`` (tokenizer.bin) or
    ``from_parts`` (pieces as str or bytes, scores)."""

    BOS_ID = 1
    EOS_ID = 2

    def __init__(self, handle: ctypes.c_void_p):
        self.handle = handle

    @classmethod
    def from_file(cls, path: str, vocab_size: int) -> "BpeTokenizer":
        h = ctypes.c_void_p()
        call("ammon_bpe_load", str(path).encode(), vocab_size, ctypes.byref(h))
        return cls(h)

    @classmethod
    def from_parts(cls, pieces, scores, max_token_length: int = 0) -> "BpeTokenizer":
        raw = [p.encode() if isinstance(p, str) else bytes(p) for p in pieces]
        n = len(raw)
        arr = (ctypes.c_char_p * max(n, 1))(*raw)
        lens = (ctypes.c_uint32 * max(n, 1))(*[len(p) for p in raw])
        sc = (ctypes.c_float * max(n, 1))(*[float(s) for s in scores])
        h = ctypes.c_void_p()
        call("ammon_bpe_from_parts", arr, lens, sc, n, max_token_length, ctypes.byref(h))
        return cls(h)

    def close(self) -> None:
        if self.handle:
            call("ammon_bpe_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def vocab_size(self) -> int:
        return int(_abi.lib.ammon_bpe_vocab_size(self.handle))

    @property
    def max_token_length(self) -> int:
        return int(_abi.lib.ammon_bpe_max_token_length(self.handle))

    def encode(self, text, bos: bool = True, eos: bool = False) -> list:
        data = text.encode() if isinstance(text, str) else bytes(text)
        n = ctypes.c_size_t()
        call("ammon_bpe_encode", self.handle, data, len(data), int(bos), int(eos), None, 0,
             ctypes.byref(n))
        ids = np.empty(max(n.value, 1), np.int32)
        call("ammon_bpe_encode", self.handle, data, len(data), int(bos), int(eos),
             ids.ctypes.data, ids.size, ctypes.byref(n))
        return [int(i) for i in ids[: n.value]]

    def decode_bytes(self, prev_token: int, token: int) -> bytes:
        n = ctypes.c_size_t()
        call("ammon_bpe_decode", self.handle, prev_token, token, None, 0, ctypes.byref(n))
        buf = ctypes.create_string_buffer(n.value + 1)
        call("ammon_bpe_decode", self.handle, prev_token, token, buf, n.value + 1,
             ctypes.byref(n))
        return buf.raw[: n.value]

    def decode(self, prev_token: int, token: int) -> str:
        return self.decode_bytes(prev_token, token).decode()
