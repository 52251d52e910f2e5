"""CPU oracle for koubaa/ammon's decode-layer path -- TEST INFRASTRUCTURE.

A numpy/ctypes wrapper over ``libammon_oracle.so`` (built from
``ammon_oracle.c`` by ``oracle/Makefile``).  The C file restates the
reference kernels (``src/kernels.rs``), launch sequences (``src/blocks.rs``),
greedy loop (``src/generate.rs``) and argmax (``src/tokenizer.rs:179-189``),
citing file:line per function.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this package, and only to check results (or as the reported
CPU baseline).  The product package ``ammon_amd`` never calls it.

Layouts are the reference's: KV cache ``[seq, kv_heads, head]`` per layer,
weights ``[out, in]`` row-major, attention scratch ``[q_heads, splits,
head + 2]`` with splits of 8 positions.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass, field

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libammon_oracle.so")

F32 = 0
BF16 = 1

_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_I32 = ctypes.c_int32
_F = ctypes.c_float


def build() -> None:
    """Compile the oracle library in place (gcc + OpenMP)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _load() -> ctypes.CDLL:
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    sig = {
        "orc_f32_to_bf16": (ctypes.c_uint16, [_F]),
        "orc_bf16_to_f32": (_F, [ctypes.c_uint16]),
        "orc_f32_to_bf16_array": (None, [_P, _P, ctypes.c_size_t]),
        "orc_bf16_to_f32_array": (None, [_P, _P, ctypes.c_size_t]),
        "orc_fill_normal": (None, [_P, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_uint64, _F, _F]),
        "orc_pseudo_random": (None, [_P, ctypes.c_size_t, _U32]),
        "orc_embed": (None, [_P, ctypes.c_int, _U32, _U32, _P, _U32, _P]),
        "orc_rmsnorm": (None, [_P, _P, ctypes.c_int, _P, _U32, _U32, _F]),
        "orc_rope_table": (None, [_F, _U32, _U32, _P]),
        "orc_rope_store": (None, [_P, _P, _P, ctypes.c_int, _U32, _U32, _U32, _U32, _U32, _P]),
        "orc_cache_store": (None, [_P, _P, ctypes.c_int, _U32, _U32, _U32]),
        "orc_attention_splits": (_U32, [_U32, _U32]),
        "orc_attention_partial": (None, [_P, _P, _P, ctypes.c_int, _U32, _U32, _U32, _U32, _U32, _P]),
        "orc_attention_combine": (None, [_P, _U32, _U32, _U32, _U32, _P]),
        "orc_attention_serial": (None, [_P, _P, _P, ctypes.c_int, _U32, _U32, _U32, _U32, _U32, _P, _P]),
        "orc_swiglu": (None, [_P, _P, _U32]),
        "orc_gemv": (None, [_P, ctypes.c_int, _U32, _U32, _P, _P]),
        "orc_gemv_scalar": (None, [_P, ctypes.c_int, _U32, _U32, _P, _P]),
        "orc_set_gemv_order": (None, [ctypes.c_int]),
        "orc_add": (None, [_P, _P, _P, _U32]),
        "orc_sample_argmax": (_I32, [_P, _U32]),
        "orc_model_create": (_P, [_P, _P]),
        "orc_model_destroy": (None, [_P]),
        "orc_model_step": (None, [_P, _U32, _U32, _P]),
        "orc_model_key_cache": (_P, [_P, _U32]),
        "orc_model_key_row": (_P, [_P, _U32]),
        "orc_model_value_row": (_P, [_P, _U32]),
        "orc_model_set_kv_store": (None, [_P, ctypes.c_int]),
        "orc_model_value_cache": (_P, [_P, _U32]),
        "orc_generate_tokens": (ctypes.c_int, [_P, _P, _U32, _U32, ctypes.c_int, _I32, _P, _P, _P]),
        "orc_num_threads": (ctypes.c_int, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = _load()


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data


def num_threads() -> int:
    return int(_lib.orc_num_threads())


# ---- bf16 -------------------------------------------------------------------
def to_bf16(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round-to-nearest-even."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    _lib.orc_f32_to_bf16_array(_ptr(a), _ptr(out), a.size)
    return out


def from_bf16(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    _lib.orc_bf16_to_f32_array(_ptr(h), _ptr(out), h.size)
    return out


def storage(a: np.ndarray, dtype: int) -> np.ndarray:
    """fp32 values in the storage format of ``dtype`` (F32 or BF16 bits)."""
    return to_bf16(a) if dtype == BF16 else np.ascontiguousarray(a, dtype=np.float32)


def widen(a: np.ndarray, dtype: int) -> np.ndarray:
    return from_bf16(a) if dtype == BF16 else np.asarray(a, dtype=np.float32)


# ---- seeded inputs ------------------------------------------------------------
def normal(n: int, seed: int, stream: int = 0, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(int(n), dtype=np.float32)
    _lib.orc_fill_normal(_ptr(out), out.size, seed, stream, mean, std)
    return out


def pseudo_random(n: int, seed: int) -> np.ndarray:
    """The reference tests' xorshift32 values in [-1, 1] (tests/kernels.rs:380-390)."""
    out = np.empty(int(n), dtype=np.float32)
    _lib.orc_pseudo_random(_ptr(out), out.size, seed)
    return out


# ---- kernels ------------------------------------------------------------------
def embed(table: np.ndarray, dtype: int, ids) -> np.ndarray:
    vocab, dim = table.shape
    ids = np.ascontiguousarray(ids, dtype=np.uint32).reshape(-1)
    table = np.ascontiguousarray(table)
    x = np.empty((ids.size, dim), dtype=np.float32)
    _lib.orc_embed(_ptr(table), dtype, vocab, dim, _ptr(ids), ids.size, _ptr(x))
    return x


def rmsnorm(x: np.ndarray, w: np.ndarray, w_dtype: int = F32, eps: float = 1e-5) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, dim = (1, x.size) if x.ndim == 1 else x.shape
    w = np.ascontiguousarray(w)
    out = np.empty_like(x)
    _lib.orc_rmsnorm(_ptr(x), _ptr(w), w_dtype, _ptr(out), rows, dim, eps)
    return out


def rope_table(theta: float, head: int, seq: int) -> np.ndarray:
    t = np.empty((seq, head // 2, 2), dtype=np.float32)
    _lib.orc_rope_table(theta, head, seq, _ptr(t))
    return t


def rope_store(q: np.ndarray, k_proj: np.ndarray, k_cache: np.ndarray, kv_dtype: int,
               head: int, pos: int, table: np.ndarray) -> None:
    """In place on ``q`` and ``k_cache`` ([seq, kv_heads, head] storage array)."""
    seq = k_cache.shape[0]
    kv_dim = k_proj.size
    _lib.orc_rope_store(_ptr(q), _ptr(k_proj), _ptr(k_cache), kv_dtype, q.size, kv_dim,
                        head, seq, pos, _ptr(table))


def cache_store(v: np.ndarray, v_cache: np.ndarray, kv_dtype: int, pos: int) -> None:
    _lib.orc_cache_store(_ptr(v), _ptr(v_cache), kv_dtype, v.size, v_cache.shape[0], pos)


def attention_splits(seq: int, split_len: int = 8) -> int:
    return int(_lib.orc_attention_splits(seq, split_len))


def attention_partial(q, k_cache, v_cache, kv_dtype, pos, partial=None):
    q_heads, head = q.shape
    seq, kv_heads, _ = k_cache.shape
    splits = attention_splits(seq)
    if partial is None:
        partial = np.full((q_heads, splits, head + 2), np.nan, dtype=np.float32)
    _lib.orc_attention_partial(_ptr(q), _ptr(k_cache), _ptr(v_cache), kv_dtype, q_heads,
                               kv_heads, head, seq, pos, _ptr(partial))
    return partial


def attention_combine(partial, seq, pos):
    q_heads, _, slot = partial.shape
    head = slot - 2
    out = np.empty((q_heads, head), dtype=np.float32)
    _lib.orc_attention_combine(_ptr(partial), q_heads, head, seq, pos, _ptr(out))
    return out


def attention(q, k_cache, v_cache, kv_dtype, pos):
    """Split (decode-path) attention: partial pass then combine."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    partial = attention_partial(q, k_cache, v_cache, kv_dtype, pos)
    return attention_combine(partial, k_cache.shape[0], pos)


def attention_serial(q, k_cache, v_cache, kv_dtype, pos):
    q = np.ascontiguousarray(q, dtype=np.float32)
    q_heads, head = q.shape
    seq, kv_heads, _ = k_cache.shape
    att = np.zeros((q_heads, seq), dtype=np.float32)
    out = np.empty((q_heads, head), dtype=np.float32)
    _lib.orc_attention_serial(_ptr(q), _ptr(k_cache), _ptr(v_cache), kv_dtype, q_heads,
                              kv_heads, head, seq, pos, _ptr(att), _ptr(out))
    return out


def swiglu(hb: np.ndarray, hb2: np.ndarray) -> np.ndarray:
    out = np.array(hb, dtype=np.float32, copy=True)
    hb2 = np.ascontiguousarray(hb2, dtype=np.float32)
    _lib.orc_swiglu(_ptr(out), _ptr(hb2), out.size)
    return out


def gemv(w: np.ndarray, w_dtype: int, x: np.ndarray) -> np.ndarray:
    d, n = w.shape
    w = np.ascontiguousarray(w)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(d, dtype=np.float32)
    _lib.orc_gemv(_ptr(w), w_dtype, d, n, _ptr(x), _ptr(y))
    return y


def gemv_scalar(w: np.ndarray, w_dtype: int, x: np.ndarray) -> np.ndarray:
    """gemv with one scalar chain per row (the check of the vector path)."""
    d, n = w.shape
    w = np.ascontiguousarray(w)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(d, dtype=np.float32)
    _lib.orc_gemv_scalar(_ptr(w), w_dtype, d, n, _ptr(x), _ptr(y))
    return y


def set_gemv_order(descending: bool) -> None:
    """Every GEMV row summed with j descending (True) or ascending, the
    reference's order (False, the default).  Process-wide; only for
    measuring how far two valid summation orders drift apart."""
    _lib.orc_set_gemv_order(int(bool(descending)))


def add(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.empty_like(a)
    _lib.orc_add(_ptr(a), _ptr(b), _ptr(out), a.size)
    return out


def sample_argmax(logits: np.ndarray) -> int:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    return int(_lib.orc_sample_argmax(_ptr(logits), logits.size))


# ---- test model -----------------------------------------------------------------
class _Config(ctypes.Structure):
    _fields_ = [("dim", _U32), ("n_layers", _U32), ("n_heads", _U32), ("n_kv_heads", _U32),
                ("hidden", _U32), ("vocab", _U32), ("max_seq", _U32), ("theta", _F),
                ("eps", _F), ("w_dtype", ctypes.c_int), ("kv_dtype", ctypes.c_int)]


class _Weights(ctypes.Structure):
    _fields_ = [(n, _P) for n in ("tok_emb", "rms_att", "rms_ffn", "wq", "wk", "wv", "wo",
                                  "w1", "w2", "w3", "rms_final", "wcls")]


@dataclass
class LlamaConfig:
    """Shape of the llama2.c-convention test model."""
    dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    hidden: int
    vocab: int
    max_seq: int
    theta: float = 10000.0
    eps: float = 1e-5
    w_dtype: int = F32
    kv_dtype: int = F32

    @property
    def head(self) -> int:
        return self.dim // self.n_heads

    @property
    def q_dim(self) -> int:
        return self.head * self.n_heads

    @property
    def kv_dim(self) -> int:
        return self.head * self.n_kv_heads


WEIGHT_NAMES = ("tok_emb", "rms_att", "rms_ffn", "wq", "wk", "wv", "wo", "w1", "w2", "w3",
                "rms_final", "wcls")


def weight_shapes(c: LlamaConfig) -> dict:
    L = c.n_layers
    return {
        "tok_emb": (c.vocab, c.dim),
        "rms_att": (L, c.dim),
        "rms_ffn": (L, c.dim),
        "wq": (L, c.q_dim, c.dim),
        "wk": (L, c.kv_dim, c.dim),
        "wv": (L, c.kv_dim, c.dim),
        "wo": (L, c.dim, c.q_dim),
        "w1": (L, c.hidden, c.dim),
        "w2": (L, c.dim, c.hidden),
        "w3": (L, c.hidden, c.dim),
        "rms_final": (c.dim,),
        "wcls": (c.vocab, c.dim),
    }


def random_weights(c: LlamaConfig, seed: int, std: float = 0.02) -> dict:
    """Seeded N(0, std) matrices (stored as ``c.w_dtype``) and unit norm weights."""
    out = {}
    for i, (name, shape) in enumerate(weight_shapes(c).items()):
        n = int(np.prod(shape))
        if name.startswith("rms"):
            out[name] = np.ones(shape, dtype=np.float32)
        else:
            out[name] = storage(normal(n, seed, stream=i, std=std), c.w_dtype).reshape(shape)
    return out


@dataclass
class Model:
    """The oracle's test model holding references to its weight arrays."""
    config: LlamaConfig
    weights: dict
    _handle: int = field(default=0, repr=False)

    def __post_init__(self):
        c = self.config
        cfg = _Config(c.dim, c.n_layers, c.n_heads, c.n_kv_heads, c.hidden, c.vocab, c.max_seq,
                      c.theta, c.eps, c.w_dtype, c.kv_dtype)
        for name in WEIGHT_NAMES:
            self.weights[name] = np.ascontiguousarray(self.weights[name])
        w = _Weights(*[_ptr(self.weights[n]) for n in WEIGHT_NAMES])
        self._handle = _lib.orc_model_create(ctypes.byref(cfg), ctypes.byref(w))

    def close(self):
        if self._handle:
            _lib.orc_model_destroy(self._handle)
            self._handle = 0

    def __del__(self):
        self.close()

    def step(self, token: int, pos: int) -> np.ndarray:
        logits = np.empty(self.config.vocab, dtype=np.float32)
        _lib.orc_model_step(self._handle, token, pos, _ptr(logits))
        return logits

    def kv_layer(self, layer: int):
        """(key, value) caches of ``layer`` as [seq, kv_heads, head] storage arrays."""
        c = self.config
        dt = np.uint16 if c.kv_dtype == BF16 else np.float32
        shape = (c.max_seq, c.n_kv_heads, c.head)
        n = int(np.prod(shape))
        out = []
        for fn in (_lib.orc_model_key_cache, _lib.orc_model_value_cache):
            p = fn(self._handle, layer)
            buf = (ctypes.c_char * (n * np.dtype(dt).itemsize)).from_address(p)
            out.append(np.frombuffer(buf, dtype=dt).reshape(shape).copy())
        return out[0], out[1]

    def _kv_dtype(self):
        return np.uint16 if self.config.kv_dtype == BF16 else np.float32

    def kv_rows(self, layer: int):
        """(key, value) rows [kv_heads, head] (storage arrays) that the
        latest step computed for ``layer``, whether or not it stored them."""
        c = self.config
        dt = self._kv_dtype()
        n = c.n_kv_heads * c.head
        out = []
        for fn in (_lib.orc_model_key_row, _lib.orc_model_value_row):
            buf = (ctypes.c_char * (n * np.dtype(dt).itemsize)).from_address(fn(self._handle, layer))
            out.append(np.frombuffer(buf, dtype=dt).reshape(c.n_kv_heads, c.head).copy())
        return out[0], out[1]

    def set_kv_store(self, on: bool) -> None:
        """Whether steps store their K / V rows into the cache (the default)
        or leave the cache as the caller wrote it (a test that writes the
        position's rows itself)."""
        _lib.orc_model_set_kv_store(self._handle, int(bool(on)))

    def write_kv(self, layer: int, start: int, key: np.ndarray, value: np.ndarray) -> None:
        """Write rows [n, kv_heads, head] (storage arrays in the cache dtype)
        into ``layer``'s caches at positions start .. start + n."""
        c = self.config
        dt = self._kv_dtype()
        row = c.n_kv_heads * c.head * np.dtype(dt).itemsize
        for fn, a in ((_lib.orc_model_key_cache, key), (_lib.orc_model_value_cache, value)):
            a = np.ascontiguousarray(a, dtype=dt).reshape(-1, c.n_kv_heads, c.head)
            if start < 0 or start + a.shape[0] > c.max_seq:
                raise ValueError("write_kv: rows outside the cache")
            ctypes.memmove(fn(self._handle, layer) + start * row, a.ctypes.data, a.nbytes)

    def generate_tokens(self, prompt, max_new_tokens: int, stop_on=None):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(max(int(max_new_tokens), 1), dtype=np.int32)
        n_out = _U32(0)
        logits = np.empty(self.config.vocab, dtype=np.float32)
        rc = _lib.orc_generate_tokens(self._handle, _ptr(prompt), prompt.size, max_new_tokens,
                                      int(stop_on is not None),
                                      int(stop_on) if stop_on is not None else 0,
                                      _ptr(out), ctypes.byref(n_out), _ptr(logits))
        if rc != 0:
            raise ValueError("expected at least one prompt token")
        return out[: n_out.value].copy(), logits
