"""Python handle on the C++ host layer's test model (include/ammon/ammon_model.h).

``LlamaModel`` wraps ``ammon_llama``: the llama2.c-convention graph the C++
layer records from its modules (Embedding, CausalAttentionBlock,
SwiGluBlock, Linear with the final norm) and replays per token as a HIP
graph.  ``step`` is the reference's ``AutoregressiveModel::step``
(src/model.rs:10); ``generate_tokens`` is its greedy loop
(src/generate.rs:43-91); ``generate_tokens_device`` runs the same loop with
the argmax and DecodeStep update on the device.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _abi
from ._abi import BF16, F32, call
from .runtime import Runtime

WEIGHT_NAMES = ("tok_emb", "rms_att", "rms_ffn", "wq", "wk", "wv", "wo", "w1", "w2", "w3",
                "rms_final", "wcls")


def weight_shapes(cfg) -> dict:
    head = cfg.dim // cfg.n_heads
    q_dim, kv_dim, L = head * cfg.n_heads, head * cfg.n_kv_heads, cfg.n_layers
    return {
        "tok_emb": (cfg.vocab, cfg.dim), "rms_att": (L, cfg.dim), "rms_ffn": (L, cfg.dim),
        "wq": (L, q_dim, cfg.dim), "wk": (L, kv_dim, cfg.dim), "wv": (L, kv_dim, cfg.dim),
        "wo": (L, cfg.dim, q_dim), "w1": (L, cfg.hidden, cfg.dim),
        "w2": (L, cfg.dim, cfg.hidden), "w3": (L, cfg.hidden, cfg.dim),
        "rms_final": (cfg.dim,), "wcls": (cfg.vocab, cfg.dim),
    }


def weight_dtype(cfg, name: str) -> int:
    return F32 if name.startswith("rms") else cfg.w_dtype


class CheckpointConfig:
    """A model shape read from a checkpoint header (attributes as the C
    config's fields)."""

    def __init__(self, c):
        for name, _ in _abi.LlamaConfig._fields_:
            setattr(self, name, getattr(c, name))


def probe_checkpoint(path: str):
    """(CheckpointConfig, layout 0 legacy / 1 version 1, shared classifier,
    expected file bytes) from the header alone (no device)."""
    c, fmt, shared, size = _abi.LlamaConfig(), ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64()
    call("ammon_checkpoint_probe", str(path).encode(), ctypes.byref(c), ctypes.byref(fmt),
         ctypes.byref(shared), ctypes.byref(size))
    return CheckpointConfig(c), fmt.value, bool(shared.value), size.value


class Checkpoint:
    """Device weights loaded by ammon_checkpoint_load."""

    def __init__(self, rt: Runtime, path: str, w_dtype: int = F32):
        self.rt = rt
        h = ctypes.c_void_p()
        call("ammon_checkpoint_load", rt.handle, str(path).encode(), w_dtype, ctypes.byref(h))
        self.handle = h

    def config(self) -> CheckpointConfig:
        c = _abi.LlamaConfig()
        call("ammon_checkpoint_config", self.handle, ctypes.byref(c))
        return CheckpointConfig(c)

    def weights(self) -> dict:
        w = _abi.LlamaWeights()
        call("ammon_checkpoint_weights", self.handle, ctypes.byref(w))
        return {n: getattr(w, n) for n in WEIGHT_NAMES}

    def close(self) -> None:
        if self.handle:
            call("ammon_checkpoint_free", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class LlamaModel:
    """A device model over caller-owned device weights.

    ``cfg`` is any object with dim, n_layers, n_heads, n_kv_heads, hidden,
    vocab, max_seq, theta, eps, w_dtype, kv_dtype.
    """

    def __init__(self, rt: Runtime, cfg, weights: dict, use_graph: bool = True,
                 split_len: int = 0):
        self.rt = rt
        self.cfg = cfg
        self.weights = weights  # keeps the device buffers alive
        c = _abi.LlamaConfig(cfg.dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.hidden,
                             cfg.vocab, cfg.max_seq, cfg.theta, cfg.eps, cfg.w_dtype,
                             cfg.kv_dtype, int(use_graph), split_len)
        w = _abi.LlamaWeights(*[ctypes.c_void_p(int(weights[n])) for n in WEIGHT_NAMES])
        h = ctypes.c_void_p()
        call("ammon_llama_create", rt.handle, ctypes.byref(c), ctypes.byref(w), ctypes.byref(h))
        self.handle = h
        self.head = cfg.dim // cfg.n_heads

    @classmethod
    def from_host(cls, rt: Runtime, cfg, host_weights: dict, **kw) -> "LlamaModel":
        """Upload host arrays (storage dtype: fp32, or bf16 bit patterns)."""
        dev = {n: rt.upload(np.ascontiguousarray(host_weights[n])) for n in WEIGHT_NAMES}
        return cls(rt, cfg, dev, **kw)

    @classmethod
    def synthetic(cls, rt: Runtime, cfg, seed: int, std: float = 0.02, **kw) -> "LlamaModel":
        """Seeded N(0, std) matrices generated on the device; norm weights 1."""
        dev = {}
        for i, (name, shape) in enumerate(weight_shapes(cfg).items()):
            n = int(np.prod(shape))
            dt = weight_dtype(cfg, name)
            buf = rt.alloc(n * (2 if dt == BF16 else 4))
            if name.startswith("rms"):
                rt.fill(buf, F32, n, 1.0)
            else:
                rt.fill_normal(buf, dt, n, seed, i, 0.0, std)
            dev[name] = buf
        rt.synchronize()
        return cls(rt, cfg, dev, **kw)

    @classmethod
    def from_checkpoint(cls, rt: Runtime, path: str, w_dtype: int = F32, kv_dtype: int = None,
                        max_seq: int = None, theta: float = None, **kw) -> "LlamaModel":
        """A llama2.c checkpoint (legacy or version-1 layout) loaded onto the
        device in w_dtype; the shape comes from its header (max_seq and theta
        may be overridden: the file carries neither theta nor a KV budget)."""
        ck = Checkpoint(rt, path, w_dtype)
        cfg = ck.config()
        if kv_dtype is not None:
            cfg.kv_dtype = kv_dtype
        if max_seq is not None:
            cfg.max_seq = max_seq
        if theta is not None:
            cfg.theta = theta
        m = cls(rt, cfg, ck.weights(), **kw)
        m.checkpoint = ck  # keeps the device weights alive
        return m

    def close(self) -> None:
        if self.handle:
            call("ammon_llama_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- AutoregressiveModel ----------------------------------------------
    def step(self, token: int, pos: int) -> np.ndarray:
        logits = np.empty(self.cfg.vocab, np.float32)
        call("ammon_llama_step", self.handle, token, pos, logits.ctypes.data)
        return logits

    def _generate(self, fn, prompt, max_new_tokens, stop_on):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(max(int(max_new_tokens), 1), np.int32)
        n = ctypes.c_uint32()
        tps = ctypes.c_double()
        logits = np.empty(self.cfg.vocab, np.float32)
        call(fn, self.handle, prompt.ctypes.data, prompt.size, max_new_tokens,
             int(stop_on is not None), int(stop_on or 0), out.ctypes.data, ctypes.byref(n),
             ctypes.byref(tps), logits.ctypes.data)
        return out[: n.value].copy(), logits, tps.value

    def generate_tokens(self, prompt, max_new_tokens: int, stop_on=None):
        """Reference greedy loop with host argmax: (tokens, last logits, tok/s)."""
        return self._generate("ammon_llama_generate_tokens", prompt, max_new_tokens, stop_on)

    def generate_tokens_device(self, prompt, max_new_tokens: int, stop_on=None):
        """Same loop, argmax and prompt forcing on the device."""
        return self._generate("ammon_llama_generate_tokens_device", prompt, max_new_tokens,
                              stop_on)

    def generate_tokens_prefill(self, prompt, max_new_tokens: int, stop_on=None):
        """Same loop with the prompt prefilled in one pass (GEMMs on matrix
        cores, token-batched attention) before the device greedy steps."""
        return self._generate("ammon_llama_generate_tokens_prefill", prompt, max_new_tokens,
                              stop_on)

    def generate_text(self, tokenizer, prompt: str, max_new_tokens: int = 50, bos: bool = True,
                      eos: bool = False, stop_on=None, loop: str = "host"):
        """The reference's generate (src/generate.rs:93-118): (text, tokens,
        tok/s).  loop: "host" (argmax on the host per step, the reference's
        loop), "device" (device greedy loop) or "prefill" (one-pass prompt
        prefill, then the device loop)."""
        modes = {"host": 0, "device": 1, "prefill": 2}
        data = prompt.encode()
        cap = 1 << 16
        text = ctypes.create_string_buffer(cap)
        tokens = np.empty(max(int(max_new_tokens), 1), np.int32)
        tlen, n, tps = ctypes.c_size_t(), ctypes.c_uint32(), ctypes.c_double()
        call("ammon_llama_generate_text", self.handle, tokenizer.handle, data, len(data),
             max_new_tokens, int(bos), int(eos), int(stop_on is not None), int(stop_on or 0),
             modes[loop], text, cap, ctypes.byref(tlen), tokens.ctypes.data, tokens.size,
             ctypes.byref(n), ctypes.byref(tps))
        if tlen.value >= cap:
            raise RuntimeError("generated text exceeds the 64 KiB buffer")
        return text.raw[: tlen.value].decode(), tokens[: n.value].copy(), tps.value

    def prefill(self, tokens, start_pos: int = 0) -> np.ndarray:
        """Run tokens at positions start_pos.. in one pass; the last
        position's logits."""
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        logits = np.empty(self.cfg.vocab, np.float32)
        call("ammon_llama_prefill", self.handle, tokens.ctypes.data, tokens.size, start_pos,
             logits.ctypes.data)
        return logits

    def decode(self, token: int, start_pos: int, n_steps: int, read_tokens: bool = False):
        """Enqueue n_steps device-greedy steps from (token, start_pos)."""
        toks = np.empty(n_steps, np.int32) if read_tokens else None
        call("ammon_llama_decode", self.handle, token, start_pos, n_steps,
             toks.ctypes.data if toks is not None else None)
        return toks

    def read_tokens(self, start: int, n: int) -> np.ndarray:
        """Tokens the device greedy step wrote for positions [start, start + n)."""
        out = np.empty(n, np.int32)
        call("ammon_llama_tokens", self.handle, start, n, out.ctypes.data)
        return out

    # ---- introspection ------------------------------------------------------
    @property
    def stream(self):
        s = ctypes.c_void_p()
        call("ammon_llama_stream", self.handle, ctypes.byref(s))
        return s

    @property
    def launches(self) -> int:
        n = ctypes.c_uint32()
        call("ammon_llama_launches", self.handle, ctypes.byref(n))
        return n.value

    def synchronize(self) -> None:
        self.rt.synchronize(self.stream)

    def kv_layer(self, layer: int):
        """(key, value) of `layer` in the reference order [seq, kv_heads, head]."""
        from .runtime import kv_unpermute
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        call("ammon_llama_kv_layer", self.handle, layer, ctypes.byref(k), ctypes.byref(v))
        c = self.cfg
        dt = np.uint16 if c.kv_dtype == BF16 else np.float32
        shape = (c.n_kv_heads, c.max_seq, self.head)
        out = []
        self.synchronize()
        for ptr in (k, v):
            a = np.empty(shape, dt)
            call("ammon_memcpy", self.rt.handle, a.ctypes.data, ptr, a.nbytes, _abi.COPY_D2H,
                 None)
            self.rt.synchronize()
            out.append(kv_unpermute(a, c.n_kv_heads, c.max_seq, self.head))
        return out[0], out[1]

