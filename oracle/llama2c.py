"""llama2.c checkpoint images -- TEST INFRASTRUCTURE.

Writes fp32 model weights in the two public layouts of karpathy/llama2.c
(a third-party project, not part of the reference or of this repository;
no version is pinned here, the layouts are restated from its run.c
``read_checkpoint`` / ``memory_map_weights`` and export.py
``legacy_export`` / ``version1_export``):

- legacy: 7 little-endian int32 (dim, hidden_dim, n_layers, n_heads,
  n_kv_heads, vocab_size -- negated when the classifier is not the
  embedding table -- and seq_len), then fp32 token_embedding [vocab, dim],
  rms_att [L, dim], wq [L, dim, dim], wk [L, kv_dim, dim], wv, wo
  [L, dim, dim], rms_ffn [L, dim], w1 [L, hidden, dim], w2 [L, dim, hidden],
  w3, rms_final [dim], freq_cis_real and freq_cis_imag [seq_len, head/2]
  (which run.c skips), then the classifier [vocab, dim] when not shared;
- version 1: uint32 0x616b3432 ("ak42"), int32 1, the same 7 int32 (vocab
  positive), uint8 shared_classifier, zeros to 256 bytes, then rms_att,
  rms_ffn, rms_final, token_embedding, wq, wk, wv, wo, w1, w2, w3 and the
  classifier when not shared.

Matrices are [out, in] row-major (the ``matmul(xout, x, w, n, d)`` of run.c
reads ``w[i * n + j]`` for output i), the layout the model here uses.
Only tests/ use this module.
"""
from __future__ import annotations

import struct

import numpy as np

MAGIC = 0x616B3432


def _f32(a) -> bytes:
    return np.ascontiguousarray(a, dtype=np.float32).tobytes()


def write(path, cfg, weights: dict, version: int = 0, shared: bool = False) -> None:
    """weights: fp32 arrays named as oracle.weight_shapes (tok_emb, rms_att,
    rms_ffn, wq, wk, wv, wo, w1, w2, w3, rms_final, wcls); with shared, wcls
    is taken to be tok_emb."""
    head = cfg.dim // cfg.n_heads
    vocab = cfg.vocab if shared or version == 1 else -cfg.vocab
    dims = struct.pack("<7i", cfg.dim, cfg.hidden, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads,
                       vocab, cfg.max_seq)
    w = weights
    with open(path, "wb") as f:
        if version == 0:
            f.write(dims)
            for name in ("tok_emb", "rms_att", "wq", "wk", "wv", "wo", "rms_ffn", "w1", "w2",
                         "w3", "rms_final"):
                f.write(_f32(w[name]))
            rope = np.zeros(cfg.max_seq * head // 2, np.float32) + 0.5  # skipped by the reader
            f.write(_f32(rope))
            f.write(_f32(rope))
        else:
            header = struct.pack("<Ii", MAGIC, 1) + dims + struct.pack("<B", int(shared))
            f.write(header + b"\0" * (256 - len(header)))
            for name in ("rms_att", "rms_ffn", "rms_final", "tok_emb", "wq", "wk", "wv", "wo",
                         "w1", "w2", "w3"):
                f.write(_f32(w[name]))
        if not shared:
            f.write(_f32(w["wcls"]))
