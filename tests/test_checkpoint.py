"""CPU tests of llama2.c checkpoint header parsing (ammon_checkpoint_probe):
both layouts, shared and separate classifiers, and the rejections."""
import struct

import numpy as np
import pytest

import oracle
from ammon_amd import AmmonError
from ammon_amd.model import probe_checkpoint
from oracle import llama2c

CFG = oracle.LlamaConfig(dim=64, n_layers=2, n_heads=4, n_kv_heads=2, hidden=96, vocab=50,
                         max_seq=24, theta=10000.0, w_dtype=oracle.F32, kv_dtype=oracle.F32)


@pytest.fixture(scope="module")
def weights():
    return oracle.random_weights(CFG, seed=3, std=0.1)


@pytest.mark.parametrize("version", [0, 1])
@pytest.mark.parametrize("shared", [False, True])
def test_probe_reads_the_header(tmp_path, weights, version, shared):
    path = tmp_path / "m.bin"
    llama2c.write(path, CFG, weights, version=version, shared=shared)
    cfg, fmt, sh, size = probe_checkpoint(str(path))
    assert (cfg.dim, cfg.hidden, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.vocab,
            cfg.max_seq) == (64, 96, 2, 4, 2, 50, 24)
    assert cfg.theta == 10000.0 and abs(cfg.eps - 1e-5) < 1e-12 and cfg.w_dtype == oracle.F32
    assert fmt == version and sh == shared
    assert size == path.stat().st_size


def test_probe_sizes_need_64_bit_arithmetic(tmp_path):
    # dim 65536: dim * dim is 2^32, which a 32-bit product wraps to 0.  The
    # legacy layout (negative vocab: separate classifier) needs
    # 4 * (V D + 2 L D + D + L (D D + 2 kvd D + D D + 3 H D) + seq head + V D)
    # bytes after the 28-byte header.
    D, H, L, heads, kv, V, S = 65536, 8, 1, 1, 1, 3, 2
    p = tmp_path / "wide.bin"
    p.write_bytes(struct.pack("<7i", D, H, L, heads, kv, -V, S))
    kvd = D // heads * kv
    floats = V * D + 2 * L * D + D + L * (D * D + 2 * kvd * D + D * D + 3 * H * D) + S * D + V * D
    _, _, shared, size = probe_checkpoint(str(p))
    assert not shared and size == 28 + 4 * floats


def test_probe_rejections(tmp_path):
    p = tmp_path / "bad.bin"
    p.write_bytes(struct.pack("<Ii", llama2c.MAGIC, 2) + b"\0" * 300)
    with pytest.raises(AmmonError, match="unsupported export version 2"):
        probe_checkpoint(str(p))
    p.write_bytes(struct.pack("<7i", 64, 96, 0, 4, 2, 50, 24))
    with pytest.raises(AmmonError, match="header field 2 is 0"):
        probe_checkpoint(str(p))
    p.write_bytes(struct.pack("<7i", 64, 96, 2, 5, 2, 50, 24))
    with pytest.raises(AmmonError, match="do not divide"):
        probe_checkpoint(str(p))
    p.write_bytes(struct.pack("<3i", 64, 96, 2))
    with pytest.raises(AmmonError, match="truncated header"):
        probe_checkpoint(str(p))
    with pytest.raises(AmmonError, match="cannot open"):
        probe_checkpoint(str(tmp_path / "missing.bin"))
