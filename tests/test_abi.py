"""CPU tests of the C ABI: the library loads, exports every function the
public headers declare, and its host-only utilities behave (no device used).
"""
import ctypes
import os
import re

import numpy as np
import pytest

import ammon_amd
import oracle
from ammon_amd import _abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", "ammon", h)
           for h in sorted(os.listdir(os.path.join(ROOT, "include", "ammon"))) if h.endswith(".h")]


def declared_functions():
    names = set()
    for path in HEADERS:
        text = open(path).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(ammon_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return sorted(names)


def test_headers_declare_functions():
    names = declared_functions()
    assert "ammon_runtime_create" in names and "ammon_qkv_rope_store" in names
    assert len(names) >= 40


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_abi.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_covers_every_header_function():
    assert set(declared_functions()) <= set(_abi.SIGNATURES), \
        sorted(set(declared_functions()) - set(_abi.SIGNATURES))


def test_abi_version():
    assert _abi.lib.ammon_abi_version() == 1


def test_rope_table_host_matches_oracle_bitwise():
    for theta, head, seq in ((10000.0, 48, 256), (500000.0, 128, 8192), (10000.0, 2, 3)):
        np.testing.assert_array_equal(ammon_amd.rope_table_host(theta, head, seq),
                                      oracle.rope_table(theta, head, seq))
    assert _abi.lib.ammon_rope_table_bytes(128, 8192) == 8192 * 64 * 2 * 4


def test_rope_table_rejects_odd_head():
    out = np.empty(16, np.float32)
    assert _abi.lib.ammon_rope_table_host(10000.0, 3, 2, out.ctypes.data) == _abi.E_VALIDATION
    assert "even" in _abi.last_error()


@pytest.mark.parametrize("dtype", [np.float32, np.uint16])
def test_kv_permute_round_trip(dtype):
    kv_heads, seq, head = 3, 7, 4
    pm = np.arange(seq * kv_heads * head).astype(dtype).reshape(seq, kv_heads, head)
    hm = ammon_amd.kv_permute(pm, kv_heads, seq, head)
    np.testing.assert_array_equal(hm, pm.transpose(1, 0, 2))
    np.testing.assert_array_equal(ammon_amd.kv_unpermute(hm, kv_heads, seq, head), pm)


def test_attention_scratch_geometry():
    # reference src/blocks.rs:317-320 and src/modules.rs:223-227 at split 8
    assert ammon_amd.attention_splits(256, 8) == 32
    assert ammon_amd.attention_splits(33, 8) == 5
    assert ammon_amd.attention_splits(0, 8) == 1
    assert ammon_amd.attention_scratch_bytes(6, 48, 256, 8) == 6 * 32 * 50 * 4
    split = _abi.lib.ammon_attention_default_split(None, 8, 8192)
    assert 16 <= split <= 1024 and split & (split - 1) == 0
    assert 8 * ammon_amd.attention_splits(8192, split) <= 2 * 256
    assert split == 128
    # without a runtime there is no kernel to size for: two units per CU
    for q_heads, kv_heads, seq in ((32, 8, 8192), (64, 8, 32768), (6, 6, 1000), (8, 8, 256)):
        assert (_abi.lib.ammon_attention_default_split_for(None, q_heads, kv_heads, 128,
                                                           _abi.BF16, seq)
                == _abi.lib.ammon_attention_default_split(None, kv_heads, seq))


def test_null_runtime_is_a_validation_error():
    st = _abi.lib.ammon_gemv(None, None, None, 0, 2, 2, None, None, None)
    assert st == _abi.E_VALIDATION
    assert "runtime is NULL" in _abi.last_error()
    with pytest.raises(_abi.AmmonError):
        _abi.call("ammon_swiglu", None, None, None, None, 4)


def test_argmax_scratch_bytes():
    assert _abi.lib.ammon_argmax_scratch_bytes(4) == 8
    assert _abi.lib.ammon_argmax_scratch_bytes(128256) == 251 * 8  # ceil(n / 512) blocks
    assert _abi.lib.ammon_argmax_scratch_bytes(1 << 20) == 256 * 8  # capped at 256
