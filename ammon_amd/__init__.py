"""ammon_amd -- MI355X (gfx950) decode-layer kernels of koubaa/ammon.

The product is ``libammon_amd.so``: hand-written HIP kernels behind the C ABI
in ``include/ammon/ammon.h`` and a C++ host layer mirroring Ammon's module
API (``include/ammon/ammon.hpp``).  This Python package is a thin ctypes
binding over that library for tests and benchmarks; importing it fails if
the library has not been built.
"""
from . import _abi
from ._abi import (ATTENTION_MAX_HEAD, ATTENTION_SPLIT_REF, BF16, DEFAULT_ROPE_THETA, F32,
                   AmmonError, DecodeStep)
from .runtime import (DeviceBuffer, Runtime, Timer, argmax_scratch_bytes, attention_scratch_bytes,
                      attention_splits, kv_permute, kv_unpermute, rope_table_host, storage_dtype)

from . import model
from .model import LlamaModel
from .tokenizer import BpeTokenizer

LIB_PATH = _abi.LIB_PATH

__all__ = [
    "ATTENTION_MAX_HEAD", "ATTENTION_SPLIT_REF", "BF16", "DEFAULT_ROPE_THETA", "F32",
    "AmmonError", "DecodeStep", "DeviceBuffer", "Runtime", "Timer", "argmax_scratch_bytes",
    "attention_scratch_bytes", "attention_splits", "kv_permute", "kv_unpermute",
    "rope_table_host", "storage_dtype", "LIB_PATH", "LlamaModel", "model", "BpeTokenizer",
]
