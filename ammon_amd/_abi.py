"""ctypes binding of ``include/ammon/ammon.h`` (the C ABI of libammon_amd.so).

This is the Python-side counterpart of the FFI crate a Rust host would bind:
plain pointers and sizes, status codes turned into exceptions.  It loads the
in-tree ``ammon_amd/libammon_amd.so`` only; if the library is missing the
import fails loudly -- there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libammon_amd.so")

OK, E_VALIDATION, E_HIP, E_OOM, E_NO_DEVICE = 0, 1, 2, 3, 4
F32, BF16 = 0, 1
COPY_H2D, COPY_D2H, COPY_D2D = 1, 2, 3
STREAM_VALIDATE = ctypes.c_void_p(1)

ATTENTION_SPLIT_REF = 8
ATTENTION_MAX_HEAD = 128
DEFAULT_ROPE_THETA = 10000.0

_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_I32 = ctypes.c_int32
_U64 = ctypes.c_uint64
_F = ctypes.c_float
_SZ = ctypes.c_size_t
_ST = ctypes.c_int  # ammon_status
_DT = ctypes.c_int  # ammon_dtype


class DecodeStep(ctypes.Structure):
    """ammon_decode_step: {token, position} (reference src/kernels.rs:10-15)."""
    _fields_ = [("token", _U32), ("position", _U32)]


class DeviceInfo(ctypes.Structure):
    _fields_ = [("device", ctypes.c_int), ("compute_units", ctypes.c_int),
                ("max_shared_per_block", ctypes.c_int), ("warp_size", ctypes.c_int),
                ("total_memory", _SZ), ("arch", ctypes.c_char * 64),
                ("name", ctypes.c_char * 128)]


# name -> (restype, argtypes), in the order of include/ammon/ammon.h, then
# include/ammon/ammon_model.h.
SIGNATURES = {
    "ammon_runtime_create": (_ST, [ctypes.c_int, ctypes.POINTER(_P)]),
    "ammon_runtime_release": (_ST, [_P]),
    "ammon_last_error": (ctypes.c_char_p, []),
    "ammon_abi_version": (ctypes.c_int, []),
    "ammon_runtime_info": (_ST, [_P, ctypes.POINTER(DeviceInfo)]),
    "ammon_alloc": (_ST, [_P, _SZ, ctypes.POINTER(_P)]),
    "ammon_free": (_ST, [_P, _P]),
    "ammon_alloc_host": (_ST, [_P, _SZ, ctypes.POINTER(_P)]),
    "ammon_free_host": (_ST, [_P, _P]),
    "ammon_memcpy": (_ST, [_P, _P, _P, _SZ, ctypes.c_int, _P]),
    "ammon_stream_create": (_ST, [_P, ctypes.POINTER(_P)]),
    "ammon_stream_destroy": (_ST, [_P, _P]),
    "ammon_stream_synchronize": (_ST, [_P, _P]),
    "ammon_event_create": (_ST, [_P, ctypes.POINTER(_P)]),
    "ammon_event_destroy": (_ST, [_P, _P]),
    "ammon_event_record": (_ST, [_P, _P, _P]),
    "ammon_event_synchronize": (_ST, [_P, _P]),
    "ammon_event_elapsed_ms": (_ST, [_P, _P, _P, ctypes.POINTER(_F)]),
    "ammon_capture_begin": (_ST, [_P, _P]),
    "ammon_capture_end": (_ST, [_P, _P, ctypes.POINTER(_P)]),
    "ammon_graph_launch": (_ST, [_P, _P, _P]),
    "ammon_graph_destroy": (_ST, [_P, _P]),
    "ammon_fill": (_ST, [_P, _P, _P, _DT, _SZ, _F]),
    "ammon_fill_normal": (_ST, [_P, _P, _P, _DT, _SZ, _U64, _U64, _F, _F]),
    "ammon_checksum": (_ST, [_P, _P, _P, _SZ, _P]),
    "ammon_stream_read": (_ST, [_P, _P, _P, _SZ]),
    "ammon_rope_table_bytes": (_SZ, [_U32, _U32]),
    "ammon_rope_table_host": (_ST, [_F, _U32, _U32, _P]),
    "ammon_kv_unpermute": (_ST, [_P, _P, _U32, _U32, _U32, _U32]),
    "ammon_kv_permute": (_ST, [_P, _P, _U32, _U32, _U32, _U32]),
    "ammon_attention_splits": (_U32, [_U32, _U32]),
    "ammon_attention_scratch_bytes": (_SZ, [_U32, _U32, _U32, _U32]),
    "ammon_attention_default_split": (_U32, [_P, _U32, _U32]),
    "ammon_attention_default_split_for": (_U32, [_P, _U32, _U32, _U32, _DT, _U32]),
    "ammon_embed": (_ST, [_P, _P, _P, _DT, _U32, _U32, _P, _P]),
    "ammon_embed_rows": (_ST, [_P, _P, _P, _DT, _U32, _U32, _P, _U32, _P]),
    "ammon_rmsnorm": (_ST, [_P, _P, _P, _P, _DT, _P, _U32, _U32, _F]),
    "ammon_rope_store": (_ST, [_P, _P, _P, _U32, _P, _U32, _U32, _P, _DT, _U32, _P, _P]),
    "ammon_rope": (_ST, [_P, _P, _P, _U32, _U32, _U32, _P, _DT, _U32, _P, _P]),
    "ammon_cache_store": (_ST, [_P, _P, _P, _U32, _U32, _P, _DT, _U32, _P]),
    "ammon_attention_partial": (_ST, [_P, _P, _P, _U32, _P, _P, _DT, _U32, _U32, _U32, _P,
                                      _U32, _P]),
    "ammon_attention_combine": (_ST, [_P, _P, _P, _U32, _U32, _U32, _P, _U32, _P]),
    "ammon_attention_combine_warm": (_ST, [_P, _P, _P, _U32, _U32, _U32, _P, _U32, _P, _P, _DT,
                                           _U32, _U32, _U32, _U32]),
    "ammon_attention_decode": (_ST, [_P, _P, _P, _U32, _P, _P, _DT, _U32, _U32, _U32, _P,
                                     _U32, _P, _SZ, _P]),
    "ammon_attention_decode_noalloc": (_ST, [_P, _P, _P, _U32, _P, _P, _DT, _U32, _U32, _U32,
                                             _P, _U32, _P]),
    "ammon_swiglu": (_ST, [_P, _P, _P, _P, _U32]),
    "ammon_add": (_ST, [_P, _P, _P, _P, _P, _U32]),
    "ammon_gemv": (_ST, [_P, _P, _P, _DT, _U32, _U32, _P, _P, _P]),
    "ammon_gemv_at_position": (_ST, [_P, _P, _P, _DT, _U32, _U32, _P, _P, _U32, _P]),
    "ammon_gemv_rmsnorm": (_ST, [_P, _P, _P, _P, _DT, _F, _P, _DT, _U32, _U32, _P]),
    "ammon_qkv_rope_store": (_ST, [_P, _P, _P, _P, _DT, _F, _P, _P, _P, _DT, _U32, _U32, _U32,
                                   _U32, _P, _P, _P, _DT, _U32, _P, _P]),
    "ammon_gate_up_swiglu": (_ST, [_P, _P, _P, _P, _DT, _F, _P, _P, _DT, _U32, _U32, _P]),
    "ammon_argmax_scratch_bytes": (_SZ, [_U32]),
    "ammon_argmax": (_ST, [_P, _P, _P, _U32, _P, _P]),
    "ammon_greedy_next": (_ST, [_P, _P, _P, _U32, _P, _P, _U32, _P, _P, _U32]),
    "ammon_greedy_lm_head_scratch_bytes": (_SZ, [_P]),
    "ammon_greedy_lm_head": (_ST, [_P, _P, _P, _P, _DT, _F, _P, _DT, _U32, _U32, _P, _P, _SZ,
                                   _P, _U32, _P, _P, _U32]),
    "ammon_prefill_gemm": (_ST, [_P, _P, _P, _DT, _U32, _U32, _P, _U32, _P, _P]),
    "ammon_prefill_gemm_workspace_bytes": (_SZ, [_U32, _U32]),
    "ammon_prefill_gemm_ws": (_ST, [_P, _P, _P, _DT, _U32, _U32, _P, _U32, _P, _P, _P, _SZ]),
    "ammon_prefill_qkv_rope_store_ws": (_ST, [_P, _P, _P, _U32, _P, _P, _P, _DT, _U32, _U32, _U32,
                                              _U32, _P, _P, _P, _DT, _U32, _P, _P, _P, _SZ]),
    "ammon_prefill_qkv_rope_store": (_ST, [_P, _P, _P, _U32, _P, _P, _P, _DT, _U32, _U32, _U32,
                                           _U32, _P, _P, _P, _DT, _U32, _P, _P]),
    "ammon_prefill_gate_up_swiglu": (_ST, [_P, _P, _P, _U32, _P, _P, _DT, _U32, _U32, _P]),
    "ammon_attention_prefill_scratch_bytes": (_SZ, [_U32, _U32, _U32, _U32, _U32]),
    "ammon_attention_prefill": (_ST, [_P, _P, _P, _U32, _U32, _P, _P, _DT, _U32, _U32, _U32, _P,
                                      _U32, _U32, _P, _SZ, _P]),
}


class LlamaConfig(ctypes.Structure):
    """ammon_llama_config (include/ammon/ammon_model.h)."""
    _fields_ = [("dim", _U32), ("n_layers", _U32), ("n_heads", _U32), ("n_kv_heads", _U32),
                ("hidden", _U32), ("vocab", _U32), ("max_seq", _U32), ("theta", _F),
                ("eps", _F), ("w_dtype", ctypes.c_int), ("kv_dtype", ctypes.c_int),
                ("use_graph", _U32), ("split_len", _U32)]


class LlamaWeights(ctypes.Structure):
    """ammon_llama_weights: device pointers, stacked per layer."""
    _fields_ = [(n, _P) for n in ("tok_emb", "rms_att", "rms_ffn", "wq", "wk", "wv", "wo",
                                  "w1", "w2", "w3", "rms_final", "wcls")]


SIGNATURES.update({
    "ammon_llama_create": (_ST, [_P, ctypes.POINTER(LlamaConfig), ctypes.POINTER(LlamaWeights),
                                 ctypes.POINTER(_P)]),
    "ammon_llama_destroy": (_ST, [_P]),
    "ammon_llama_step": (_ST, [_P, _U32, _U32, _P]),
    "ammon_llama_generate_tokens": (_ST, [_P, _P, _U32, _U32, ctypes.c_int, _I32, _P,
                                          ctypes.POINTER(_U32), ctypes.POINTER(ctypes.c_double),
                                          _P]),
    "ammon_llama_generate_tokens_device": (_ST, [_P, _P, _U32, _U32, ctypes.c_int, _I32, _P,
                                                 ctypes.POINTER(_U32),
                                                 ctypes.POINTER(ctypes.c_double), _P]),
    "ammon_llama_prefill": (_ST, [_P, _P, _U32, _U32, _P]),
    "ammon_llama_generate_tokens_prefill": (_ST, [_P, _P, _U32, _U32, ctypes.c_int, _I32, _P,
                                                  ctypes.POINTER(_U32),
                                                  ctypes.POINTER(ctypes.c_double), _P]),
    "ammon_llama_decode": (_ST, [_P, _U32, _U32, _U32, _P]),
    "ammon_llama_tokens": (_ST, [_P, _U32, _U32, _P]),
    "ammon_llama_kv_layer": (_ST, [_P, _U32, ctypes.POINTER(_P), ctypes.POINTER(_P)]),
    "ammon_llama_stream": (_ST, [_P, ctypes.POINTER(_P)]),
    "ammon_llama_logits": (_ST, [_P, ctypes.POINTER(_P)]),
    "ammon_llama_launches": (_ST, [_P, ctypes.POINTER(_U32)]),
})

# include/ammon/ammon_checkpoint.h
SIGNATURES.update({
    "ammon_checkpoint_probe": (_ST, [ctypes.c_char_p, ctypes.POINTER(LlamaConfig),
                                     ctypes.POINTER(_U32), ctypes.POINTER(_U32),
                                     ctypes.POINTER(_U64)]),
    "ammon_checkpoint_load": (_ST, [_P, ctypes.c_char_p, _DT, ctypes.POINTER(_P)]),
    "ammon_checkpoint_config": (_ST, [_P, ctypes.POINTER(LlamaConfig)]),
    "ammon_checkpoint_weights": (_ST, [_P, ctypes.POINTER(LlamaWeights)]),
    "ammon_checkpoint_free": (_ST, [_P]),
})

# include/ammon/ammon_tokenizer.h
SIGNATURES.update({
    "ammon_bpe_load": (_ST, [ctypes.c_char_p, _U32, ctypes.POINTER(_P)]),
    "ammon_bpe_from_parts": (_ST, [ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_U32),
                                   ctypes.POINTER(_F), _U32, _U32, ctypes.POINTER(_P)]),
    "ammon_bpe_destroy": (_ST, [_P]),
    "ammon_bpe_vocab_size": (_U32, [_P]),
    "ammon_bpe_max_token_length": (_U32, [_P]),
    "ammon_bpe_encode": (_ST, [_P, ctypes.c_char_p, _SZ, ctypes.c_int, ctypes.c_int, _P, _SZ,
                               ctypes.POINTER(_SZ)]),
    "ammon_bpe_decode": (_ST, [_P, _I32, _I32, _P, _SZ, ctypes.POINTER(_SZ)]),
    "ammon_llama_generate_text": (_ST, [_P, _P, ctypes.c_char_p, _SZ, _U32, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int, _I32, ctypes.c_int, _P, _SZ,
                                        ctypes.POINTER(_SZ), _P, _U32, ctypes.POINTER(_U32),
                                        ctypes.POINTER(ctypes.c_double)]),
})


class AmmonError(RuntimeError):
    """A non-OK ammon_status with the library's thread-local message."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[status {status}] {message}")
        self.status = status
        self.message = message


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
            f"g.build()'` (make -C ammon_amd/csrc)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def last_error() -> str:
    msg = lib.ammon_last_error()
    return msg.decode() if msg else ""


def check(status: int) -> None:
    if status != OK:
        raise AmmonError(int(status), last_error())


def call(name: str, *args) -> None:
    """Call a status-returning ABI function and raise on failure."""
    check(getattr(lib, name)(*args))
