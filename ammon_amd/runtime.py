"""Host-side helpers over the C ABI: a device runtime handle and device buffers.

``Runtime`` mirrors the reference's ``create_runtime`` (src/gpu.rs:6-13): it
holds an ``ammon_runtime`` (device bootstrap + prepared-kernel cache, shared
per device).  ``DeviceBuffer`` is a caller-owned device allocation, the
counterpart of a Goldy ``Tensor``'s storage.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _abi
from ._abi import BF16, F32, DecodeStep, call, lib

_NP_DTYPES = {F32: np.float32, BF16: np.uint16}


def storage_dtype(dtype: int):
    return _NP_DTYPES[dtype]


class DeviceBuffer:
    """A device allocation of ``nbytes`` owned by this object."""

    def __init__(self, rt: "Runtime", nbytes: int):
        self.rt = rt
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        call("ammon_alloc", rt.handle, ctypes.c_size_t(self.nbytes), ctypes.byref(p))
        self.ptr = p.value or 0

    def __int__(self) -> int:
        return self.ptr

    @property
    def _as_parameter_(self):
        return ctypes.c_void_p(self.ptr)

    def offset(self, nbytes: int) -> ctypes.c_void_p:
        """Raw pointer ``nbytes`` into the buffer (a view, not owned)."""
        assert 0 <= nbytes <= self.nbytes
        return ctypes.c_void_p(self.ptr + int(nbytes))

    def upload(self, array: np.ndarray, stream=None) -> "DeviceBuffer":
        a = np.ascontiguousarray(array)
        assert a.nbytes <= self.nbytes, (a.nbytes, self.nbytes)
        call("ammon_memcpy", self.rt.handle, ctypes.c_void_p(self.ptr), a.ctypes.data,
             a.nbytes, _abi.COPY_H2D, stream)
        self.rt.synchronize(stream)
        return self

    def download(self, shape, dtype=np.float32, stream=None) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes, (out.nbytes, self.nbytes)
        self.rt.synchronize(stream)
        call("ammon_memcpy", self.rt.handle, out.ctypes.data, ctypes.c_void_p(self.ptr),
             out.nbytes, _abi.COPY_D2H, stream)
        self.rt.synchronize(stream)
        return out

    def free(self) -> None:
        if self.ptr:
            call("ammon_free", self.rt.handle, ctypes.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            if self.ptr and self.rt.handle:
                lib.ammon_free(self.rt.handle, ctypes.c_void_p(self.ptr))
                self.ptr = 0
        except Exception:
            pass


class Runtime:
    """One device's ammon_runtime (reference create_runtime, src/gpu.rs:6-13)."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        call("ammon_runtime_create", device, ctypes.byref(h))
        self.handle = h
        self.device = device
        info = _abi.DeviceInfo()
        call("ammon_runtime_info", self.handle, ctypes.byref(info))
        self.info = info

    def close(self) -> None:
        if self.handle:
            call("ammon_runtime_release", self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- memory ----------------------------------------------------------
    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, max(int(nbytes), 1))

    def upload(self, array: np.ndarray) -> DeviceBuffer:
        a = np.ascontiguousarray(array)
        return self.alloc(a.nbytes).upload(a)

    def step(self, token: int, position: int) -> DeviceBuffer:
        """A device-resident DecodeStep parcel (reference DecodeStep::parcel)."""
        s = DecodeStep(token, position)
        buf = self.alloc(ctypes.sizeof(DecodeStep))
        call("ammon_memcpy", self.handle, ctypes.c_void_p(buf.ptr), ctypes.addressof(s),
             ctypes.sizeof(s), _abi.COPY_H2D, None)
        self.synchronize()
        return buf

    def deposit(self, buf: DeviceBuffer, token: int, position: int, stream=None) -> None:
        """Overwrite a DecodeStep parcel (the reference's MemoryExchange deposit)."""
        s = DecodeStep(token, position)
        call("ammon_memcpy", self.handle, ctypes.c_void_p(buf.ptr), ctypes.addressof(s),
             ctypes.sizeof(s), _abi.COPY_H2D, stream)
        self.synchronize(stream)

    def read_step(self, buf: DeviceBuffer):
        s = DecodeStep()
        self.synchronize()
        call("ammon_memcpy", self.handle, ctypes.addressof(s), ctypes.c_void_p(buf.ptr),
             ctypes.sizeof(s), _abi.COPY_D2H, None)
        self.synchronize()
        return int(s.token), int(s.position)

    def synchronize(self, stream=None) -> None:
        call("ammon_stream_synchronize", self.handle, stream)

    # ---- fills ------------------------------------------------------------
    def fill(self, buf, dtype: int, count: int, value: float, stream=None) -> None:
        call("ammon_fill", self.handle, stream, buf, dtype, count, value)

    def fill_normal(self, buf, dtype: int, count: int, seed: int, stream_id: int,
                    mean: float = 0.0, std: float = 1.0, stream=None) -> None:
        call("ammon_fill_normal", self.handle, stream, buf, dtype, count, seed, stream_id,
             mean, std)


class Timer:
    """HIP event pair on a stream (for per-kernel timing)."""

    def __init__(self, rt: Runtime):
        self.rt = rt
        a, b = ctypes.c_void_p(), ctypes.c_void_p()
        call("ammon_event_create", rt.handle, ctypes.byref(a))
        call("ammon_event_create", rt.handle, ctypes.byref(b))
        self.start_ev, self.stop_ev = a, b

    def start(self, stream=None):
        call("ammon_event_record", self.rt.handle, self.start_ev, stream)

    def stop(self, stream=None):
        call("ammon_event_record", self.rt.handle, self.stop_ev, stream)

    def elapsed_ms(self) -> float:
        call("ammon_event_synchronize", self.rt.handle, self.stop_ev)
        ms = ctypes.c_float()
        call("ammon_event_elapsed_ms", self.rt.handle, self.start_ev, self.stop_ev,
             ctypes.byref(ms))
        return float(ms.value)

    def close(self):
        for ev in (self.start_ev, self.stop_ev):
            if ev:
                lib.ammon_event_destroy(self.rt.handle, ev)
        self.start_ev = self.stop_ev = None


def rope_table_host(theta: float, head: int, seq: int) -> np.ndarray:
    """The cos/sin table the kernels read ([seq, head/2, 2] fp32), built on the host."""
    t = np.empty((seq, head // 2, 2), dtype=np.float32)
    call("ammon_rope_table_host", theta, head, seq, t.ctypes.data)
    return t


def kv_unpermute(head_major: np.ndarray, kv_heads: int, seq: int, head: int) -> np.ndarray:
    """[kv_heads, seq, head] -> reference layout [seq, kv_heads, head]."""
    src = np.ascontiguousarray(head_major)
    out = np.empty((seq, kv_heads, head), dtype=src.dtype)
    call("ammon_kv_unpermute", src.ctypes.data, out.ctypes.data, kv_heads, seq, head,
         src.dtype.itemsize)
    return out


def kv_permute(pos_major: np.ndarray, kv_heads: int, seq: int, head: int) -> np.ndarray:
    """Reference layout [seq, kv_heads, head] -> [kv_heads, seq, head]."""
    src = np.ascontiguousarray(pos_major)
    out = np.empty((kv_heads, seq, head), dtype=src.dtype)
    call("ammon_kv_permute", src.ctypes.data, out.ctypes.data, kv_heads, seq, head,
         src.dtype.itemsize)
    return out


def attention_splits(seq: int, split_len: int) -> int:
    return int(lib.ammon_attention_splits(seq, split_len))


def attention_scratch_bytes(q_heads: int, head: int, seq: int, split_len: int) -> int:
    return int(lib.ammon_attention_scratch_bytes(q_heads, head, seq, split_len))


def argmax_scratch_bytes(n: int) -> int:
    return int(lib.ammon_argmax_scratch_bytes(n))
