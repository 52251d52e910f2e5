"""The per-device runtime cache (the reference's prepared-kernel cache,
Blocks::shared over weak references, src/blocks.rs:72-86,322): while any
holder is alive, ammon_runtime_create(device) returns the one shared
runtime; releases are counted, so a release by one holder leaves the runtime
usable for the others; after the last release a create sets the device up
again (code objects reloaded) and the new runtime launches kernels.

Runs in a fresh process: the test session's own runtime would otherwise
hold a reference for the whole session.
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SCRIPT = r"""
import ctypes, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from ammon_amd import _abi
from ammon_amd._abi import call, lib, F32

def create():
    h = ctypes.c_void_p()
    call("ammon_runtime_create", 0, ctypes.byref(h))
    return h

def fill_and_read(h, value):
    # a kernel launch (ammon_fill) and a copy back through the runtime h
    p = ctypes.c_void_p()
    call("ammon_alloc", h, ctypes.c_size_t(64), ctypes.byref(p))
    call("ammon_fill", h, None, p, F32, 16, ctypes.c_float(value))
    call("ammon_stream_synchronize", h, None)
    out = np.empty(16, np.float32)
    call("ammon_memcpy", h, out.ctypes.data, p, 64, _abi.COPY_D2H, None)
    call("ammon_stream_synchronize", h, None)
    call("ammon_free", h, p)
    return out

a = create()
b = create()
assert a.value == b.value, "a second create for the device must return the shared runtime"
print("shared", flush=True)
call("ammon_runtime_release", a)
# one release of two: the runtime (modules, stream) must still serve b
assert (fill_and_read(b, 2.5) == 2.5).all()
info = _abi.DeviceInfo()
call("ammon_runtime_info", b, ctypes.byref(info))
assert info.device == 0 and info.arch.startswith(b"gfx950")
print("refcounted", flush=True)
call("ammon_runtime_release", b)  # the last holder: unloads
c = create()                      # sets the device up again
assert (fill_and_read(c, -1.0) == -1.0).all()
d = create()
assert d.value == c.value
call("ammon_runtime_release", d)
call("ammon_runtime_release", c)
print("reloaded", flush=True)
"""


def test_runtime_cache_is_shared_refcounted_and_reloads():
    r = subprocess.run([sys.executable, "-c", SCRIPT, ROOT], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.split() == ["shared", "refcounted", "reloaded"], r.stdout
