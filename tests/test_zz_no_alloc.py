"""GPU tests of ammon_attention_decode_noalloc, the attention decode pair with
the split partials in the library's own per-GPU scratch (no counterpart in
the reference: it serves callers that cannot allocate device memory).

Its output must equal ammon_attention_decode's with a caller buffer bit for
bit -- same kernels, same split -- on calls in a row, each smaller than the
one before (the scratch keeps the previous call's contents), including a
cache one split covers (pass 1 then writes the output and the scratch is
not touched); captured into a HIP graph and replayed, each replay at a new
position, it must again equal the caller-buffer call; and it must reject
shapes whose partials exceed the scratch.  Collected last (the file name
sorts last) so a failure here cannot hide other tests under -x.
"""
import ctypes

import numpy as np
import pytest

import oracle
from ammon_amd import AmmonError, _abi
from ammon_amd._abi import BF16, F32, call

pytestmark = pytest.mark.gpu

SCRATCH = 4 << 20


def head_major(pm, kv_heads, seq, head):
    return np.ascontiguousarray(pm.reshape(seq, kv_heads, head).transpose(1, 0, 2))


def inputs(rt, case):
    q_heads, kv_heads, head, seq, pos, split, kv_dtype, seed = case
    qh = oracle.normal(q_heads * head, seed).reshape(q_heads, head)
    kh = oracle.storage(oracle.normal(seq * kv_heads * head, seed + 1), kv_dtype)
    vh = oracle.storage(oracle.normal(seq * kv_heads * head, seed + 2), kv_dtype)
    q = rt.upload(qh)
    kc = rt.upload(head_major(kh, kv_heads, seq, head))
    vc = rt.upload(head_major(vh, kv_heads, seq, head))
    return qh, kh, vh, q, kc, vc


def attend(rt, case, noalloc):
    q_heads, kv_heads, head, seq, pos, split, kv_dtype, seed = case
    qh, kh, vh, q, kc, vc = inputs(rt, case)
    out = rt.alloc(q_heads * head * 4)
    step = rt.step(0, pos)
    if noalloc:
        call("ammon_attention_decode_noalloc", rt.handle, None, q, q_heads, kc, vc, kv_dtype,
             kv_heads, head, seq, step, split, out)
    else:
        nbytes = _abi.lib.ammon_attention_scratch_bytes(q_heads, head, seq, split)
        part = rt.alloc(nbytes)
        call("ammon_attention_decode", rt.handle, None, q, q_heads, kc, vc, kv_dtype, kv_heads,
             head, seq, step, split, part, nbytes, out)
    got = out.download((q_heads, head))
    want = oracle.attention(qh, kh.reshape(seq, kv_heads, head), vh.reshape(seq, kv_heads, head),
                            kv_dtype, pos)
    return got, want


# (q_heads, kv_heads, head, seq, position, split, kv dtype, seed): the
# Llama-3-8B attention at context 8192 with the library's split, then a
# smaller one (fewer heads, shorter cache, another position and split), then
# a 256-position cache with one split (the scratch is not written)
CASES = [
    (32, 8, 128, 8192, 8191, 128, BF16, 71),
    (8, 2, 64, 1024, 700, 32, F32, 81),
    (32, 8, 128, 256, 200, 256, BF16, 91),
]


def test_noalloc_matches_caller_buffer_on_two_calls(rt):
    for case in CASES:
        print(f"noalloc case {case}", flush=True)
        got, want = attend(rt, case, noalloc=True)
        ref, _ = attend(rt, case, noalloc=False)
        np.testing.assert_array_equal(got, ref)
        err = float(np.max(np.abs(got - want)) / np.max(np.abs(want)))
        assert err <= 1e-5, (case, err)


def test_noalloc_captured_in_a_graph_and_replayed(rt):
    # The use the entry point is for: recorded under HIP graph capture (no
    # allocation may happen there), then replayed.  Each replay reads the
    # position from the DecodeStep, which eager work between the replays
    # moves; every replay must equal the caller-buffer call at that position.
    case = (32, 8, 128, 4096, 4095, 64, BF16, 101)
    q_heads, kv_heads, head, seq, _, split, kv_dtype, _ = case
    qh, kh, vh, q, kc, vc = inputs(rt, case)
    out, ref = rt.alloc(q_heads * head * 4), rt.alloc(q_heads * head * 4)
    nbytes = _abi.lib.ammon_attention_scratch_bytes(q_heads, head, seq, split)
    part = rt.alloc(nbytes)
    step = rt.step(0, 0)
    call("ammon_capture_begin", rt.handle, None)
    call("ammon_attention_decode_noalloc", rt.handle, None, q, q_heads, kc, vc, kv_dtype,
         kv_heads, head, seq, step, split, out)
    graph = ctypes.c_void_p()
    call("ammon_capture_end", rt.handle, None, ctypes.byref(graph))
    try:
        for pos in (4095, 63, 2000, 4095):
            print(f"noalloc graph replay at position {pos}", flush=True)
            rt.deposit(step, 0, pos)
            call("ammon_graph_launch", rt.handle, graph, None)
            rt.synchronize()
            got = out.download((q_heads, head))
            call("ammon_attention_decode", rt.handle, None, q, q_heads, kc, vc, kv_dtype,
                 kv_heads, head, seq, step, split, part, nbytes, ref)
            want = ref.download((q_heads, head))
            np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
            f64 = oracle.attention(qh, kh.reshape(seq, kv_heads, head),
                                   vh.reshape(seq, kv_heads, head), kv_dtype, pos)
            assert float(np.max(np.abs(got - f64)) / np.max(np.abs(f64))) <= 1e-5, pos
    finally:
        call("ammon_graph_destroy", rt.handle, graph)


def test_noalloc_rejects_partials_beyond_the_scratch(rt):
    assert _abi.lib.ammon_attention_scratch_bytes(64, 128, 32768, 64) > SCRATCH
    q = rt.alloc(64 * 128 * 4)
    kv = rt.alloc(8)
    step = rt.step(0, 0)
    with pytest.raises(AmmonError, match="above the 4194304-byte library scratch"):
        call("ammon_attention_decode_noalloc", rt.handle, None, q, 64, kv, kv, BF16, 8, 128,
             32768, step, 64, q)
