"""GPU tests of ammon_attention_decode_noalloc, the attention decode pair with
the split partials in the library's own per-GPU scratch (no counterpart in
the reference: it serves callers that cannot allocate device memory).

Its output must equal ammon_attention_decode's with a caller buffer bit for
bit -- same kernels, same split -- on two calls in a row, the second with a
smaller input (the scratch keeps the first call's contents), and it must
reject shapes whose partials exceed the scratch.  Collected last (the file
name sorts last) so a failure here cannot hide other tests under -x.
"""
import numpy as np
import pytest

import oracle
from ammon_amd import AmmonError, _abi
from ammon_amd._abi import BF16, F32, call

pytestmark = pytest.mark.gpu

SCRATCH = 4 << 20


def head_major(pm, kv_heads, seq, head):
    return np.ascontiguousarray(pm.reshape(seq, kv_heads, head).transpose(1, 0, 2))


def attend(rt, case, noalloc):
    q_heads, kv_heads, head, seq, pos, split, kv_dtype, seed = case
    qh = oracle.normal(q_heads * head, seed).reshape(q_heads, head)
    kh = oracle.storage(oracle.normal(seq * kv_heads * head, seed + 1), kv_dtype)
    vh = oracle.storage(oracle.normal(seq * kv_heads * head, seed + 2), kv_dtype)
    q = rt.upload(qh)
    kc = rt.upload(head_major(kh, kv_heads, seq, head))
    vc = rt.upload(head_major(vh, kv_heads, seq, head))
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
# smaller one (fewer heads, shorter cache, another position and split)
CASES = [
    (32, 8, 128, 8192, 8191, 128, BF16, 71),
    (8, 2, 64, 1024, 700, 32, F32, 81),
]


def test_noalloc_matches_caller_buffer_on_two_calls(rt):
    for case in CASES:
        print(f"noalloc case {case}", flush=True)
        got, want = attend(rt, case, noalloc=True)
        ref, _ = attend(rt, case, noalloc=False)
        np.testing.assert_array_equal(got, ref)
        err = float(np.max(np.abs(got - want)) / np.max(np.abs(want)))
        assert err <= 1e-5, (case, err)


def test_noalloc_rejects_partials_beyond_the_scratch(rt):
    assert _abi.lib.ammon_attention_scratch_bytes(64, 128, 32768, 64) > SCRATCH
    q = rt.alloc(64 * 128 * 4)
    kv = rt.alloc(8)
    step = rt.step(0, 0)
    with pytest.raises(AmmonError, match="above the 4194304-byte library scratch"):
        call("ammon_attention_decode_noalloc", rt.handle, None, q, 64, kv, kv, BF16, 8, 128,
             32768, step, 64, q)
