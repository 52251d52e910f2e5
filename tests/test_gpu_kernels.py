"""GPU parity tests of the gfx950 kernels through the C ABI.

Each kernel is compared with the CPU oracle on identical seeded inputs:
bit-exact for gathers, cache stores, adds and argmax; relative error
<= 1e-5 (normwise: max |err| / max |ref|) for fp32 norm / attention / SwiGLU
/ GEMV.  The reference's own known-answer tests (tests/kernels.rs) are
restated first in each group.
"""
import ctypes

import numpy as np
import pytest

import oracle
from ammon_amd import _abi
from ammon_amd._abi import BF16, F32, AmmonError, call

pytestmark = pytest.mark.gpu

P = ctypes.c_void_p
RTOL = 1e-5


def rel_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


def up(rt, a):
    return rt.upload(np.ascontiguousarray(a))


def down(buf, shape, dtype=np.float32):
    return buf.download(shape, dtype)


def npdt(dtype):
    return np.uint16 if dtype == BF16 else np.float32


# ---- embed ------------------------------------------------------------------------
def test_embed_gathers_selected_row(rt):
    # tests/kernels.rs:36-52
    table = up(rt, np.array([[1.0, 2.0], [3.0, 4.0]], np.float32))
    x = up(rt, np.zeros(2, np.float32))
    step = rt.step(1, 0)
    call("ammon_embed", rt.handle, None, table, F32, 2, 2, step, x)
    np.testing.assert_array_equal(down(x, 2), [3.0, 4.0])


def test_deposit_feeds_embed_without_relaunch_changes(rt):
    # tests/kernels.rs:184-222: the same launch, a new deposit per token.
    table = up(rt, np.array([[10.0, 20.0], [30.0, 40.0]], np.float32))
    x = up(rt, np.zeros(2, np.float32))
    step = rt.step(0, 0)
    for token, want in ((0, [10.0, 20.0]), (1, [30.0, 40.0])):
        rt.deposit(step, token, 0)
        call("ammon_embed", rt.handle, None, table, F32, 2, 2, step, x)
        np.testing.assert_array_equal(down(x, 2), want)


@pytest.mark.parametrize("dtype", [BF16, F32])
def test_embed_rows_c2_bit_exact(rt, dtype):
    vocab, dim, rows = 128256, 4096, 4096
    table = oracle.storage(oracle.normal(vocab * dim, 101), dtype).reshape(vocab, dim)
    ids = np.random.default_rng(5).integers(0, vocab, rows).astype(np.uint32)
    t = up(rt, table)
    i = up(rt, ids)
    x = rt.alloc(rows * dim * 4)
    call("ammon_embed_rows", rt.handle, None, t, dtype, vocab, dim, i, rows, x)
    np.testing.assert_array_equal(down(x, (rows, dim)), oracle.embed(table, dtype, ids))
    # the single-token form from a device DecodeStep
    step = rt.step(int(ids[7]), 0)
    call("ammon_embed", rt.handle, None, t, dtype, vocab, dim, step, x)
    np.testing.assert_array_equal(down(x, dim), oracle.embed(table, dtype, ids[7:8])[0])


def test_embed_out_of_range_token_gives_nan_row(rt):
    table = up(rt, np.ones((4, 8), np.float32))
    x = up(rt, np.zeros(8, np.float32))
    step = rt.step(4, 0)
    call("ammon_embed", rt.handle, None, table, F32, 4, 8, step, x)
    assert np.all(np.isnan(down(x, 8)))


def test_embed_validation(rt):
    table = up(rt, np.ones((2, 2), np.float32))
    with pytest.raises(AmmonError, match="step"):
        call("ammon_embed", rt.handle, None, table, F32, 2, 2, None, table)
    with pytest.raises(AmmonError, match="dtype"):
        call("ammon_embed", rt.handle, None, table, 7, 2, 2, rt.step(0, 0), table)


# ---- rmsnorm ------------------------------------------------------------------------
def test_rmsnorm_matches_llama3_formula(rt):
    # tests/kernels.rs:163-182
    x = up(rt, np.ones(4, np.float32))
    w = up(rt, np.ones(4, np.float32))
    o = up(rt, np.zeros(4, np.float32))
    call("ammon_rmsnorm", rt.handle, None, x, w, F32, o, 1, 4, 1e-5)
    scale = 1.0 / np.sqrt(np.float32(1.0) + np.float32(1e-5))
    assert np.all(np.abs(down(o, 4) - scale) < 1e-5)


@pytest.mark.parametrize("rows", [1, 2, 7, 16, 64])
@pytest.mark.parametrize("w_dtype", [F32, BF16])
def test_rmsnorm_c2(rt, rows, w_dtype):
    dim = 4096
    xh = oracle.normal(rows * dim, 200 + rows).reshape(rows, dim)
    wh = oracle.storage(oracle.normal(dim, 300), w_dtype)
    x, w, o = up(rt, xh), up(rt, wh), rt.alloc(xh.nbytes)
    call("ammon_rmsnorm", rt.handle, None, x, w, w_dtype, o, rows, dim, 1e-5)
    want = oracle.rmsnorm(xh, wh, w_dtype)
    assert rel_err(down(o, (rows, dim)), want) <= RTOL
    # in place (rmsnorm_inplace, reference src/kernels.rs:103-128)
    call("ammon_rmsnorm", rt.handle, None, x, w, w_dtype, x, rows, dim, 1e-5)
    assert rel_err(down(x, (rows, dim)), want) <= RTOL


@pytest.mark.parametrize("dim", [288, 300, 3, 8192])
def test_rmsnorm_odd_widths(rt, dim):
    xh = oracle.normal(dim, 7)
    wh = oracle.normal(dim, 8)
    x, w, o = up(rt, xh), up(rt, wh), rt.alloc(xh.nbytes)
    call("ammon_rmsnorm", rt.handle, None, x, w, F32, o, 1, dim, 1e-5)
    assert rel_err(down(o, dim), oracle.rmsnorm(xh, wh)) <= RTOL


# ---- RoPE + cache stores -------------------------------------------------------------
def head_major(pos_major, kv_heads, seq, head):
    from ammon_amd import kv_permute
    return kv_permute(pos_major, kv_heads, seq, head)


def pos_major(head_major_arr, kv_heads, seq, head):
    from ammon_amd import kv_unpermute
    return kv_unpermute(head_major_arr, kv_heads, seq, head)


def test_rope_store_writes_rotated_k_from_scratch(rt):
    # tests/kernels.rs:239-283: head 2, one query head, pos 1, theta 10000.
    table = up(rt, oracle.rope_table(10000.0, 2, 2))
    q = up(rt, np.array([1.0, 2.0], np.float32))
    kp = up(rt, np.array([3.0, 4.0], np.float32))
    k = up(rt, np.zeros((1, 2, 2), np.float32))  # [kv_heads=1, seq=2, head=2]
    step = rt.step(0, 1)
    call("ammon_rope_store", rt.handle, None, q, 1, kp, 1, 2, k, F32, 2, step, table)
    c, s = np.cos(1.0), np.sin(1.0)
    qo = down(q, 2)
    ko = down(k, 4)
    assert np.allclose(qo, [1 * c - 2 * s, 1 * s + 2 * c], atol=1e-5)
    np.testing.assert_array_equal(ko[:2], [0.0, 0.0])
    assert np.allclose(ko[2:], [3 * c - 4 * s, 3 * s + 4 * c], atol=1e-5)


def test_rope_at_pos_zero_is_identity(rt):
    # tests/kernels.rs:54-81 (in-place rope on q and the K row)
    table = up(rt, oracle.rope_table(10000.0, 2, 1))
    q = up(rt, np.array([1.0, 2.0, 3.0, 4.0], np.float32))
    k = up(rt, np.array([5.0, 6.0, 7.0, 8.0], np.float32))  # [2 kv heads, 1 pos, 2]
    step = rt.step(0, 0)
    call("ammon_rope", rt.handle, None, q, 2, 2, 2, k, F32, 1, step, table)
    np.testing.assert_array_equal(down(q, 4), [1.0, 2.0, 3.0, 4.0])
    np.testing.assert_array_equal(down(k, 4), [5.0, 6.0, 7.0, 8.0])


@pytest.mark.parametrize("kv_dtype", [F32, BF16])
def test_rope_store_c2_bit_exact(rt, kv_dtype):
    theta, q_heads, kv_heads, head, seq = 500000.0, 32, 8, 128, 8192
    table_h = oracle.rope_table(theta, head, seq)
    table = up(rt, table_h)
    positions = np.random.default_rng(3).integers(0, seq, 64)
    kc_h = np.zeros((seq, kv_heads, head), npdt(kv_dtype))
    kc = up(rt, head_major(kc_h, kv_heads, seq, head))
    q = rt.alloc(q_heads * head * 4)
    kp = rt.alloc(kv_heads * head * 4)
    step = rt.step(0, 0)
    for i, pos in enumerate(positions):
        qh = oracle.normal(q_heads * head, 1000 + i)
        kh = oracle.normal(kv_heads * head, 2000 + i)
        q.upload(qh)
        kp.upload(kh)
        rt.deposit(step, 0, int(pos))
        call("ammon_rope_store", rt.handle, None, q, q_heads, kp, kv_heads, head, kc, kv_dtype,
             seq, step, table)
        oracle.rope_store(qh, kh, kc_h, kv_dtype, head, int(pos), table_h)
        np.testing.assert_array_equal(down(q, q_heads * head), qh)
    got = pos_major(down(kc, (kv_heads, seq, head), npdt(kv_dtype)), kv_heads, seq, head)
    np.testing.assert_array_equal(got, kc_h)


@pytest.mark.parametrize("kv_dtype", [F32, BF16])
def test_cache_store_bit_exact(rt, kv_dtype):
    # tests/kernels.rs:285-307 first, then random rows at random positions
    src = up(rt, np.array([9.0, 8.0], np.float32))
    dst = up(rt, np.zeros(6, npdt(kv_dtype)))
    call("ammon_cache_store", rt.handle, None, src, 1, 2, dst, kv_dtype, 3, rt.step(0, 2))
    np.testing.assert_array_equal(oracle.widen(down(dst, 6, npdt(kv_dtype)), kv_dtype),
                                  [0, 0, 0, 0, 9, 8])
    kv_heads, head, seq = 8, 128, 512
    ref = np.zeros((seq, kv_heads, head), npdt(kv_dtype))
    cache = up(rt, head_major(ref, kv_heads, seq, head))
    v = rt.alloc(kv_heads * head * 4)
    step = rt.step(0, 0)
    for i, pos in enumerate((0, 1, 17, 511, 300)):
        vh = oracle.normal(kv_heads * head, 50 + i)
        v.upload(vh)
        rt.deposit(step, 0, pos)
        call("ammon_cache_store", rt.handle, None, v, kv_heads, head, cache, kv_dtype, seq, step)
        oracle.cache_store(vh, ref, kv_dtype, pos)
    got = pos_major(down(cache, (kv_heads, seq, head), npdt(kv_dtype)), kv_heads, seq, head)
    np.testing.assert_array_equal(got, ref)


def test_rope_rejects_bad_shapes(rt):
    table = up(rt, oracle.rope_table(10000.0, 2, 1))
    q = up(rt, np.zeros(4, np.float32))
    with pytest.raises(AmmonError, match="no wider than q"):
        call("ammon_rope_store", rt.handle, None, q, 1, q, 2, 2, q, F32, 1, rt.step(0, 0), table)
    with pytest.raises(AmmonError, match="even"):
        call("ammon_rope_store", rt.handle, None, q, 1, q, 1, 3, q, F32, 1, rt.step(0, 0), table)


# ---- attention -------------------------------------------------------------------------
def cpu_attention_f64(q, key, value, q_heads, kv_heads, head, pos):
    """The reference's f64 attention (tests/kernels.rs:400-427), pos-major cache."""
    kv_mul = q_heads // kv_heads
    q = q.reshape(q_heads, head).astype(np.float64)
    out = np.zeros((q_heads, head))
    for h in range(q_heads):
        g = h // kv_mul
        s = key[: pos + 1, g, :].astype(np.float64) @ q[h] / np.sqrt(head)
        w = np.exp(s - s.max())
        out[h] = (w[:, None] * value[: pos + 1, g, :].astype(np.float64)).sum(0) / w.sum()
    return out


REF_CASES = [
    (6, 6, 48, 256, [0, 1, 7, 8, 9, 31, 32, 33, 100, 255]),
    (4, 2, 64, 80, [0, 47, 79]),
    (2, 1, 128, 40, [39]),
    (3, 3, 20, 33, [5, 32]),
    (1, 1, 32, 2112, [2047, 2111]),
]


def run_attention(rt, qh, kc_pm, vc_pm, kv_dtype, q_heads, kv_heads, head, seq, pos, split,
                  poison=True):
    q = up(rt, qh)
    kc = up(rt, head_major(kc_pm, kv_heads, seq, head))
    vc = up(rt, head_major(vc_pm, kv_heads, seq, head))
    splits = _abi.lib.ammon_attention_splits(seq, split)
    part_h = np.full((q_heads, splits, head + 2), np.nan if poison else 0.0, np.float32)
    part = up(rt, part_h)
    out = rt.alloc(q_heads * head * 4)
    step = rt.step(0, pos)
    call("ammon_attention_decode", rt.handle, None, q, q_heads, kc, vc, kv_dtype, kv_heads, head,
         seq, step, split, part, part_h.nbytes, out)
    return down(out, (q_heads, head)), down(part, part_h.shape)


@pytest.mark.parametrize("q_heads,kv_heads,head,seq,positions", REF_CASES)
@pytest.mark.parametrize("split", [8, 16, 64])
def test_split_attention_matches_reference(rt, q_heads, kv_heads, head, seq, positions, split):
    # tests/kernels.rs:429-538 with the reference's seeds and tolerance, plus
    # the oracle's split-8 restatement at 1e-5 relative.
    qh = oracle.pseudo_random(q_heads * head, 11).reshape(q_heads, head)
    kh = oracle.pseudo_random(seq * kv_heads * head, 12).reshape(seq, kv_heads, head)
    vh = oracle.pseudo_random(seq * kv_heads * head, 13).reshape(seq, kv_heads, head)
    for pos in positions:
        got, part = run_attention(rt, qh, kh, vh, F32, q_heads, kv_heads, head, seq, pos, split)
        want = cpu_attention_f64(qh, kh, vh, q_heads, kv_heads, head, pos)
        assert np.max(np.abs(got - want)) < 1e-4, (pos, split)
        assert rel_err(got, oracle.attention(qh, kh, vh, F32, pos)) <= RTOL, (pos, split)
        if part.shape[1] == 1:
            continue  # one split: pass 1 writes the output, no partial
        live = pos // split + 1
        assert np.all(np.isfinite(part[:, :live])), pos
        assert np.all(np.isnan(part[:, live:])), "a dead split was written"


@pytest.mark.parametrize("kv_dtype,q_heads,kv_heads,head", [
    (F32, 6, 6, 48), (F32, 8, 2, 64), (BF16, 32, 8, 128), (BF16, 8, 8, 128), (BF16, 16, 8, 128),
    (BF16, 32, 4, 128), (F32, 32, 8, 128)])
def test_single_split_decode_matches_two_launches(rt, kv_dtype, q_heads, kv_heads, head):
    # A split covering the whole cache: ammon_attention_decode runs pass 1
    # alone, which writes acc / l -- the merge of one split -- so the output
    # equals the explicit partial + combine pair bit for bit, and a position
    # past the cache gives the combine's NaN row.
    seq = 256
    qh = oracle.normal(q_heads * head, 151).reshape(q_heads, head)
    kh = oracle.storage(oracle.normal(seq * kv_heads * head, 152), kv_dtype).reshape(
        seq, kv_heads, head)
    vh = oracle.storage(oracle.normal(seq * kv_heads * head, 153), kv_dtype).reshape(
        seq, kv_heads, head)
    q = up(rt, qh)
    kc, vc = up(rt, head_major(kh, kv_heads, seq, head)), up(rt, head_major(vh, kv_heads, seq, head))
    part = rt.alloc(q_heads * (head + 2) * 4)
    one, two = rt.alloc(q_heads * head * 4), rt.alloc(q_heads * head * 4)
    step = rt.step(0, 0)
    for pos in (0, 1, 63, 64, 200, 255, 256):
        rt.deposit(step, 0, pos)
        call("ammon_attention_decode", rt.handle, None, q, q_heads, kc, vc, kv_dtype, kv_heads,
             head, seq, step, seq, part, q_heads * (head + 2) * 4, one)
        call("ammon_attention_partial", rt.handle, None, q, q_heads, kc, vc, kv_dtype, kv_heads,
             head, seq, step, seq, part)
        call("ammon_attention_combine", rt.handle, None, part, q_heads, head, seq, step, seq, two)
        got, want = down(one, (q_heads, head)), down(two, (q_heads, head))
        if pos >= seq:
            assert np.all(np.isnan(got)) and np.all(np.isnan(want))
            continue
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=str(pos))
        assert rel_err(got, oracle.attention(qh, kh, vh, kv_dtype, pos)) <= RTOL, pos


@pytest.mark.parametrize("q_heads,kv_heads", [(8, 8), (16, 8), (32, 8), (32, 4)])
@pytest.mark.parametrize("split", [64, 128, 192])
def test_staged_attention_every_group_size(rt, q_heads, kv_heads, split):
    # The matrix-core unit (bf16 cache, head 128) at 1, 2, 4 and 8 q heads per
    # kv head over several splits: one chunk per unit, two (both requested
    # at the start) and three (the two-buffer ring refilled); positions that
    # end mid-chunk and on a chunk boundary; dead splits must stay poisoned.
    head, seq = 128, 1024
    qh = oracle.normal(q_heads * head, 171).reshape(q_heads, head)
    kh = oracle.storage(oracle.normal(seq * kv_heads * head, 172), BF16).reshape(
        seq, kv_heads, head)
    vh = oracle.storage(oracle.normal(seq * kv_heads * head, 173), BF16).reshape(
        seq, kv_heads, head)
    for pos in (1023, 700, 191, 64, 5):
        got, part = run_attention(rt, qh, kh, vh, BF16, q_heads, kv_heads, head, seq, pos, split)
        assert rel_err(got, oracle.attention(qh, kh, vh, BF16, pos)) <= RTOL, (pos, split)
        live = pos // split + 1
        assert np.all(np.isfinite(part[:, :live])), (pos, split)
        assert np.all(np.isnan(part[:, live:])), (pos, split)


def test_combine_warm_matches_combine(rt):
    # ammon_attention_combine_warm merges exactly as ammon_attention_combine
    # (bit for bit) whether it warms the next GEMV's rows (the Llama-3-8B wo,
    # 4096 x 4096 bf16: one row block per workgroup), warms whole rows, or
    # skips warming (a position below the threshold, a matrix whose blocks
    # do not line up with the merge grid, one whose last block is ragged, no
    # matrix); a bad next matrix is a validation error.
    q_heads, kv_heads, head, seq, split = 32, 8, 128, 2048, 128
    qh = oracle.normal(q_heads * head, 181).reshape(q_heads, head)
    kh = oracle.storage(oracle.normal(seq * kv_heads * head, 182), BF16).reshape(
        seq, kv_heads, head)
    vh = oracle.storage(oracle.normal(seq * kv_heads * head, 183), BF16).reshape(
        seq, kv_heads, head)
    q = up(rt, qh)
    kc, vc = up(rt, head_major(kh, kv_heads, seq, head)), up(rt, head_major(vh, kv_heads, seq, head))
    splits = -(-seq // split)
    part = rt.alloc(q_heads * splits * (head + 2) * 4)
    plain, warm = rt.alloc(q_heads * head * 4), rt.alloc(q_heads * head * 4)
    dim = q_heads * head
    wo = rt.alloc(dim * dim * 2)
    rt.fill_normal(wo, BF16, dim * dim, 184, 0, 0.0, 0.02)
    step = rt.step(0, 0)
    for pos in (2047, 1000, 130):
        rt.deposit(step, 0, pos)
        call("ammon_attention_partial", rt.handle, None, q, q_heads, kc, vc, BF16, kv_heads,
             head, seq, step, split, part)
        call("ammon_attention_combine", rt.handle, None, part, q_heads, head, seq, step, split,
             plain)
        want = down(plain, (q_heads, head))
        assert rel_err(want, oracle.attention(qh, kh, vh, BF16, pos)) <= RTOL, pos
        for nxt, rows, n, row_bytes in ((wo, dim, dim, 0), (wo, dim, dim, 2 * dim),
                                        (wo, 100, dim, 0), (wo, dim - 4, dim, 0),
                                        (None, 0, 0, 0)):
            rt.fill(warm, F32, q_heads * head, float("nan"))
            call("ammon_attention_combine_warm", rt.handle, None, part, q_heads, head, seq, step,
                 split, warm, nxt, BF16, rows, n, row_bytes, 1024)
            got = down(warm, (q_heads, head))
            np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32),
                                          err_msg=f"pos {pos} rows {rows} bytes {row_bytes}")
    with pytest.raises(AmmonError):
        call("ammon_attention_combine_warm", rt.handle, None, part, q_heads, head, seq, step,
             split, warm, wo, 7, dim, dim, 0, 0)
    with pytest.raises(AmmonError):
        call("ammon_attention_combine_warm", rt.handle, None, part, q_heads, head, seq, step,
             split, warm, wo, BF16, 0, dim, 0, 0)
    rt.synchronize()
    wo.free()


def test_attention_partials_match_oracle_split8(rt):
    q_heads, kv_heads, head, seq, pos = 6, 6, 48, 256, 100
    qh = oracle.pseudo_random(q_heads * head, 11).reshape(q_heads, head)
    kh = oracle.pseudo_random(seq * kv_heads * head, 12).reshape(seq, kv_heads, head)
    vh = oracle.pseudo_random(seq * kv_heads * head, 13).reshape(seq, kv_heads, head)
    _, part = run_attention(rt, qh, kh, vh, F32, q_heads, kv_heads, head, seq, pos, 8)
    want = oracle.attention_partial(qh, kh, vh, F32, pos)
    live = pos // 8 + 1
    np.testing.assert_allclose(part[:, :live], want[:, :live], rtol=2e-6, atol=1e-6)


def test_default_split_sizes_units_to_kernel_occupancy(rt):
    """The model's split: two pass-1 units per CU where two of the shape's
    workgroups fit on a CU, one where only one does (the generic bf16
    kernel of an 8:1 group runs one workgroup per CU: one round of longer
    splits; the head-128 kernels fit two)."""
    lib = _abi.lib
    cus = rt.info.compute_units
    units = lambda kv_heads, seq, split: kv_heads * int(lib.ammon_attention_splits(seq, split))
    # 4:1 and 8:1 at head 128, two per CU: the kv-head-count choice
    for q_heads, seq in ((32, 8192), (64, 32768)):
        s = lib.ammon_attention_default_split_for(rt.handle, q_heads, 8, 128, BF16, seq)
        assert s == lib.ammon_attention_default_split(rt.handle, 8, seq)
        assert units(8, seq, s) <= 2 * cus < units(8, seq, s // 2)
    # 8:1 at head 64 (the generic kernel), one per CU: at most one unit per CU
    s = lib.ammon_attention_default_split_for(rt.handle, 64, 8, 64, BF16, 32768)
    assert units(8, 32768, s) <= cus < units(8, 32768, s // 2)
    # the matrix-core kernels score 64-position chunks: no split below 64,
    # where the VALU kernels (fp32 cache) keep the unit-count choice
    for seq in (1024, 2048):
        assert lib.ammon_attention_default_split_for(rt.handle, 32, 8, 128, BF16, seq) == 64
        assert (lib.ammon_attention_default_split_for(rt.handle, 32, 8, 128, F32, seq)
                == lib.ammon_attention_default_split(rt.handle, 8, seq))
    # a cache of at most 256 positions: one split, whatever the shape
    assert lib.ammon_attention_default_split_for(rt.handle, 64, 8, 128, BF16, 256) == 256


@pytest.mark.parametrize("ctx", [1024, 4096, 8192])
@pytest.mark.parametrize("kv_dtype", [BF16, F32])
@pytest.mark.parametrize("cache", ["seq8192", "seq_ctx"])
def test_attention_c3(rt, ctx, kv_dtype, cache):
    """Single-layer decode attention at the Llama-3-8B head shape, position
    ctx - 1.  "seq8192": a cache sized 8192 at the kv-head-count split;
    "seq_ctx": a cache of exactly ctx positions at the split the library
    picks for the shape (ammon_attention_default_split_for: 64 at 1024 and
    4096 positions for the bf16 matrix-core kernel, one 64-position chunk
    per unit), as the decode attention of a ctx-sized cache runs it.  The
    other positions of each split are checked too: the split's first,
    a ragged last split, and a split boundary."""
    q_heads, kv_heads, head = 32, 8, 128
    seq = 8192 if cache == "seq8192" else ctx
    qh = oracle.normal(q_heads * head, 31).reshape(q_heads, head)
    kh = oracle.storage(oracle.normal(seq * kv_heads * head, 32), kv_dtype).reshape(
        seq, kv_heads, head)
    vh = oracle.storage(oracle.normal(seq * kv_heads * head, 33), kv_dtype).reshape(
        seq, kv_heads, head)
    if cache == "seq8192":
        split = int(_abi.lib.ammon_attention_default_split(rt.handle, kv_heads, seq))
        positions = [ctx - 1]
    else:
        split = int(_abi.lib.ammon_attention_default_split_for(rt.handle, q_heads, kv_heads, head,
                                                                kv_dtype, seq))
        if kv_dtype == BF16 and ctx <= 4096:
            assert split == 64, split
        # the last position, a ragged last split, a split's first position
        positions = [ctx - 1, ctx - 1 - split // 2, ctx - split]
    for pos in positions:
        got, part = run_attention(rt, qh, kh, vh, kv_dtype, q_heads, kv_heads, head, seq, pos,
                                  split)
        want = oracle.attention(qh, kh, vh, kv_dtype, pos)
        assert rel_err(got, want) <= RTOL, (pos, split)
        f64 = cpu_attention_f64(qh, oracle.widen(kh, kv_dtype), oracle.widen(vh, kv_dtype),
                                q_heads, kv_heads, head, pos)
        assert rel_err(got, f64) <= RTOL, (pos, split)
        if part.shape[1] > 1:
            live = pos // split + 1
            assert np.all(np.isfinite(part[:, :live])), (pos, split)
            assert np.all(np.isnan(part[:, live:])), "a dead split was written"


def test_attention_gqa8_c5_shape(rt):
    q_heads, kv_heads, head, seq, pos = 64, 8, 128, 4096, 4095
    qh = oracle.normal(q_heads * head, 41).reshape(q_heads, head)
    kh = oracle.to_bf16(oracle.normal(seq * kv_heads * head, 42)).reshape(seq, kv_heads, head)
    vh = oracle.to_bf16(oracle.normal(seq * kv_heads * head, 43)).reshape(seq, kv_heads, head)
    got, _ = run_attention(rt, qh, kh, vh, BF16, q_heads, kv_heads, head, seq, pos, 64)
    assert rel_err(got, oracle.attention(qh, kh, vh, BF16, pos)) <= RTOL


def test_attention_validation(rt):
    q = up(rt, np.zeros(4, np.float32))
    step = rt.step(0, 0)
    with pytest.raises(AmmonError, match="exceeds 128"):
        call("ammon_attention_partial", rt.handle, None, q, 1, q, q, F32, 1, 130, 4, step, 8, q)
    with pytest.raises(AmmonError, match="multiple of kv_heads"):
        call("ammon_attention_partial", rt.handle, None, q, 3, q, q, F32, 2, 4, 4, step, 8, q)
    with pytest.raises(AmmonError, match="partial scratch must be"):
        call("ammon_attention_decode", rt.handle, None, q, 1, q, q, F32, 1, 4, 64, step, 8, q,
             16, q)


# ---- SwiGLU / add ----------------------------------------------------------------------------
def test_swiglu_of_zero_is_zero(rt):
    # tests/kernels.rs:148-161
    hb = up(rt, np.zeros(2, np.float32))
    hb2 = up(rt, np.array([5.0, 7.0], np.float32))
    call("ammon_swiglu", rt.handle, None, hb, hb2, 2)
    np.testing.assert_array_equal(down(hb, 2), [0.0, 0.0])


def test_swiglu_c2(rt):
    n = 14336
    gh, uh = oracle.normal(n, 61) * 3, oracle.normal(n, 62)
    g, u = up(rt, gh), up(rt, uh)
    call("ammon_swiglu", rt.handle, None, g, u, n)
    got = down(g, n)
    want = oracle.swiglu(gh, uh)
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)) <= RTOL


def test_tensor_add_into_is_elementwise(rt):
    # tests/kernels.rs:224-237
    a = up(rt, np.array([1.0, 2.0], np.float32))
    b = up(rt, np.array([3.0, 4.0], np.float32))
    o = rt.alloc(8)
    call("ammon_add", rt.handle, None, a, b, o, 2)
    np.testing.assert_array_equal(down(o, 2), [4.0, 6.0])
    ah, bh = oracle.normal(4099, 1), oracle.normal(4099, 2)
    a, b = up(rt, ah), up(rt, bh)
    call("ammon_add", rt.handle, None, a, b, a, 4099)
    np.testing.assert_array_equal(down(a, 4099), ah + bh)


# ---- GEMV family ---------------------------------------------------------------------------------
def test_matmul_identity(rt):
    # tests/kernels.rs:83-97 and :342-355
    w = up(rt, np.eye(2, dtype=np.float32))
    for xv in ([1.0, 2.0], [3.0, 4.0]):
        x = up(rt, np.array(xv, np.float32))
        y = rt.alloc(8)
        call("ammon_gemv", rt.handle, None, w, F32, 2, 2, x, y, None)
        np.testing.assert_array_equal(down(y, 2), xv)


# n > 4096 without a norm stages x by direct-to-LDS loads: whole and ragged
# tiles for 8-wide (bf16), 4-wide (fp32) and 1-wide chunks (bf16, n % 8 = 4)
GEMV_SHAPES = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336), (288, 288), (768, 288),
               (288, 768), (7, 5), (33, 300), (1, 1), (5, 4100), (17, 5000), (9, 8200),
               (3, 12292)]


@pytest.mark.parametrize("d,n", GEMV_SHAPES)
@pytest.mark.parametrize("w_dtype", [BF16, F32])
def test_gemv_matches_oracle(rt, d, n, w_dtype):
    wh = oracle.storage(oracle.normal(d * n, 71, std=0.02), w_dtype).reshape(d, n)
    xh = oracle.normal(n, 72)
    w, x, y = up(rt, wh), up(rt, xh), rt.alloc(d * 4)
    call("ammon_gemv", rt.handle, None, w, w_dtype, d, n, x, y, None)
    want = oracle.gemv(wh, w_dtype, xh)
    assert rel_err(down(y, d), want) <= RTOL
    # residual epilogue, in place on the residual (x += W h)
    rh = oracle.normal(d, 73)
    r = up(rt, rh)
    call("ammon_gemv", rt.handle, None, w, w_dtype, d, n, x, r, r)
    assert rel_err(down(r, d), rh + want) <= RTOL


# (65541, 2056): the 4-rows-per-wave kernel (>= 65536 rows of <= 8 KiB) with a
# ragged last row block and a partial last tile
@pytest.mark.parametrize("d,n", [(128256, 4096), (32000, 288), (4096, 4096), (65541, 2056)])
def test_gemv_rmsnorm_lm_head(rt, d, n):
    w_dtype = BF16 if n != 288 else F32
    wh = oracle.storage(oracle.normal(d * n, 81, std=0.02), w_dtype).reshape(d, n)
    xh = oracle.normal(n, 82) * 3
    gh = 1.0 + 0.1 * oracle.normal(n, 83)
    w, x, g, y = up(rt, wh), up(rt, xh), up(rt, gh), rt.alloc(d * 4)
    call("ammon_gemv_rmsnorm", rt.handle, None, x, g, F32, 1e-5, w, w_dtype, d, n, y)
    want = oracle.gemv(wh, w_dtype, oracle.rmsnorm(xh, gh).reshape(-1))
    assert rel_err(down(y, d), want) <= RTOL


@pytest.mark.parametrize("n,g_dtype", [(8192, F32), (8192, BF16), (14336, F32), (8190, F32)])
def test_gemv_rmsnorm_prologue_matches_separate_norm(rt, n, g_dtype):
    # Rows longer than the register-staged prologue covers (dim 8192 and up;
    # 8190 takes the scalar staging): the fused norm normalises x exactly as
    # ammon_rmsnorm does, so the GEMV outputs are bit-identical.
    d = 1024
    wh = oracle.storage(oracle.normal(d * n, 91, std=0.02), BF16).reshape(d, n)
    xh = oracle.normal(n, 92) * 3
    gh = oracle.storage(1.0 + 0.1 * oracle.normal(n, 93), g_dtype)
    w, x, g = up(rt, wh), up(rt, xh), up(rt, gh)
    y1, y2, xn = rt.alloc(d * 4), rt.alloc(d * 4), rt.alloc(n * 4)
    call("ammon_gemv_rmsnorm", rt.handle, None, x, g, g_dtype, 1e-5, w, BF16, d, n, y1)
    call("ammon_rmsnorm", rt.handle, None, x, g, g_dtype, xn, 1, n, 1e-5)
    call("ammon_gemv", rt.handle, None, w, BF16, d, n, xn, y2, None)
    got, sep = down(y1, d), down(y2, d)
    np.testing.assert_array_equal(got.view(np.uint32), sep.view(np.uint32))
    want = oracle.gemv(wh, BF16, oracle.rmsnorm(xh, gh, g_dtype).reshape(-1))
    assert rel_err(got, want) <= RTOL


@pytest.mark.parametrize("n", [4096, 8192])
def test_gemv_rmsnorm_unaligned_bf16_norm_weight(rt, n):
    # A bf16 norm weight 2 bytes into its buffer takes the element-wise
    # pass instead of 8-byte loads; the output is the same bit for bit.
    d = 512
    wh = oracle.storage(oracle.normal(d * n, 95, std=0.02), BF16).reshape(d, n)
    xh = oracle.normal(n, 96) * 3
    gh = oracle.storage(1.0 + 0.1 * oracle.normal(n, 97), BF16)
    w, x = up(rt, wh), up(rt, xh)
    g = up(rt, gh)
    g_off = up(rt, np.concatenate([np.zeros(1, np.uint16), gh]))
    y1, y2 = rt.alloc(d * 4), rt.alloc(d * 4)
    call("ammon_gemv_rmsnorm", rt.handle, None, x, g, BF16, 1e-5, w, BF16, d, n, y1)
    call("ammon_gemv_rmsnorm", rt.handle, None, x, g_off.offset(2), BF16, 1e-5, w, BF16, d, n, y2)
    np.testing.assert_array_equal(down(y2, d).view(np.uint32), down(y1, d).view(np.uint32))


def test_gemv_validation(rt):
    x = up(rt, np.zeros(8, np.float32))
    with pytest.raises(AmmonError, match="y overlaps x"):
        call("ammon_gemv", rt.handle, None, x, F32, 2, 2, x, x, None)
    with pytest.raises(AmmonError, match="LDS"):
        call("ammon_gemv", rt.handle, None, x, F32, 1, 1 << 20, x, P(int(x) + 8 * 4 * 4), None)


def fused_qkv_reference(xh, gh, wq, wk, wv, w_dtype, q_heads, kv_heads, head, seq, pos, table,
                        kv_dtype, kc_pm, vc_pm):
    xn = oracle.rmsnorm(xh, gh).reshape(-1)
    q = oracle.gemv(wq, w_dtype, xn)
    kp = oracle.gemv(wk, w_dtype, xn)
    v = oracle.gemv(wv, w_dtype, xn)
    oracle.rope_store(q, kp, kc_pm, kv_dtype, head, pos, table)
    oracle.cache_store(v, vc_pm, kv_dtype, pos)
    return q


@pytest.mark.parametrize("shape", ["c1", "c4"])
@pytest.mark.parametrize("kv_dtype", [F32, BF16])
def test_qkv_rope_store_fused(rt, shape, kv_dtype):
    if shape == "c1":
        dim, q_heads, kv_heads, head, seq, w_dtype, theta = 288, 6, 6, 48, 256, F32, 10000.0
    else:
        dim, q_heads, kv_heads, head, seq, w_dtype, theta = 4096, 32, 8, 128, 512, BF16, 500000.0
    qd, kd = q_heads * head, kv_heads * head
    wq = oracle.storage(oracle.normal(qd * dim, 91, std=0.02), w_dtype).reshape(qd, dim)
    wk = oracle.storage(oracle.normal(kd * dim, 92, std=0.02), w_dtype).reshape(kd, dim)
    wv = oracle.storage(oracle.normal(kd * dim, 93, std=0.02), w_dtype).reshape(kd, dim)
    gh = 1.0 + 0.1 * oracle.normal(dim, 94)
    table_h = oracle.rope_table(theta, head, seq)
    kc_pm = np.zeros((seq, kv_heads, head), npdt(kv_dtype))
    vc_pm = np.zeros_like(kc_pm)
    dq, dk, dv, dg = up(rt, wq), up(rt, wk), up(rt, wv), up(rt, gh)
    kc, vc = up(rt, head_major(kc_pm, kv_heads, seq, head)), up(rt, head_major(vc_pm, kv_heads,
                                                                              seq, head))
    table = up(rt, table_h)
    x, q = rt.alloc(dim * 4), rt.alloc(qd * 4)
    kproj, vproj, xn = rt.alloc(kd * 4), rt.alloc(kd * 4), rt.alloc(dim * 4)
    step = rt.step(0, 0)
    for i, pos in enumerate((0, 1, seq - 1, 37)):
        xh = oracle.normal(dim, 95 + i)
        x.upload(xh)
        rt.deposit(step, 0, pos)
        call("ammon_qkv_rope_store", rt.handle, None, x, dg, F32, 1e-5, dq, dk, dv, w_dtype, dim,
             q_heads, kv_heads, head, q, kc, vc, kv_dtype, seq, step, table)
        want_q = fused_qkv_reference(xh, gh, wq, wk, wv, w_dtype, q_heads, kv_heads, head, seq,
                                     pos, table_h, kv_dtype, kc_pm, vc_pm)
        assert rel_err(down(q, qd), want_q) <= RTOL
        # Bit-exactness of the K/V stores given identical pre-store vectors:
        # the unfused GPU GEMVs (same per-row reduction) give the projections,
        # the oracle rotates/stores them, and the fused kernel's cache rows
        # must equal that bit for bit.
        call("ammon_gemv_rmsnorm", rt.handle, None, x, dg, F32, 1e-5, dk, w_dtype, kd, dim,
             kproj)
        call("ammon_gemv_rmsnorm", rt.handle, None, x, dg, F32, 1e-5, dv, w_dtype, kd, dim,
             vproj)
        kr = np.zeros((seq, kv_heads, head), npdt(kv_dtype))
        vr = np.zeros_like(kr)
        qscratch = np.zeros(qd, np.float32)
        oracle.rope_store(qscratch, down(kproj, kd), kr, kv_dtype, head, pos, table_h)
        oracle.cache_store(down(vproj, kd), vr, kv_dtype, pos)
        got_k = pos_major(down(kc, (kv_heads, seq, head), npdt(kv_dtype)), kv_heads, seq, head)
        got_v = pos_major(down(vc, (kv_heads, seq, head), npdt(kv_dtype)), kv_heads, seq, head)
        np.testing.assert_array_equal(got_k[pos], kr[pos])
        np.testing.assert_array_equal(got_v[pos], vr[pos])
        # and against the oracle's own serial projections within tolerance:
        # a bf16 row can differ by a rounding flip, one bf16 ulp of an
        # element (at most 2^-7 of it, so of the row's largest)
        assert rel_err(oracle.widen(got_k[pos], kv_dtype), oracle.widen(kc_pm[pos], kv_dtype)) \
            <= (RTOL if kv_dtype == F32 else 2.0 ** -7)


@pytest.mark.parametrize("dim,hidden,w_dtype", [(288, 768, F32), (4096, 14336, BF16)])
def test_gate_up_swiglu_fused(rt, dim, hidden, w_dtype):
    w1 = oracle.storage(oracle.normal(hidden * dim, 111, std=0.02), w_dtype).reshape(hidden, dim)
    w3 = oracle.storage(oracle.normal(hidden * dim, 112, std=0.02), w_dtype).reshape(hidden, dim)
    gh = 1.0 + 0.1 * oracle.normal(dim, 113)
    xh = oracle.normal(dim, 114)
    d1, d3, g, x, hb = up(rt, w1), up(rt, w3), up(rt, gh), up(rt, xh), rt.alloc(hidden * 4)
    call("ammon_gate_up_swiglu", rt.handle, None, x, g, F32, 1e-5, d1, d3, w_dtype, dim, hidden,
         hb)
    xn = oracle.rmsnorm(xh, gh).reshape(-1)
    want = oracle.swiglu(oracle.gemv(w1, w_dtype, xn), oracle.gemv(w3, w_dtype, xn))
    assert rel_err(down(hb, hidden), want) <= RTOL


# ---- argmax / greedy feedback ---------------------------------------------------------------------
def gpu_argmax(rt, logits):
    n = logits.size
    lg = up(rt, logits.astype(np.float32))
    scratch = rt.alloc(_abi.lib.ammon_argmax_scratch_bytes(n))
    out = rt.alloc(4)
    call("ammon_argmax", rt.handle, None, lg, n, scratch, out)
    return int(down(out, 1, np.int32)[0])


def test_argmax_picks_first_on_ties(rt):
    # src/tokenizer.rs:225-228
    assert gpu_argmax(rt, np.array([1.0, 3.0, 3.0, 2.0])) == 1


@pytest.mark.parametrize("case", [
    [1.0, np.nan, 0.5], [np.nan, 5.0, 9.0], [-np.inf, -np.inf], [0.0, -0.0, 1.0, 1.0],
    [-0.0, 0.0], [np.nan, np.nan], [2.0, np.nan, 2.0]])
def test_argmax_nan_and_signed_zero_rules(rt, case):
    a = np.array(case, np.float32)
    assert gpu_argmax(rt, a) == oracle.sample_argmax(a)


def test_argmax_large_with_spread_ties(rt):
    v = oracle.normal(128256, 121)
    assert gpu_argmax(rt, v) == oracle.sample_argmax(v)
    top = v.max() + 1
    for idx in (127000, 70001, 513, 90000):
        v[idx] = top
    assert gpu_argmax(rt, v) == 513 == oracle.sample_argmax(v)
    v[3] = np.nan
    assert gpu_argmax(rt, v) == 513
    v[0] = np.nan
    assert gpu_argmax(rt, v) == 0 == oracle.sample_argmax(v)


def test_greedy_next_feeds_decode_step(rt):
    n = 1000
    logits_h = oracle.normal(n, 131)
    best = int(np.argmax(logits_h))
    lg = up(rt, logits_h)
    scratch = rt.alloc(_abi.lib.ammon_argmax_scratch_bytes(n))
    prompt = up(rt, np.array([5, 6, 7], np.int32))
    tokens = up(rt, np.full(8, -1, np.int32))
    step = rt.step(5, 0)
    for _ in range(4):
        call("ammon_greedy_next", rt.handle, None, lg, n, scratch, prompt, 3, step, tokens, 8)
    # pos 0, 1 force prompt[1], prompt[2]; pos 2, 3 take the argmax
    np.testing.assert_array_equal(down(tokens, 8, np.int32), [6, 7, best, best, -1, -1, -1, -1])
    assert rt.read_step(step) == (best, 4)


# ---- fills ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [F32, BF16])
def test_fill_normal_matches_oracle_generator(rt, dtype):
    n = 1 << 20
    buf = rt.alloc(n * 4)
    rt.fill_normal(buf, dtype, n, 17, 5, 0.0, 0.02)
    got = down(buf, n, npdt(dtype))
    want = oracle.storage(oracle.normal(n, 17, 5, std=0.02), dtype)
    # Same integer stream and Box-Muller formula; the device's f64 log/sincos
    # may differ from libm in the last f64 ulp, which survives rounding to
    # fp32/bf16 only on an exact rounding boundary.
    assert np.mean(got != want) < 1e-5


@pytest.mark.parametrize("nbytes", [0, 8, 24, 4096, (1 << 22) + 8, (3 << 24) + 48])
def test_checksum_matches_numpy(rt, nbytes):
    # wrapping sum and xor of the little-endian 64-bit words, including an
    # 8-byte tail and sizes past the kernel's unrolled sweep
    rng = np.random.default_rng(nbytes)
    words = rng.integers(0, 1 << 63, size=nbytes // 8, dtype=np.uint64) * np.uint64(3)
    buf = up(rt, words) if nbytes else rt.alloc(16)
    out = rt.alloc(16)
    call("ammon_checksum", rt.handle, None, buf, nbytes, out)
    s, x = down(out, 2, np.uint64)
    assert int(s) == int(np.sum(words, dtype=np.uint64))
    assert int(x) == int(np.bitwise_xor.reduce(words)) if nbytes else int(x) == 0
    # twice in a row: the result words are cleared by the call itself
    call("ammon_checksum", rt.handle, None, buf, nbytes, out)
    np.testing.assert_array_equal(down(out, 2, np.uint64), [s, x])
    with pytest.raises(AmmonError, match="64-bit words"):
        call("ammon_checksum", rt.handle, None, buf, 12, out)


def test_stream_read_runs_at_every_size_and_leaves_memory_alone(rt):
    # a pure read: sizes below one window, ragged tails and several windows
    # per workgroup complete (the buffer resource reads past-the-end bytes as
    # zero) and the buffer is unchanged; misaligned sources are refused
    words = np.arange(1 << 21, dtype=np.uint64)
    buf = up(rt, words)
    for nbytes in (0, 16, 40, 16384 + 16, 3 << 20, words.nbytes):
        call("ammon_stream_read", rt.handle, None, buf, nbytes)
    rt.synchronize()
    np.testing.assert_array_equal(down(buf, words.size, np.uint64), words)
    with pytest.raises(AmmonError, match="16-byte aligned"):
        call("ammon_stream_read", rt.handle, None, ctypes.c_void_p(int(buf) + 8), 64)


def test_fill_const(rt):
    buf = rt.alloc(1000 * 4)
    rt.fill(buf, F32, 1000, 2.5)
    np.testing.assert_array_equal(down(buf, 1000), 2.5)
    rt.fill(buf, BF16, 1000, 1.0)
    np.testing.assert_array_equal(down(buf, 1000, np.uint16), 0x3F80)


@pytest.mark.parametrize("vocab,dim,w_dtype", [(32000, 288, F32), (128256, 512, BF16),
                                                (65541, 256, BF16)])
def test_greedy_lm_head_matches_unfused(rt, vocab, dim, w_dtype):
    """The LM head with the argmax folded into it gives the logits of
    ammon_gemv_rmsnorm bit for bit and the token of ammon_greedy_next on
    them, with ties (duplicated rows) and NaN rows in play."""
    wh = oracle.storage(oracle.normal(vocab * dim, 141, std=0.05), w_dtype).reshape(vocab, dim)
    gh = 1.0 + 0.1 * oracle.normal(dim, 142)
    xh = oracle.normal(dim, 143)
    top = int(np.argmax(oracle.gemv(wh, w_dtype, oracle.rmsnorm(xh, gh).reshape(-1))))
    for idx in (vocab - 3, 70, vocab // 2 + 1):  # copies of the winning row
        wh[idx] = wh[top]
    nan = 0x7FC0 if w_dtype == BF16 else np.nan  # bf16 rows hold raw bits
    wh[11] = nan  # a NaN logit never wins
    w, g, x = up(rt, wh), up(rt, gh), up(rt, xh)
    ref, fused = rt.alloc(vocab * 4), rt.alloc(vocab * 4)
    scratch = rt.alloc(max(_abi.lib.ammon_argmax_scratch_bytes(vocab),
                           _abi.lib.ammon_greedy_lm_head_scratch_bytes(rt.handle)))
    prompt = up(rt, np.array([5, 6], np.int32))
    tok_ref, tok_fused = up(rt, np.full(6, -1, np.int32)), up(rt, np.full(6, -1, np.int32))
    s_ref, s_fused = rt.step(5, 0), rt.step(5, 0)
    for i in range(4):
        call("ammon_gemv_rmsnorm", rt.handle, None, x, g, F32, 1e-5, w, w_dtype, vocab, dim, ref)
        call("ammon_greedy_next", rt.handle, None, ref, vocab, scratch, prompt, 2, s_ref,
             tok_ref, 6)
        call("ammon_greedy_lm_head", rt.handle, None, x, g, F32, 1e-5, w, w_dtype, vocab, dim,
             fused, scratch, _abi.lib.ammon_greedy_lm_head_scratch_bytes(rt.handle), prompt, 2,
             s_fused, tok_fused, 6)
        lr, lf = down(ref, vocab), down(fused, vocab)
        np.testing.assert_array_equal(lf.view(np.uint32), lr.view(np.uint32))
        assert rt.read_step(s_fused) == rt.read_step(s_ref)
        if i >= 1:  # past the forced prompt token
            assert rt.read_step(s_fused)[0] == oracle.sample_argmax(lf)
    got = down(tok_fused, 6, np.int32)
    np.testing.assert_array_equal(got, down(tok_ref, 6, np.int32))
    assert got[0] == 6 and got[4] == -1
    lr = down(ref, vocab)
    if lr[70] == lr[top]:  # bitwise tie between copies: the lowest index wins
        assert got[1] == min(70, top)
    # logits[0] NaN: the reference's comparison keeps index 0
    wh[0] = nan
    w.upload(wh)
    call("ammon_greedy_lm_head", rt.handle, None, x, g, F32, 1e-5, w, w_dtype, vocab, dim, fused,
         scratch, _abi.lib.ammon_greedy_lm_head_scratch_bytes(rt.handle), prompt, 2, s_fused,
         tok_fused, 6)
    assert rt.read_step(s_fused)[0] == 0


def test_greedy_lm_head_validation(rt):
    n = _abi.lib.ammon_greedy_lm_head_scratch_bytes(rt.handle)
    assert n > 0 and n % 8 == 0
    w, g, x, y = rt.alloc(64 * 64 * 4), rt.alloc(64 * 4), rt.alloc(64 * 4), rt.alloc(64 * 4)
    scratch, prompt, tokens = rt.alloc(n), rt.alloc(4), rt.alloc(16)
    step = rt.step(0, 0)
    with pytest.raises(AmmonError, match="scratch"):
        call("ammon_greedy_lm_head", rt.handle, None, x, g, F32, 1e-5, w, F32, 64, 64, y,
             scratch, 8, prompt, 1, step, tokens, 4)
