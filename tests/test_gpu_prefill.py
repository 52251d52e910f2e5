"""GPU tests of prompt prefill (multi-token GEMMs on matrix cores, token-
batched attention) through the C ABI.

Each prefill GEMM row is compared with the oracle's serial GEMV of that row
(<= 1e-5 relative, normwise: the products are exact in fp32 -- fp32 W on the
fp32 MFMA, bf16 W against x split into three bf16 parts -- so only the fp32
summation order differs).  Token-batched attention must equal the decode
attention of each token bit for bit (same splits, same units).  At model
level, prefilling a prompt must give the stepped prompt's logits and KV
cache within tolerance and the same greedy tokens, including the C1 golden
fixture.
"""
import ctypes
import json
import os

import numpy as np
import pytest

import oracle
from ammon_amd import LlamaModel, _abi
from ammon_amd._abi import BF16, F32, AmmonError, call

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
RTOL = 1e-5
# bf16 KV: the two sides' fp32 K/V differ only by summation order, which can
# flip a bf16 rounding by one ulp (at most 2^-7 of the element): stored rows
# within 2^-7 normwise, logits within 1e-3 normwise
KV_STORE_TOL = 2.0**-7
BF16_KV_TOL = 1e-3


def rel_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


def up(rt, a):
    return rt.upload(np.ascontiguousarray(a))


def npdt(dtype):
    return np.uint16 if dtype == BF16 else np.float32


def head_major(pm, kv_heads, seq, head):
    return np.ascontiguousarray(pm.reshape(seq, kv_heads, head).transpose(1, 0, 2))


def pos_major(hm, kv_heads, seq, head):
    return np.ascontiguousarray(hm.reshape(kv_heads, seq, head).transpose(1, 0, 2))


# ---- GEMM -----------------------------------------------------------------------------------
# (d, n, tokens): tails in every dimension -- rows past a 64-row tile, n past
# a 256-wide chunk (288 = 256 + 32), tokens past 16- and 32-token tiles.  The
# library splits the reduction over a workgroup's waves (16-row tiles) when
# 64-row tiles would not fill the device; the last two shapes take 64-row
# tiles (16- and 32-token variants).  From 64 tokens bf16 weights take 64-token
# tiles with 2 or 4 16-row tiles per wave: tails in rows (520, 1000), in the
# 64-wide reduction chunks (4104, 520) and in tokens (130 = 2 * 64 + 2).
GEMM_SHAPES = [(4096, 4096, 16), (1024, 4096, 33), (288, 288, 8), (768, 288, 40),
               (288, 768, 7), (100, 264, 5), (5, 8, 3), (64, 256, 1), (130, 4104, 64),
               (32768, 64, 16), (4096, 264, 256), (1000, 520, 130), (520, 4104, 64),
               (8192, 1024, 100)]


@pytest.mark.parametrize("d,n,tokens", GEMM_SHAPES)
@pytest.mark.parametrize("w_dtype", [BF16, F32])
def test_prefill_gemm_matches_oracle_gemv(rt, d, n, tokens, w_dtype):
    wh = oracle.storage(oracle.normal(d * n, 201, std=0.02), w_dtype).reshape(d, n)
    xh = oracle.normal(tokens * n, 202).reshape(tokens, n) * 2
    w, x, y = up(rt, wh), up(rt, xh), rt.alloc(tokens * d * 4)
    call("ammon_prefill_gemm", rt.handle, None, w, w_dtype, d, n, x, tokens, y, None)
    got = y.download((tokens, d))
    want = np.stack([oracle.gemv(wh, w_dtype, xh[t]) for t in range(tokens)])
    assert rel_err(got, want) <= RTOL
    # residual epilogue in place (x += W h, per row)
    rh = oracle.normal(tokens * d, 203).reshape(tokens, d)
    r = up(rt, rh)
    call("ammon_prefill_gemm", rt.handle, None, w, w_dtype, d, n, x, tokens, r, r)
    assert rel_err(r.download((tokens, d)), rh + want) <= RTOL


@pytest.mark.parametrize("d,n,tokens", [(1024, 8192, 64), (520, 4104, 100), (256, 2048, 40)])
def test_prefill_gemm_split_reduction(rt, d, n, tokens):
    """With a workspace, few-row projections split the reduction into ranges
    summed in order by a second launch: oracle parity, the residual form in
    place, repeatable to the bit, and equal within rounding to the unsplit
    GEMM."""
    wh = oracle.storage(oracle.normal(d * n, 205, std=0.02), BF16).reshape(d, n)
    xh = oracle.normal(tokens * n, 206).reshape(tokens, n)
    w, x = up(rt, wh), up(rt, xh)
    nbytes = _abi.lib.ammon_prefill_gemm_workspace_bytes(d, tokens)
    assert nbytes == 8 * tokens * d * 4
    ws = rt.alloc(nbytes)
    want = np.stack([oracle.gemv(wh, BF16, xh[t]) for t in range(tokens)])
    y1, y2, y0 = rt.alloc(tokens * d * 4), rt.alloc(tokens * d * 4), rt.alloc(tokens * d * 4)
    for y in (y1, y2):
        call("ammon_prefill_gemm_ws", rt.handle, None, w, BF16, d, n, x, tokens, y, None, ws, nbytes)
    call("ammon_prefill_gemm", rt.handle, None, w, BF16, d, n, x, tokens, y0, None)
    g1, g2, g0 = (b.download((tokens, d)) for b in (y1, y2, y0))
    np.testing.assert_array_equal(g1.view(np.uint32), g2.view(np.uint32))
    assert rel_err(g1, want) <= RTOL and rel_err(g1, g0) <= RTOL
    rh = oracle.normal(tokens * d, 207).reshape(tokens, d)
    r = up(rt, rh)
    call("ammon_prefill_gemm_ws", rt.handle, None, w, BF16, d, n, x, tokens, r, r, ws, nbytes)
    assert rel_err(r.download((tokens, d)), rh + want) <= RTOL
    with pytest.raises(AmmonError, match="workspace overlaps"):
        call("ammon_prefill_gemm_ws", rt.handle, None, w, BF16, d, n, x, tokens, y1, None, y1,
             nbytes)


def test_prefill_gemm_random_shapes(rt):
    """Seeded random shapes through every tile family and the split
    reduction (rows, reduction length and tokens off every tile multiple),
    bf16 weights, with and without a workspace, against the oracle."""
    rng = np.random.default_rng(12)
    for case in range(16):
        d = int(rng.integers(1, 700))
        n = 8 * int(rng.integers(1, 700))
        tokens = int(rng.choice([1, 3, 16, 17, 31, 33, 63, 64, 65, 100, 130]))
        wh = oracle.storage(oracle.normal(d * n, 300 + case, std=0.05), BF16).reshape(d, n)
        xh = oracle.normal(tokens * n, 400 + case).reshape(tokens, n)
        rh = oracle.normal(tokens * d, 500 + case).reshape(tokens, d)
        want = np.stack([oracle.gemv(wh, BF16, xh[t]) for t in range(tokens)])
        w, x = up(rt, wh), up(rt, xh)
        nbytes = _abi.lib.ammon_prefill_gemm_workspace_bytes(d, tokens)
        ws = rt.alloc(nbytes)
        for use_ws in (False, True):
            r = up(rt, rh)
            if use_ws:
                call("ammon_prefill_gemm_ws", rt.handle, None, w, BF16, d, n, x, tokens, r, r, ws,
                     nbytes)
            else:
                call("ammon_prefill_gemm", rt.handle, None, w, BF16, d, n, x, tokens, r, r)
            # the projection part (y - residual: exact but for y's rounding)
            got = r.download((tokens, d)).astype(np.float64) - rh
            assert rel_err(got, want) <= 2 * RTOL, (d, n, tokens, use_ws)


def test_prefill_gemm_identity_is_exact(rt):
    # the reference's identity GEMV (tests/kernels.rs:83-97) per row: exact
    for w_dtype in (F32, BF16):
        n = 64
        wh = oracle.storage(np.eye(n, dtype=np.float32), w_dtype)
        xh = oracle.normal(3 * n, 204).reshape(3, n)
        w, x, y = up(rt, wh), up(rt, xh), rt.alloc(3 * n * 4)
        call("ammon_prefill_gemm", rt.handle, None, w, w_dtype, n, n, x, 3, y, None)
        np.testing.assert_array_equal(y.download((3, n)), xh)


def test_prefill_gemm_validation(rt):
    w = up(rt, np.zeros((8, 12), np.float32))
    x = up(rt, np.zeros((2, 12), np.float32))
    y = rt.alloc(2 * 8 * 4)
    with pytest.raises(AmmonError, match="multiple of 8"):
        call("ammon_prefill_gemm", rt.handle, None, w, F32, 8, 12, x, 2, y, None)
    x8 = up(rt, np.zeros((2, 8), np.float32))
    with pytest.raises(AmmonError, match="y overlaps x"):
        call("ammon_prefill_gemm", rt.handle, None, w, F32, 8, 8, x8, 2, x8, None)
    with pytest.raises(AmmonError, match="empty shape"):
        call("ammon_prefill_gemm", rt.handle, None, w, F32, 8, 8, x8, 0, y, None)


@pytest.mark.parametrize("dim,hidden,tokens,w_dtype",
                         [(288, 768, 8, F32), (4096, 14336, 16, BF16), (64, 200, 35, BF16),
                          (64, 16400, 16, BF16), (64, 4100, 100, F32), (256, 1000, 130, BF16),
                          (512, 8192, 64, BF16)])
def test_prefill_gate_up_swiglu(rt, dim, hidden, tokens, w_dtype):
    w1 = oracle.storage(oracle.normal(hidden * dim, 211, std=0.02), w_dtype).reshape(hidden, dim)
    w3 = oracle.storage(oracle.normal(hidden * dim, 212, std=0.02), w_dtype).reshape(hidden, dim)
    xh = oracle.normal(tokens * dim, 213).reshape(tokens, dim)
    d1, d3, x, hb = up(rt, w1), up(rt, w3), up(rt, xh), rt.alloc(tokens * hidden * 4)
    call("ammon_prefill_gate_up_swiglu", rt.handle, None, x, tokens, d1, d3, w_dtype, dim,
         hidden, hb)
    want = np.stack([oracle.swiglu(oracle.gemv(w1, w_dtype, xh[t]), oracle.gemv(w3, w_dtype, xh[t]))
                     for t in range(tokens)])
    assert rel_err(hb.download((tokens, hidden)), want) <= RTOL


@pytest.mark.parametrize("shape", ["c1", "c4", "c4_long"])
@pytest.mark.parametrize("kv_dtype", [F32, BF16])
@pytest.mark.parametrize("use_ws", [False, True])
def test_prefill_qkv_rope_store(rt, shape, kv_dtype, use_ws):
    """use_ws: the workspace entry, whose c4 shape (6144 rows, 40 tokens)
    splits the reduction and rotates / stores in the summing launch."""
    if shape == "c1":
        dim, q_heads, kv_heads, head, seq, w_dtype, theta, p0, T = 288, 6, 6, 48, 64, F32, 1e4, 0, 9
    elif shape == "c4":
        dim, q_heads, kv_heads, head, seq, w_dtype, theta, p0, T = 4096, 32, 8, 128, 96, BF16, 5e5, 30, 40
    else:  # enough token tiles for 64-row tiles; a narrow model keeps the oracle quick
        dim, q_heads, kv_heads, head, seq, w_dtype, theta, p0, T = 512, 32, 8, 128, 256, BF16, 5e5, 5, 200
    qd, kd = q_heads * head, kv_heads * head
    wq = oracle.storage(oracle.normal(qd * dim, 221, std=0.02), w_dtype).reshape(qd, dim)
    wk = oracle.storage(oracle.normal(kd * dim, 222, std=0.02), w_dtype).reshape(kd, dim)
    wv = oracle.storage(oracle.normal(kd * dim, 223, std=0.02), w_dtype).reshape(kd, dim)
    xh = oracle.normal(T * dim, 224).reshape(T, dim)
    table_h = oracle.rope_table(theta, head, seq)
    kc_pm = np.zeros((seq, kv_heads, head), npdt(kv_dtype))
    vc_pm = np.zeros_like(kc_pm)
    want_q = np.zeros((T, qd), np.float32)
    for t in range(T):
        q = oracle.gemv(wq, w_dtype, xh[t])
        oracle.rope_store(q, oracle.gemv(wk, w_dtype, xh[t]), kc_pm, kv_dtype, head, p0 + t, table_h)
        oracle.cache_store(oracle.gemv(wv, w_dtype, xh[t]), vc_pm, kv_dtype, p0 + t)
        want_q[t] = q
    kc = up(rt, np.zeros((kv_heads, seq, head), npdt(kv_dtype)))
    vc = up(rt, np.zeros((kv_heads, seq, head), npdt(kv_dtype)))
    x, q, table = up(rt, xh), rt.alloc(T * qd * 4), up(rt, table_h)
    step = rt.step(0, p0)
    if use_ws:
        nbytes = _abi.lib.ammon_prefill_gemm_workspace_bytes(qd + 2 * kd, T)
        call("ammon_prefill_qkv_rope_store_ws", rt.handle, None, x, T, up(rt, wq), up(rt, wk),
             up(rt, wv), w_dtype, dim, q_heads, kv_heads, head, q, kc, vc, kv_dtype, seq, step,
             table, rt.alloc(nbytes), nbytes)
    else:
        call("ammon_prefill_qkv_rope_store", rt.handle, None, x, T, up(rt, wq), up(rt, wk),
             up(rt, wv), w_dtype, dim, q_heads, kv_heads, head, q, kc, vc, kv_dtype, seq, step,
             table)
    assert rel_err(q.download((T, qd)), want_q) <= RTOL
    got_k = pos_major(kc.download((kv_heads, seq, head), npdt(kv_dtype)), kv_heads, seq, head)
    got_v = pos_major(vc.download((kv_heads, seq, head), npdt(kv_dtype)), kv_heads, seq, head)
    tol = RTOL if kv_dtype == F32 else KV_STORE_TOL
    for got, want in ((got_k, kc_pm), (got_v, vc_pm)):
        assert rel_err(oracle.widen(got, kv_dtype), oracle.widen(want, kv_dtype)) <= tol
        # rows outside [p0, p0 + T) untouched
        np.testing.assert_array_equal(got[:p0], 0)
        np.testing.assert_array_equal(got[p0 + T:], 0)


def test_prefill_qkv_positions_past_cache_poison_q(rt):
    # tokens whose position reaches seq: q rows are NaN, no cache write
    dim, q_heads, kv_heads, head, seq, T = 64, 2, 1, 32, 20, 8
    qd, kd = q_heads * head, kv_heads * head
    wq = oracle.storage(oracle.normal(qd * dim, 231, std=0.1), BF16).reshape(qd, dim)
    wk = oracle.storage(oracle.normal(kd * dim, 232, std=0.1), BF16).reshape(kd, dim)
    wv = oracle.storage(oracle.normal(kd * dim, 233, std=0.1), BF16).reshape(kd, dim)
    kc = up(rt, np.zeros((kv_heads, seq + 4, head), np.float32))  # guard rows past seq
    vc = up(rt, np.zeros((kv_heads, seq + 4, head), np.float32))
    x, q = up(rt, oracle.normal(T * dim, 234).reshape(T, dim)), rt.alloc(T * qd * 4)
    table = up(rt, oracle.rope_table(5e5, head, seq))
    step = rt.step(0, seq - 3)
    call("ammon_prefill_qkv_rope_store", rt.handle, None, x, T, up(rt, wq), up(rt, wk), up(rt, wv),
         BF16, dim, q_heads, kv_heads, head, q, kc, vc, F32, seq, step, table)
    got_q = q.download((T, qd))
    assert np.isfinite(got_q[:3]).all() and np.isnan(got_q[3:]).all()
    for c in (kc, vc):
        rows = c.download((kv_heads, seq + 4, head))[0]
        assert np.count_nonzero(rows[seq - 3:seq].any(axis=1)) == 3
        np.testing.assert_array_equal(rows[seq:], 0)


# ---- attention ------------------------------------------------------------------------------
@pytest.mark.parametrize("q_heads,kv_heads,head,seq,p0,T,split,kv_dtype", [
    (32, 8, 128, 512, 0, 40, 16, BF16),
    (32, 8, 128, 512, 300, 17, 64, BF16),
    (6, 6, 48, 256, 0, 9, 16, F32),
    (4, 2, 64, 80, 10, 70, 8, F32),
    (8, 1, 128, 300, 250, 50, 32, F32),
    (4, 2, 64, 1200, 1100, 5, 8, F32),    # 138..139 live splits: several per split lane
    (2, 1, 32, 4200, 4100, 3, 8, BF16),   # 513+: the decode merge's second pass
])
def test_attention_prefill_equals_decode_per_token(rt, q_heads, kv_heads, head, seq, p0, T, split,
                                                  kv_dtype):
    dt = npdt(kv_dtype)
    kc_pm = oracle.storage(oracle.normal(seq * kv_heads * head, 241), kv_dtype).reshape(
        seq, kv_heads, head)
    vc_pm = oracle.storage(oracle.normal(seq * kv_heads * head, 242), kv_dtype).reshape(
        seq, kv_heads, head)
    qh = oracle.normal(T * q_heads * head, 243).reshape(T, q_heads, head)
    kc, vc = up(rt, head_major(kc_pm, kv_heads, seq, head)), up(rt, head_major(vc_pm, kv_heads, seq, head))
    q, out = up(rt, qh), rt.alloc(T * q_heads * head * 4)
    ctx = p0 + T
    nbytes = _abi.lib.ammon_attention_prefill_scratch_bytes(T, q_heads, head, ctx, split)
    part = up(rt, np.full(nbytes // 4, np.nan, np.float32))
    step = rt.step(0, p0)
    call("ammon_attention_prefill", rt.handle, None, q, T, q_heads, kc, vc, kv_dtype, kv_heads,
         head, seq, step, ctx, split, part, nbytes, out)
    got = out.download((T, q_heads, head))
    # the decode attention of each token at its position: identical units
    dpart_n = _abi.lib.ammon_attention_scratch_bytes(q_heads, head, seq, split)
    dpart, dout = rt.alloc(dpart_n), rt.alloc(q_heads * head * 4)
    for t in range(T):
        qt = up(rt, qh[t])
        rt.deposit(step, 0, p0 + t)
        call("ammon_attention_decode", rt.handle, None, qt, q_heads, kc, vc, kv_dtype, kv_heads,
             head, seq, step, split, dpart, dpart_n, dout)
        np.testing.assert_array_equal(got[t], dout.download((q_heads, head)))
    # and the oracle's split attention (split 8) within tolerance
    for t in (0, T // 2, T - 1):
        want = oracle.attention(qh[t], kc_pm, vc_pm, kv_dtype, p0 + t)
        assert rel_err(got[t], want) <= RTOL


@pytest.mark.parametrize("kv_dtype", [F32, BF16])
def test_attention_prefill_positions_past_ctx_are_poisoned(rt, kv_dtype):
    # The grid and the scratch cover ctx positions; the host cannot see
    # step->position, so a token at position >= ctx (but < seq) must get NaN
    # and write no partial instead of silently dropping the keys past ctx.
    q_heads, kv_heads, head, seq, split, T, ctx, p0 = 4, 2, 64, 64, 8, 6, 20, 17
    kc_pm = oracle.storage(oracle.normal(seq * kv_heads * head, 251), kv_dtype).reshape(
        seq, kv_heads, head)
    vc_pm = oracle.storage(oracle.normal(seq * kv_heads * head, 252), kv_dtype).reshape(
        seq, kv_heads, head)
    qh = oracle.normal(T * q_heads * head, 253).reshape(T, q_heads, head)
    kc, vc = up(rt, head_major(kc_pm, kv_heads, seq, head)), up(rt, head_major(vc_pm, kv_heads, seq, head))
    q, out = up(rt, qh), rt.alloc(T * q_heads * head * 4)
    nbytes = _abi.lib.ammon_attention_prefill_scratch_bytes(T, q_heads, head, ctx, split)
    part_h = np.full(nbytes // 4, 7.0, np.float32)  # a sentinel no write leaves
    part = up(rt, part_h)
    step = rt.step(0, p0)
    call("ammon_attention_prefill", rt.handle, None, q, T, q_heads, kc, vc, kv_dtype, kv_heads,
         head, seq, step, ctx, split, part, nbytes, out)
    got = out.download((T, q_heads, head))
    live = ctx - p0  # tokens at positions p0 .. ctx - 1
    for t in range(live):
        want = oracle.attention(qh[t], kc_pm, vc_pm, kv_dtype, p0 + t)
        assert rel_err(got[t], want) <= RTOL, t
    assert np.isnan(got[live:]).all()
    splits = _abi.lib.ammon_attention_splits(ctx, split)
    per_token = q_heads * splits * (head + 2)
    after = part.download(nbytes // 4)
    np.testing.assert_array_equal(after[live * per_token:], 7.0)


def test_attention_prefill_validation(rt):
    q = up(rt, np.zeros((2, 2, 64), np.float32))
    kc = up(rt, np.zeros((1, 16, 64), np.float32))
    step = rt.step(0, 0)
    out = rt.alloc(2 * 2 * 64 * 4)
    part = rt.alloc(1 << 16)
    with pytest.raises(AmmonError, match="ctx"):
        call("ammon_attention_prefill", rt.handle, None, q, 2, 2, kc, kc, F32, 1, 64, 16, step, 17,
             8, part, 1 << 16, out)
    with pytest.raises(AmmonError, match="partial scratch"):
        call("ammon_attention_prefill", rt.handle, None, q, 2, 2, kc, kc, F32, 1, 64, 16, step, 16,
             8, part, 16, out)


# ---- model ----------------------------------------------------------------------------------
@pytest.mark.parametrize("heads,kv_dtype,w_dtype", [((32, 8), BF16, BF16), ((4, 4), F32, F32),
                                                    ((8, 2), F32, BF16)])
def test_model_prefill_matches_stepping(rt, heads, kv_dtype, w_dtype):
    n_heads, n_kv = heads
    cfg = oracle.LlamaConfig(dim=128 * n_heads if n_heads > 4 else 256, n_layers=2,
                             n_heads=n_heads, n_kv_heads=n_kv, hidden=1544, vocab=5003,
                             max_seq=300, theta=500000.0, w_dtype=w_dtype, kv_dtype=kv_dtype)
    stepped = LlamaModel.synthetic(rt, cfg, seed=41, std=0.05)
    filled = LlamaModel(rt, cfg, stepped.weights)
    # 100 tokens: the 64-token GEMM tiles for bf16 weights
    prompt = [int(t) for t in np.arange(100) * 131 % 5003]
    for pos, tok in enumerate(prompt):
        want = stepped.step(tok, pos)
    got = filled.prefill(prompt)
    # fp32 KV: only summation order differs; bf16 KV: a last-bit difference
    # in an fp32 K/V value can flip its bf16 rounding by one ulp
    tol = 1e-4 if kv_dtype == F32 else BF16_KV_TOL
    kv_tol = 1e-4 if kv_dtype == F32 else KV_STORE_TOL
    assert rel_err(got, want) <= tol
    for l in range(cfg.n_layers):
        for g, w in zip(filled.kv_layer(l), stepped.kv_layer(l)):
            g, w = oracle.widen(g, kv_dtype), oracle.widen(w, kv_dtype)  # bf16 storage bits
            assert rel_err(g[: len(prompt)], w[: len(prompt)]) <= kv_tol
            np.testing.assert_array_equal(g[len(prompt):], 0)
    # decoding on from the prefilled cache gives the stepped model's tokens
    nxt = oracle.sample_argmax(want)
    np.testing.assert_array_equal(filled.decode(nxt, len(prompt), 12, read_tokens=True),
                                  stepped.decode(nxt, len(prompt), 12, read_tokens=True))
    # the prefill entry also works mid-sequence (a second chunk of positions)
    more = [3, 17, 400, 5002, 1]
    p0 = len(prompt) + 12
    for i, tok in enumerate(more):
        want2 = stepped.step(tok, p0 + i)
    assert rel_err(filled.prefill(more, p0), want2) <= tol
    filled.close()
    stepped.close()


def test_generate_prefill_matches_device_loop(rt):
    cfg = oracle.LlamaConfig(dim=512, n_layers=2, n_heads=4, n_kv_heads=2, hidden=1024,
                             vocab=3001, max_seq=128, theta=500000.0, w_dtype=BF16,
                             kv_dtype=F32)
    m = LlamaModel.synthetic(rt, cfg, seed=43, std=0.05)
    prompt = [5, 900, 2999, 17, 4, 4, 1200, 31, 77, 2048, 6]
    toks_d, logits_d, _ = m.generate_tokens_device(prompt, 60)
    toks_p, logits_p, tps = m.generate_tokens_prefill(prompt, 60)
    np.testing.assert_array_equal(toks_p, toks_d)
    assert rel_err(logits_p, logits_d) <= 1e-4
    assert tps > 0
    # stop token and a limit inside the prompt behave as the stepped loop
    stop = int(toks_d[len(prompt) + 3])
    np.testing.assert_array_equal(m.generate_tokens_prefill(prompt, 60, stop_on=stop)[0],
                                  m.generate_tokens_device(prompt, 60, stop_on=stop)[0])
    np.testing.assert_array_equal(m.generate_tokens_prefill(prompt, 6)[0],
                                  m.generate_tokens_device(prompt, 6)[0])
    m.close()


def test_c1_prefill_greedy_matches_fixture(rt):
    f = np.load(os.path.join(HERE, "golden", "c1_greedy.npz"))
    cfg = oracle.LlamaConfig(**json.loads(str(f["config"])))
    weights = oracle.random_weights(cfg, seed=int(f["weight_seed"]), std=0.02)
    m = LlamaModel.from_host(rt, cfg, weights)
    toks, logits, _ = m.generate_tokens_prefill(f["prompt"], int(f["max_new_tokens"]))
    np.testing.assert_array_equal(toks, f["tokens"])
    assert rel_err(logits, f["logits"]) <= 1e-4
    m.close()


def test_model_prefill_validation(rt):
    cfg = oracle.LlamaConfig(dim=256, n_layers=1, n_heads=2, n_kv_heads=1, hidden=512, vocab=300,
                             max_seq=32, theta=500000.0, w_dtype=BF16, kv_dtype=BF16)
    m = LlamaModel.synthetic(rt, cfg, seed=44, std=0.05)
    with pytest.raises(AmmonError, match="outside the vocab"):
        m.prefill([1, 300])
    with pytest.raises(AmmonError, match="exceeds max_seq"):
        m.prefill(list(range(20)), 20)
    m.close()
