"""Pins the CPU oracle (oracle/ammon_oracle.c) before it is trusted as the
parity reference.

Each oracle function is checked against something that does not restate it:
the reference's own known-answer tests (tests/kernels.rs, src/tokenizer.rs),
the reference's f64 attention (tests/kernels.rs:400-427) on its own xorshift
inputs, numpy/scipy float64 closed forms, torch's bf16 rounding, invariants
(RoPE at position 0 is the identity; rotations keep pair norms), and an f64
brute-force model.  Tolerances are stated per test.
"""
import numpy as np
import pytest
import scipy.special

import oracle
from oracle import BF16, F32


def rel_err(got, want):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


# ---- bf16 --------------------------------------------------------------------
def test_bf16_round_to_nearest_even_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10,
        np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, 3.0e38, 1e-40, -1e-40], np.float32),
        # exact halfway cases: low 16 bits 0x8000 with even and odd kept bit
        np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x3F80FFFF, 0x3F807FFF],
                 np.uint32).view(np.float32),
    ])
    got = oracle.to_bf16(vals)
    want = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, want)
    # widening is exact
    np.testing.assert_array_equal(oracle.from_bf16(got),
                                  (got.astype(np.uint32) << 16).view(np.float32))


def test_bf16_nan_stays_nan():
    vals = np.array([np.nan, -np.nan], np.float32)
    assert np.all(np.isnan(oracle.from_bf16(oracle.to_bf16(vals))))


# ---- seeded inputs -------------------------------------------------------------
def test_pseudo_random_is_marsaglia_xorshift32():
    # tests/kernels.rs:380-390: state = seed*2654435761 + 1, then 13/17/5
    # xorshift, value = (state % 2001) / 1000 - 1.
    def xorshift(n, seed):
        s = (seed * 2654435761 + 1) & 0xFFFFFFFF
        out = []
        for _ in range(n):
            s ^= (s << 13) & 0xFFFFFFFF
            s ^= s >> 17
            s ^= (s << 5) & 0xFFFFFFFF
            out.append(np.float32(s % 2001) / np.float32(1000.0) - np.float32(1.0))
        return np.array(out, np.float32)

    for seed in (11, 12, 13, 0, 0xFFFFFFFF):
        np.testing.assert_array_equal(oracle.pseudo_random(257, seed), xorshift(257, seed))
    v = oracle.pseudo_random(100000, 12)
    assert v.min() >= -1.0 and v.max() <= 1.0


def test_normal_generator_statistics():
    v = oracle.normal(1 << 20, seed=7, stream=3, std=0.02).astype(np.float64)
    assert abs(v.mean()) < 1e-4
    assert abs(v.std() - 0.02) < 2e-4
    # distinct streams and seeds are independent draws
    w = oracle.normal(1 << 10, seed=7, stream=4)
    u = oracle.normal(1 << 10, seed=8, stream=3)
    assert not np.array_equal(w, oracle.normal(1 << 10, seed=7, stream=3))
    assert not np.array_equal(u, oracle.normal(1 << 10, seed=7, stream=3))
    # prefix stability: element i does not depend on n
    np.testing.assert_array_equal(oracle.normal(1001, 5, 1), oracle.normal(2000, 5, 1)[:1001])


# ---- embed ---------------------------------------------------------------------
def test_embed_gathers_selected_row():
    # tests/kernels.rs:36-52
    table = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    np.testing.assert_array_equal(oracle.embed(table, F32, [1])[0], [3.0, 4.0])


def test_embed_deposit_values():
    # tests/kernels.rs:184-222: token 0 -> [10, 20], token 1 -> [30, 40]
    table = np.array([[10.0, 20.0], [30.0, 40.0]], np.float32)
    np.testing.assert_array_equal(oracle.embed(table, F32, [0, 1]), [[10, 20], [30, 40]])


def test_embed_bf16_is_exact_widening():
    t = oracle.to_bf16(oracle.normal(64 * 48, 1).reshape(64, 48))
    ids = np.array([5, 0, 63, 5], np.uint32)
    np.testing.assert_array_equal(oracle.embed(t, BF16, ids), oracle.from_bf16(t)[ids])


# ---- rmsnorm --------------------------------------------------------------------
def test_rmsnorm_of_ones():
    # tests/kernels.rs:163-182: each output within 1e-5 of 1/sqrt(1 + 1e-5)
    out = oracle.rmsnorm(np.ones(4, np.float32), np.ones(4, np.float32))
    scale = 1.0 / np.sqrt(np.float32(1.0) + np.float32(1e-5))
    assert np.all(np.abs(out - scale) < 1e-5)


@pytest.mark.parametrize("dim,rows", [(4096, 1), (4096, 64), (288, 3), (300, 2), (8192, 1)])
@pytest.mark.parametrize("w_dtype", [F32, BF16])
def test_rmsnorm_matches_f64_closed_form(dim, rows, w_dtype):
    x = oracle.normal(rows * dim, 1).reshape(rows, dim)
    w = oracle.storage(oracle.normal(dim, 2), w_dtype)
    wf = oracle.widen(w, w_dtype).astype(np.float64)
    got = oracle.rmsnorm(x, w, w_dtype)
    x64 = x.astype(np.float64)
    want = wf * x64 / np.sqrt(np.mean(x64 * x64, axis=1, keepdims=True) + 1e-5)
    assert rel_err(got, want) < 1e-6


# ---- RoPE -------------------------------------------------------------------------
def test_rope_table_position_zero_is_identity():
    t = oracle.rope_table(500000.0, 128, 4)
    np.testing.assert_array_equal(t[0, :, 0], 1.0)
    np.testing.assert_array_equal(t[0, :, 1], 0.0)


@pytest.mark.parametrize("theta,head", [(10000.0, 48), (500000.0, 128), (10000.0, 2)])
def test_rope_table_matches_f64_frequencies(theta, head):
    seq = 8192
    t = oracle.rope_table(theta, head, seq).astype(np.float64)
    pos = np.arange(seq, dtype=np.float64)[:, None]
    hd = 2.0 * np.arange(head // 2, dtype=np.float64)[None, :]
    ang = pos * theta ** (-hd / head)
    # The reference rounds the angle to fp32 (src/kernels.rs:196-197): allow a
    # few ulp of the angle plus the frequency's relative rounding.
    tol = 4.0 * np.spacing(np.float32(np.maximum(ang, 1.0))).astype(np.float64) + 1e-6
    assert np.all(np.abs(t[..., 0] - np.cos(ang)) <= tol)
    assert np.all(np.abs(t[..., 1] - np.sin(ang)) <= tol)


def test_rope_store_rotates_q_and_writes_k_row():
    # tests/kernels.rs:239-283: head 2, pos 1, theta 10000 -> rotation by 1 rad;
    # K row 0 untouched, row 1 = rotated (3, 4); abs 1e-5.
    table = oracle.rope_table(10000.0, 2, 2)
    q = np.array([1.0, 2.0], np.float32)
    k_proj = np.array([3.0, 4.0], np.float32)
    k = np.zeros((2, 1, 2), np.float32)
    oracle.rope_store(q, k_proj, k, F32, head=2, pos=1, table=table)
    c, s = np.cos(1.0), np.sin(1.0)
    assert np.allclose(q, [1 * c - 2 * s, 1 * s + 2 * c], atol=1e-5)
    np.testing.assert_array_equal(k[0, 0], [0.0, 0.0])
    assert np.allclose(k[1, 0], [3 * c - 4 * s, 3 * s + 4 * c], atol=1e-5)


def test_rope_at_pos_zero_is_identity():
    # tests/kernels.rs:54-81
    table = oracle.rope_table(10000.0, 2, 1)
    q = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    k = np.zeros((1, 2, 2), np.float32)
    oracle.rope_store(q, np.array([5.0, 6.0, 7.0, 8.0], np.float32), k, F32, 2, 0, table)
    np.testing.assert_array_equal(q, [1.0, 2.0, 3.0, 4.0])
    np.testing.assert_array_equal(k.reshape(-1), [5.0, 6.0, 7.0, 8.0])


def test_rope_store_matches_complex_rotation_and_keeps_norms():
    theta, q_heads, kv_heads, head, seq = 500000.0, 32, 8, 128, 64
    table = oracle.rope_table(theta, head, seq)
    for pos in (0, 1, 7, 63):
        q = oracle.normal(q_heads * head, 10 + pos)
        kp = oracle.normal(kv_heads * head, 20 + pos)
        q0, k0 = q.copy(), kp.copy()
        k = np.zeros((seq, kv_heads, head), np.float32)
        oracle.rope_store(q, kp, k, F32, head, pos, table)
        # Independent formulation: pair (2p, 2p+1) as a complex number times
        # e^{i pos theta^(-2p/head)}, in complex128.
        for src, got in ((q0, q), (k0, k[pos].reshape(-1))):
            z = src.astype(np.float64).reshape(-1, head // 2, 2)
            zc = z[..., 0] + 1j * z[..., 1]
            ang = pos * theta ** (-2.0 * np.arange(head // 2) / head)
            rot = zc * np.exp(1j * ang)
            want = np.stack([rot.real, rot.imag], -1).reshape(-1)
            assert np.max(np.abs(got - want)) < 1e-4
            # rotation preserves each pair's norm
            gz = got.astype(np.float64).reshape(-1, 2)
            np.testing.assert_allclose(np.hypot(gz[:, 0], gz[:, 1]),
                                       np.abs(zc).reshape(-1), rtol=1e-5)
        assert np.all(k[np.arange(seq) != pos] == 0)


def test_rope_store_bf16_cache_is_rne_of_fp32():
    head, seq, pos = 64, 8, 5
    table = oracle.rope_table(10000.0, head, seq)
    q = oracle.normal(2 * head, 1)
    kp = oracle.normal(head, 2)
    k32 = np.zeros((seq, 1, head), np.float32)
    k16 = np.zeros((seq, 1, head), np.uint16)
    oracle.rope_store(q.copy(), kp, k32, F32, head, pos, table)
    oracle.rope_store(q.copy(), kp, k16, BF16, head, pos, table)
    np.testing.assert_array_equal(k16, oracle.to_bf16(k32))


# ---- cache store -------------------------------------------------------------------
def test_cache_store_writes_row_at_position():
    # tests/kernels.rs:285-307
    dst = np.zeros((3, 1, 2), np.float32)
    oracle.cache_store(np.array([9.0, 8.0], np.float32), dst, F32, pos=2)
    np.testing.assert_array_equal(dst.reshape(-1), [0, 0, 0, 0, 9, 8])


# ---- GEMV ------------------------------------------------------------------------------
def test_gemv_identity():
    # tests/kernels.rs:83-97 and :342-355
    eye = np.eye(2, dtype=np.float32)
    np.testing.assert_array_equal(oracle.gemv(eye, F32, np.array([1.0, 2.0], np.float32)),
                                  [1.0, 2.0])
    np.testing.assert_array_equal(oracle.gemv(eye, F32, np.array([3.0, 4.0], np.float32)),
                                  [3.0, 4.0])


@pytest.mark.parametrize("d,n", [(7, 5), (1024, 4096), (4096, 14336), (33, 300), (1, 1)])
@pytest.mark.parametrize("w_dtype", [F32, BF16])
def test_gemv_matches_f64_matmul(d, n, w_dtype):
    w = oracle.storage(oracle.normal(d * n, 3, std=0.02).reshape(d, n), w_dtype)
    x = oracle.normal(n, 4)
    want = oracle.widen(w, w_dtype).astype(np.float64) @ x.astype(np.float64)
    got = oracle.gemv(w, w_dtype, x)
    # normwise: fp32 accumulation over n terms
    assert np.max(np.abs(got - want)) <= 1e-6 * np.sqrt(n) * np.max(np.abs(want)) + 1e-6


@pytest.mark.parametrize("d,n", [(1, 1), (3, 7), (31, 9), (32, 8), (33, 17), (77, 1003),
                                 (1024, 4096), (300, 14336)])
@pytest.mark.parametrize("w_dtype", [F32, BF16])
@pytest.mark.parametrize("descending", [False, True])
def test_gemv_vector_path_equals_serial_chains(d, n, w_dtype, descending):
    # The vector path (8 rows per register, 8 x 8 transposes) keeps every
    # row's serial order: bit-identical to one scalar chain per row, in the
    # reference's order and in the descending order the drift study uses.
    w = oracle.storage(oracle.normal(d * n, 13, std=0.5).reshape(d, n), w_dtype)
    x = oracle.normal(n, 14)
    oracle.set_gemv_order(descending)
    try:
        got, want = oracle.gemv(w, w_dtype, x), oracle.gemv_scalar(w, w_dtype, x)
    finally:
        oracle.set_gemv_order(False)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    # the descending order is a different summation order of the same sums
    if descending and n > 8:
        ref = oracle.widen(w, w_dtype).astype(np.float64) @ x.astype(np.float64)
        assert np.max(np.abs(got - ref)) <= 1e-6 * np.sqrt(n) * np.max(np.abs(ref)) + 1e-6


def test_add_is_elementwise():
    # tests/kernels.rs:224-237
    np.testing.assert_array_equal(oracle.add(np.array([1.0, 2.0]), np.array([3.0, 4.0])), [4, 6])


# ---- SwiGLU --------------------------------------------------------------------------
def test_swiglu_of_zero_is_zero():
    # tests/kernels.rs:148-161
    np.testing.assert_array_equal(oracle.swiglu(np.zeros(2, np.float32),
                                                np.array([5.0, 7.0], np.float32)), [0.0, 0.0])


def test_swiglu_matches_expit_closed_form():
    g = oracle.normal(14336, 1) * 4
    u = oracle.normal(14336, 2)
    want = g.astype(np.float64) * scipy.special.expit(g.astype(np.float64)) * u
    got = oracle.swiglu(g, u)
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-30)


# ---- attention -----------------------------------------------------------------------
def cpu_attention_f64(q, key, value, q_heads, kv_heads, head, pos):
    """The reference's f64 attention (tests/kernels.rs:400-427), pos-major cache."""
    kv_mul = q_heads // kv_heads
    q = q.reshape(q_heads, head).astype(np.float64)
    k = key.astype(np.float64)
    v = value.astype(np.float64)
    out = np.zeros((q_heads, head))
    for h in range(q_heads):
        g = h // kv_mul
        scores = k[: pos + 1, g, :] @ q[h] / np.sqrt(head)
        w = np.exp(scores - scores.max())
        out[h] = (w[:, None] * v[: pos + 1, g, :]).sum(0) / w.sum()
    return out


REF_ATTENTION_CASES = [
    # tests/kernels.rs:493-538
    (6, 6, 48, 256, [0, 1, 7, 8, 9, 31, 32, 33, 100, 255]),
    (4, 2, 64, 80, [0, 47, 79]),
    (2, 1, 128, 40, [39]),
    (3, 3, 20, 33, [5, 32]),
    (1, 1, 32, 2112, [2047, 2111]),
]


@pytest.mark.parametrize("q_heads,kv_heads,head,seq,positions", REF_ATTENTION_CASES)
def test_split_and_serial_attention_match_f64_reference(q_heads, kv_heads, head, seq, positions):
    q = oracle.pseudo_random(q_heads * head, 11).reshape(q_heads, head)
    key = oracle.pseudo_random(seq * kv_heads * head, 12).reshape(seq, kv_heads, head)
    value = oracle.pseudo_random(seq * kv_heads * head, 13).reshape(seq, kv_heads, head)
    for pos in positions:
        want = cpu_attention_f64(q, key, value, q_heads, kv_heads, head, pos)
        # Dead splits stay NaN (the partial buffer starts poisoned); the
        # combine must never read them.
        split = oracle.attention(q, key, value, F32, pos)
        serial = oracle.attention_serial(q, key, value, F32, pos)
        assert np.max(np.abs(split - want)) < 1e-4, pos
        assert np.max(np.abs(serial - want)) < 1e-4, pos
        assert np.max(np.abs(split - want)) / np.max(np.abs(want)) < 1e-5, pos


def test_attention_partial_leaves_dead_splits_untouched():
    q_heads, kv_heads, head, seq, pos = 2, 1, 16, 64, 20
    q = oracle.pseudo_random(q_heads * head, 1).reshape(q_heads, head)
    k = oracle.pseudo_random(seq * head, 2).reshape(seq, 1, head)
    v = oracle.pseudo_random(seq * head, 3).reshape(seq, 1, head)
    part = oracle.attention_partial(q, k, v, F32, pos)
    live = pos // 8 + 1
    assert np.all(np.isfinite(part[:, :live]))
    assert np.all(np.isnan(part[:, live:]))


def test_attention_bf16_cache_matches_f64_on_widened_values():
    q_heads, kv_heads, head, seq, pos = 32, 8, 128, 1024, 1023
    q = oracle.normal(q_heads * head, 1).reshape(q_heads, head)
    k16 = oracle.to_bf16(oracle.normal(seq * kv_heads * head, 2)).reshape(seq, kv_heads, head)
    v16 = oracle.to_bf16(oracle.normal(seq * kv_heads * head, 3)).reshape(seq, kv_heads, head)
    got = oracle.attention(q, k16, v16, BF16, pos)
    want = cpu_attention_f64(q, oracle.from_bf16(k16), oracle.from_bf16(v16), q_heads, kv_heads,
                             head, pos)
    assert rel_err(got, want) < 1e-5


# ---- argmax ------------------------------------------------------------------------------
def test_argmax_picks_first_on_ties():
    # src/tokenizer.rs:225-228
    assert oracle.sample_argmax(np.array([1.0, 3.0, 3.0, 2.0], np.float32)) == 1


def test_argmax_nan_rules():
    nan = np.nan
    assert oracle.sample_argmax(np.array([1.0, nan, 0.5], np.float32)) == 0
    assert oracle.sample_argmax(np.array([nan, 5.0, 9.0], np.float32)) == 0
    assert oracle.sample_argmax(np.array([-np.inf, -np.inf], np.float32)) == 0
    assert oracle.sample_argmax(np.array([0.0, -0.0, 1.0, 1.0], np.float32)) == 2
    assert oracle.sample_argmax(np.array([-0.0, 0.0], np.float32)) == 0


def test_argmax_matches_numpy_without_nan():
    v = oracle.normal(128256, 9)
    assert oracle.sample_argmax(v) == int(np.argmax(v))
    v[77] = v[5000] = v.max() + 1
    assert oracle.sample_argmax(v) == 77


# ---- model and loop ---------------------------------------------------------------------------
TINY = dict(dim=16, n_layers=2, n_heads=4, n_kv_heads=2, hidden=40, vocab=50, max_seq=12,
            theta=10000.0)


def numpy_model_logits(cfg, w, tokens):
    """Float64 brute force of the llama2.c-convention graph over a token prefix;
    returns the logits after each token.  RoPE as complex rotation, full
    softmax attention, GQA by integer division of the head index."""
    c = cfg
    head = c.dim // c.n_heads
    kv_mul = c.n_heads // c.n_kv_heads
    f = {k: oracle.widen(v, c.w_dtype if not k.startswith("rms") else F32).astype(np.float64)
         for k, v in w.items()}

    def rms(x, g):
        return g * x / np.sqrt(np.mean(x * x) + c.eps)

    def rope(vec, pos):
        z = vec.reshape(-1, head // 2, 2)
        zc = z[..., 0] + 1j * z[..., 1]
        zc = zc * np.exp(1j * pos * c.theta ** (-2.0 * np.arange(head // 2) / head))
        return np.stack([zc.real, zc.imag], -1).reshape(-1)

    K = np.zeros((c.n_layers, len(tokens), c.n_kv_heads, head))
    V = np.zeros_like(K)
    out = []
    for pos, tok in enumerate(tokens):
        x = f["tok_emb"][tok].copy()
        for l in range(c.n_layers):
            xb = rms(x, f["rms_att"][l])
            q = rope(f["wq"][l] @ xb, pos).reshape(c.n_heads, head)
            K[l, pos] = rope(f["wk"][l] @ xb, pos).reshape(c.n_kv_heads, head)
            V[l, pos] = (f["wv"][l] @ xb).reshape(c.n_kv_heads, head)
            att = np.zeros((c.n_heads, head))
            for h in range(c.n_heads):
                g = h // kv_mul
                s = K[l, : pos + 1, g] @ q[h] / np.sqrt(head)
                p = np.exp(s - s.max())
                att[h] = (p[:, None] * V[l, : pos + 1, g]).sum(0) / p.sum()
            x = x + f["wo"][l] @ att.reshape(-1)
            xb = rms(x, f["rms_ffn"][l])
            a, b = f["w1"][l] @ xb, f["w3"][l] @ xb
            x = x + f["w2"][l] @ (a / (1 + np.exp(-a)) * b)
        out.append(f["wcls"] @ rms(x, f["rms_final"]))
    return np.array(out)


@pytest.mark.parametrize("w_dtype", [F32, BF16])
def test_model_matches_f64_brute_force(w_dtype):
    cfg = oracle.LlamaConfig(**TINY, w_dtype=w_dtype)
    w = oracle.random_weights(cfg, seed=3, std=0.3)
    w["rms_att"] = 1.0 + 0.1 * oracle.normal(cfg.n_layers * cfg.dim, 4).reshape(cfg.n_layers,
                                                                               cfg.dim)
    m = oracle.Model(cfg, w)
    tokens = [1, 7, 3, 49, 0, 12, 12, 5, 33, 2, 8]
    want = numpy_model_logits(cfg, w, tokens)
    for pos, tok in enumerate(tokens):
        got = m.step(tok, pos)
        assert rel_err(got, want[pos]) < 1e-5, pos


def test_model_kv_cache_holds_rope_of_projection():
    cfg = oracle.LlamaConfig(**TINY)
    w = oracle.random_weights(cfg, seed=5, std=0.3)
    m = oracle.Model(cfg, w)
    m.step(4, 0)
    m.step(9, 1)
    k, v = m.kv_layer(0)
    # position 0 has no rotation: K[0] = Wk rmsnorm(embed(4))
    xb = oracle.rmsnorm(w["tok_emb"][4], w["rms_att"][0])
    np.testing.assert_allclose(k[0].reshape(-1), oracle.gemv(w["wk"][0], F32, xb.reshape(-1)),
                               rtol=0, atol=0)
    np.testing.assert_allclose(v[0].reshape(-1), oracle.gemv(w["wv"][0], F32, xb.reshape(-1)),
                               rtol=0, atol=0)
    assert np.all(k[2:] == 0) and np.all(v[2:] == 0)


@pytest.mark.parametrize("kv_dtype", [F32, BF16])
def test_model_kv_hooks(kv_dtype):
    # kv_rows() returns exactly what a step stores at its position; with
    # stores off the cache is left as written; writing a step's own rows
    # and stepping with stores off gives the stored step's logits bit for
    # bit.
    cfg = oracle.LlamaConfig(**TINY, kv_dtype=kv_dtype)
    w = oracle.random_weights(cfg, seed=21, std=0.3)
    ref, m = oracle.Model(cfg, dict(w)), oracle.Model(cfg, dict(w))
    tokens = [5, 1, 9, 40, 3]
    for pos, tok in enumerate(tokens):
        want = ref.step(tok, pos)
        for layer in range(cfg.n_layers):
            k, v = ref.kv_layer(layer)
            rk, rv = ref.kv_rows(layer)
            np.testing.assert_array_equal(k[pos], rk)
            np.testing.assert_array_equal(v[pos], rv)
            m.write_kv(layer, pos, rk[None], rv[None])
        m.set_kv_store(False)
        got = m.step(tok, pos)
        m.set_kv_store(True)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    # with stores off a step leaves the cache untouched
    k_before, _ = m.kv_layer(0)
    m.set_kv_store(False)
    m.step(7, len(tokens))
    np.testing.assert_array_equal(m.kv_layer(0)[0], k_before)
    with pytest.raises(ValueError):
        m.write_kv(0, cfg.max_seq, k_before[:1], k_before[:1])


def test_generate_tokens_semantics():
    # src/generate.rs:43-91: M = min(max_new, max_seq) steps pos = 0..M-2;
    # outputs are prompt[1..] then argmax picks, stopping before stop_on.
    cfg = oracle.LlamaConfig(**TINY)
    w = oracle.random_weights(cfg, seed=11, std=0.5)
    prompt = [3, 17, 4]
    toks, last = oracle.Model(cfg, dict(w)).generate_tokens(prompt, max_new_tokens=100)
    M = min(100, cfg.max_seq)
    assert len(toks) == M - 1
    assert list(toks[: len(prompt) - 1]) == prompt[1:]
    # teacher-forced replay: each generated token is the argmax after the
    # sequence that precedes it
    m = oracle.Model(cfg, dict(w))
    seq = [prompt[0]] + list(toks)
    for pos in range(M - 1):
        logits = m.step(seq[pos], pos)
        if pos >= len(prompt) - 1:
            assert toks[pos] == int(np.argmax(logits))
    np.testing.assert_array_equal(last, logits)
    # stop_on: generation halts before pushing the stop token
    stop = int(toks[len(prompt)])
    toks2, _ = oracle.Model(cfg, dict(w)).generate_tokens(prompt, 100, stop_on=stop)
    assert list(toks2) == list(toks[: list(toks).index(stop)])
    # a one-token budget runs no step; an empty prompt is an error
    assert len(oracle.Model(cfg, dict(w)).generate_tokens(prompt, 1)[0]) == 0
    with pytest.raises(ValueError):
        oracle.Model(cfg, dict(w)).generate_tokens([], 5)
