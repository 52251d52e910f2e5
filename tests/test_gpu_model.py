"""End-to-end GPU tests of the C++ host layer's model (modules + launch
sequence + greedy loop) against the oracle: greedy token sequences identical;
logits and KV caches within 1e-5 relative (normwise) with an fp32 KV cache
(fp32 or identical bf16 weights); within 1e-3 with a bf16 KV cache and the
same weights on both sides, where the fp32 K/V before the store differ only
by summation order (~4e-6 relative) and so flip about two bf16 roundings per
1024-element row, each by one bf16 ulp (at most 2^-7 of the element), which
moves a row by ~3.5e-4 normwise; and within 2e-2 -- the bf16-weight bar --
of the unrounded fp32 model for bf16 weights."""
import json
import os

import numpy as np
import pytest

import oracle
from ammon_amd import AmmonError, LlamaModel, _abi
from ammon_amd._abi import BF16, F32

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
RTOL = 1e-5
BF16_KV_TOL = 1e-3  # same weights, bf16 KV cache (rounding flips of new K/V elements)
BF16_W_TOL = 2e-2   # bf16 weights against the unrounded fp32 model


def tol(kv_dtype):
    return RTOL if kv_dtype == F32 else BF16_KV_TOL


def attention_launches(rt, cfg, split=0):
    """The decode attention pair's launches: one where a single split covers
    the cache (pass 1 writes the output), else two."""
    split = split or int(_abi.lib.ammon_attention_default_split_for(
        rt.handle, cfg.n_heads, cfg.n_kv_heads, cfg.dim // cfg.n_heads, cfg.kv_dtype,
        cfg.max_seq))
    return 1 if int(_abi.lib.ammon_attention_splits(cfg.max_seq, split)) == 1 else 2


def layer_launches(rt, cfg, split=0):
    """Launches one layer records: norm+QKV, attention, Wo, gate/up, W2."""
    return 4 + attention_launches(rt, cfg, split)


def block_launches(rt, cfg, split=0):
    """Launches one layer records with one_launch_blocks: one per attention
    / SwiGLU block where one launch applies (bf16 weights; the attention
    block also a bf16 KV cache, head 128 and 1-4 q heads per kv head), else
    the separate launches."""
    head = cfg.dim // cfg.n_heads
    g = cfg.n_heads // cfg.n_kv_heads
    one_attn = cfg.w_dtype == BF16 and cfg.kv_dtype == BF16 and head == 128 and g in (1, 2, 4)
    one_ffn = cfg.w_dtype == BF16
    attn = 1 if one_attn else 2 + attention_launches(rt, cfg, split)
    return attn + (1 if one_ffn else 2)


def rel_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


@pytest.fixture(scope="module")
def c1():
    f = np.load(os.path.join(HERE, "golden", "c1_greedy.npz"))
    cfg = oracle.LlamaConfig(**json.loads(str(f["config"])))
    weights = oracle.random_weights(cfg, seed=int(f["weight_seed"]), std=0.02)
    return cfg, weights, f


def test_c1_greedy_tokens_match_fixture(rt, c1):
    cfg, weights, f = c1
    m = LlamaModel.from_host(rt, cfg, weights)
    toks, logits, tps = m.generate_tokens(f["prompt"], int(f["max_new_tokens"]))
    np.testing.assert_array_equal(toks, f["tokens"])
    assert rel_err(logits, f["logits"]) <= RTOL
    assert tps > 0
    m.close()


def test_c1_device_greedy_matches_fixture(rt, c1):
    cfg, weights, f = c1
    m = LlamaModel.from_host(rt, cfg, weights)
    toks, logits, tps = m.generate_tokens_device(f["prompt"], int(f["max_new_tokens"]))
    np.testing.assert_array_equal(toks, f["tokens"])
    assert rel_err(logits, f["logits"]) <= RTOL
    assert tps > 0
    m.close()


def test_c1_kv_cache_matches_oracle(rt, c1):
    cfg, weights, f = c1
    m = LlamaModel.from_host(rt, cfg, weights)
    m.generate_tokens_device(f["prompt"], int(f["max_new_tokens"]))
    om = oracle.Model(cfg, dict(weights))
    om.generate_tokens(f["prompt"], int(f["max_new_tokens"]))
    for layer in range(cfg.n_layers):
        k, v = m.kv_layer(layer)
        ok, ov = om.kv_layer(layer)
        assert rel_err(k, ok) <= RTOL, layer
        assert rel_err(v, ov) <= RTOL, layer
    m.close()


def test_graph_replay_equals_eager_launches(rt, c1):
    cfg, weights, f = c1
    dev = {k: rt.upload(np.ascontiguousarray(v)) for k, v in weights.items()}
    graph = LlamaModel(rt, cfg, dev, use_graph=True)
    eager = LlamaModel(rt, cfg, dev, use_graph=False)
    for pos, tok in enumerate(f["prompt"][:5]):
        np.testing.assert_array_equal(graph.step(int(tok), pos), eager.step(int(tok), pos))
    graph.close()
    eager.close()


@pytest.mark.parametrize("stop_index", [3, 12])
def test_stop_on_truncates_like_the_reference(rt, c1, stop_index):
    cfg, weights, f = c1
    stop = int(f["tokens"][stop_index])
    want = list(f["tokens"][: list(f["tokens"]).index(stop)])
    m = LlamaModel.from_host(rt, cfg, weights)
    assert list(m.generate_tokens(f["prompt"], 256, stop_on=stop)[0]) == want
    assert list(m.generate_tokens_device(f["prompt"], 256, stop_on=stop)[0]) == want
    m.close()


GQA = dict(dim=256, n_layers=3, n_heads=8, n_kv_heads=2, hidden=704, vocab=4099, max_seq=96,
           theta=500000.0)


@pytest.mark.parametrize("kv_dtype", [F32, BF16])
def test_gqa_bf16_weights_match_oracle(rt, kv_dtype):
    cfg = oracle.LlamaConfig(**GQA, w_dtype=BF16, kv_dtype=kv_dtype)
    weights = oracle.random_weights(cfg, seed=77, std=0.1)
    prompt = [5, 4000, 17, 2048, 3]
    m = LlamaModel.from_host(rt, cfg, weights)
    toks, logits, _ = m.generate_tokens_device(prompt, cfg.max_seq)
    want_toks, want_logits = oracle.Model(cfg, dict(weights)).generate_tokens(prompt, cfg.max_seq)
    np.testing.assert_array_equal(toks, want_toks)
    assert rel_err(logits, want_logits) <= tol(kv_dtype)
    # bf16 weights against the unrounded fp32 model: per-step logits
    cfg32 = oracle.LlamaConfig(**GQA, w_dtype=F32, kv_dtype=F32)
    w32 = oracle.random_weights(cfg32, seed=77, std=0.1)
    m32 = oracle.Model(cfg32, w32)
    m.close()
    m = LlamaModel.from_host(rt, cfg, weights)
    for pos, tok in enumerate(prompt):
        assert rel_err(m.step(tok, pos), m32.step(tok, pos)) <= BF16_W_TOL
    m.close()


@pytest.mark.parametrize("kv_dtype", [F32, BF16])
def test_llama3_8b_width_two_layers(rt, kv_dtype):
    # Full Llama-3-8B layer width and vocab, two layers, bf16 weights.
    cfg = oracle.LlamaConfig(dim=4096, n_layers=2, n_heads=32, n_kv_heads=8, hidden=14336,
                             vocab=128256, max_seq=64, theta=500000.0, w_dtype=BF16,
                             kv_dtype=kv_dtype)
    weights = oracle.random_weights(cfg, seed=4, std=0.02)
    prompt = [128000, 9906, 1917, 374]
    m = LlamaModel.from_host(rt, cfg, weights)
    toks, logits, _ = m.generate_tokens_device(prompt, 9)
    want_toks, want_logits = oracle.Model(cfg, dict(weights)).generate_tokens(prompt, 9)
    np.testing.assert_array_equal(toks, want_toks)
    assert rel_err(logits, want_logits) <= tol(kv_dtype)
    assert m.launches == 1 + layer_launches(rt, cfg) * cfg.n_layers + 1
    m.close()


def test_model_validation(rt, c1):
    cfg, weights, f = c1
    m = LlamaModel.from_host(rt, cfg, weights)
    with pytest.raises(AmmonError, match="vocab"):
        m.step(cfg.vocab, 0)
    with pytest.raises(AmmonError, match="max_seq"):
        m.step(1, cfg.max_seq)
    with pytest.raises(AmmonError, match="max_seq"):
        m.decode(1, cfg.max_seq - 2, 5)
    with pytest.raises(AmmonError, match="prompt"):
        m.generate_tokens([], 5)
    m.close()
    bad = oracle.LlamaConfig(**dict(json.loads(str(f["config"])), n_heads=7))
    with pytest.raises(AmmonError, match="divisible"):
        LlamaModel(rt, bad, m.weights)


# Persistent decode-token kernel: one cooperative launch per token must give
# the launch list's results bit for bit (same per-row and per-unit arithmetic).
PERSISTENT_SHAPES = [  # (n_heads, n_kv_heads): q heads per kv head 4, 1, 2, 8
    (32, 8), (8, 8), (16, 8), (32, 4)]


@pytest.mark.parametrize("kv_dtype", [BF16, F32])
def test_persistent_token_kernel_single_split_matches_launch_list(rt, kv_dtype):
    # A 192-position cache takes the library's single split: the launch list
    # runs pass 1 alone (acc / l), the persistent kernel its partial + merge
    # phases -- bit-identical, as the merge of one split is acc / l exactly.
    cfg = oracle.LlamaConfig(dim=4096, n_layers=2, n_heads=32, n_kv_heads=8, hidden=1544,
                             vocab=5003, max_seq=192, theta=500000.0, w_dtype=BF16,
                             kv_dtype=kv_dtype)
    ref = LlamaModel.synthetic(rt, cfg, seed=35, std=0.05)
    rt.synchronize()
    fused = LlamaModel(rt, cfg, ref.weights, persistent=True)
    assert fused.launches == 1
    assert ref.launches == 1 + 5 * cfg.n_layers + 1
    for pos, tok in enumerate([7, 4093, 12, 5002, 300, 1]):
        np.testing.assert_array_equal(fused.step(tok, pos), ref.step(tok, pos))
    got = fused.decode(11, cfg.max_seq - 8, 8, read_tokens=True)
    want = ref.decode(11, cfg.max_seq - 8, 8, read_tokens=True)
    np.testing.assert_array_equal(got, want)
    fused.close()
    ref.close()


@pytest.mark.parametrize("kv_dtype", [BF16, F32])
@pytest.mark.parametrize("heads", PERSISTENT_SHAPES)
def test_persistent_token_kernel_matches_launch_list(rt, heads, kv_dtype):
    n_heads, n_kv = heads
    cfg = oracle.LlamaConfig(dim=128 * n_heads, n_layers=2, n_heads=n_heads, n_kv_heads=n_kv,
                             hidden=1544, vocab=5003, max_seq=300, theta=500000.0,
                             w_dtype=BF16, kv_dtype=kv_dtype)
    # the same split for both, so they merge the same partials in the same order
    ref = LlamaModel.synthetic(rt, cfg, seed=31, std=0.05, split_len=32)
    for i, name in enumerate(("rms_att", "rms_ffn", "rms_final")):
        n = cfg.dim * (cfg.n_layers if name != "rms_final" else 1)
        rt.fill_normal(ref.weights[name], F32, n, 32, i, 1.0, 0.2)
    rt.synchronize()
    fused = LlamaModel(rt, cfg, ref.weights, persistent=True, split_len=32)
    assert fused.launches == 1
    assert ref.launches == 1 + layer_launches(rt, cfg, 32) * cfg.n_layers + 1
    prompt = [7, 4093, 12, 5002, 300, 1]
    for pos, tok in enumerate(prompt):
        np.testing.assert_array_equal(fused.step(tok, pos), ref.step(tok, pos))
    for l in range(cfg.n_layers):
        for got, want in zip(fused.kv_layer(l), ref.kv_layer(l)):
            np.testing.assert_array_equal(got, want)
    # greedy generation past several attention splits, device loop
    toks_f, logits_f, _ = fused.generate_tokens_device(prompt, 40)
    toks_r, logits_r, _ = ref.generate_tokens_device(prompt, 40)
    np.testing.assert_array_equal(toks_f, toks_r)
    np.testing.assert_array_equal(logits_f, logits_r)
    # decode from a late position (splits up to the cache end)
    got = fused.decode(11, cfg.max_seq - 20, 20, read_tokens=True)
    want = ref.decode(11, cfg.max_seq - 20, 20, read_tokens=True)
    np.testing.assert_array_equal(got, want)
    fused.close()
    ref.close()


def test_persistent_barrier_timeout_is_reported(rt, monkeypatch):
    # A one-poll limit on the kernel's bounded barrier wait: the waits give up
    # at once (nothing hangs, every access stays in bounds), the kernel marks
    # the timeout, and the host turns it into an error instead of results.
    cfg = oracle.LlamaConfig(dim=256, n_layers=2, n_heads=2, n_kv_heads=1, hidden=512,
                             vocab=300, max_seq=64, theta=500000.0, w_dtype=BF16, kv_dtype=BF16)
    ref = LlamaModel.synthetic(rt, cfg, seed=5, std=0.05)
    monkeypatch.setenv("AMMON_TOKEN_SPIN_LIMIT", "1")
    fused = LlamaModel(rt, cfg, ref.weights, persistent=True)
    monkeypatch.delenv("AMMON_TOKEN_SPIN_LIMIT")
    assert fused.launches == 1
    with pytest.raises(AmmonError, match="grid barrier timed out"):
        for pos in range(8):  # a timeout is certain within a few tokens
            fused.step(1, pos)
    fused.close()
    # a model built without the override is unaffected
    fused = LlamaModel(rt, cfg, ref.weights, persistent=True)
    np.testing.assert_array_equal(fused.step(3, 0), ref.step(3, 0))
    fused.close()
    ref.close()


def test_persistent_token_trace(rt, monkeypatch):
    # Barrier stamps: every workgroup arrives at each barrier before its wait
    # ends, no wait ends before the last arrival, and the phases are ordered.
    cfg = oracle.LlamaConfig(dim=256, n_layers=3, n_heads=2, n_kv_heads=1, hidden=512,
                             vocab=300, max_seq=64, theta=500000.0, w_dtype=BF16, kv_dtype=BF16)
    ref = LlamaModel.synthetic(rt, cfg, seed=6, std=0.05)
    assert ref.token_trace() is None  # launch list: nothing to trace
    monkeypatch.setenv("AMMON_TOKEN_TRACE", "1")
    fused = LlamaModel(rt, cfg, ref.weights, persistent=True)
    monkeypatch.delenv("AMMON_TOKEN_TRACE")
    toks = fused.decode(5, 0, 3, read_tokens=True)  # greedy: every barrier runs
    np.testing.assert_array_equal(toks, ref.decode(5, 0, 3, read_tokens=True))
    t = fused.token_trace().astype(np.int64)
    assert t.shape[0] == 6 * cfg.n_layers + 3 and t.shape[2] >= rt.info.compute_units
    arrive, leave = t[:, 0, :], t[:, 1, :]
    last = t.shape[0] - 1  # only workgroup 0 waits at the final barrier
    assert (arrive > 0).all() and (leave[:last] > 0).all() and leave[last, 0] > 0
    assert (leave[:last] >= arrive[:last].max(axis=1, keepdims=True)).all()
    assert (arrive[1:] >= leave[:-1].min(axis=1, keepdims=True)).all()
    fused.close()
    ref.close()



# One launch per attention / SwiGLU block (ammon_attention_block,
# ammon_swiglu_block): the same per-row and per-unit arithmetic as the
# separate launches, so logits, caches and tokens must be bit-identical.
ONE_LAUNCH_SHAPES = [  # (n_heads, n_kv_heads, kv dtype, max_seq, split)
    (32, 8, BF16, 300, 32),    # 4 q heads per kv head (Llama-3)
    (8, 8, BF16, 300, 32),     # 1
    (16, 8, BF16, 300, 0),     # 2, the library's split
    (32, 8, F32, 300, 32),     # fp32 cache: separate attention launches, one SwiGLU launch
    (32, 4, BF16, 300, 32),    # 8: separate attention launches
    (32, 8, BF16, 8192, 64),   # more attention units (1024) than workgroups
    (32, 8, BF16, 200, 0),     # one split: the launch list's attention is one launch
    (32, 8, F32, 200, 0),      # one split, fp32 cache: the same one launch on both sides
]


@pytest.mark.parametrize("shape", ONE_LAUNCH_SHAPES)
def test_one_launch_blocks_match_launch_list(rt, shape):
    n_heads, n_kv, kv_dtype, max_seq, split = shape
    print(f"one-launch blocks: shape {shape}", flush=True)
    cfg = oracle.LlamaConfig(dim=128 * n_heads, n_layers=2, n_heads=n_heads, n_kv_heads=n_kv,
                             hidden=1544, vocab=5003, max_seq=max_seq, theta=500000.0,
                             w_dtype=BF16, kv_dtype=kv_dtype)
    ref = LlamaModel.synthetic(rt, cfg, seed=33, std=0.05, split_len=split)
    for i, name in enumerate(("rms_att", "rms_ffn", "rms_final")):
        n = cfg.dim * (cfg.n_layers if name != "rms_final" else 1)
        rt.fill_normal(ref.weights[name], F32, n, 34, i, 1.0, 0.2)
    rt.synchronize()
    one = LlamaModel(rt, cfg, ref.weights, split_len=split, one_launch_blocks=True)
    assert ref.launches == 1 + layer_launches(rt, cfg, split) * cfg.n_layers + 1
    assert one.launches == 1 + block_launches(rt, cfg, split) * cfg.n_layers + 1
    prompt = [7, 4093, 12, 5002, 300, 1]
    for pos, tok in enumerate(prompt):
        np.testing.assert_array_equal(one.step(tok, pos), ref.step(tok, pos))
    for l in range(cfg.n_layers):
        for got, want in zip(one.kv_layer(l), ref.kv_layer(l)):
            np.testing.assert_array_equal(got, want)
    # greedy generation through several splits, device loop (graph replay)
    toks_o, logits_o, _ = one.generate_tokens_device(prompt, 40)
    toks_r, logits_r, _ = ref.generate_tokens_device(prompt, 40)
    np.testing.assert_array_equal(toks_o, toks_r)
    np.testing.assert_array_equal(logits_o, logits_r)
    # decode at the end of the cache (every split live)
    got = one.decode(11, cfg.max_seq - 20, 20, read_tokens=True)
    want = ref.decode(11, cfg.max_seq - 20, 20, read_tokens=True)
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(one.step(5, cfg.max_seq - 1), ref.step(5, cfg.max_seq - 1))
    one.close()
    ref.close()


def test_one_launch_block_barrier_timeout_is_reported(rt, monkeypatch):
    # A one-poll limit on the blocks' bounded barrier waits: the waits give
    # up at once (nothing hangs, every access stays in bounds), the launch is
    # flagged, and the host turns the flag into an error instead of results.
    cfg = oracle.LlamaConfig(dim=512, n_layers=2, n_heads=4, n_kv_heads=1, hidden=1024,
                             vocab=300, max_seq=64, theta=500000.0, w_dtype=BF16, kv_dtype=BF16)
    ref = LlamaModel.synthetic(rt, cfg, seed=8, std=0.05)
    monkeypatch.setenv("AMMON_BLOCK_SPIN_LIMIT", "1")
    one = LlamaModel(rt, cfg, ref.weights, one_launch_blocks=True)
    assert one.launches == 1 + 2 * cfg.n_layers + 1
    with pytest.raises(AmmonError, match="grid barrier of a one-launch block timed out"):
        for pos in range(8):  # a timeout is certain within a few tokens
            one.step(1, pos)
    monkeypatch.delenv("AMMON_BLOCK_SPIN_LIMIT")
    one.close()
    # a model built without the override is unaffected
    one = LlamaModel(rt, cfg, ref.weights, one_launch_blocks=True)
    np.testing.assert_array_equal(one.step(3, 0), ref.step(3, 0))
    one.close()
    ref.close()
