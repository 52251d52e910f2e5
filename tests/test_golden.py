"""The committed C1 fixture is reproduced exactly by the oracle (the oracle
is deterministic: OpenMP splits only independent outputs)."""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_c1_fixture  # noqa: E402


def test_c1_fixture_is_reproduced_by_the_oracle():
    f = np.load(os.path.join(HERE, "golden", "c1_greedy.npz"))
    assert json.loads(str(f["config"])) == make_c1_fixture.C1
    cfg, prompt, tokens, logits = make_c1_fixture.run()
    np.testing.assert_array_equal(prompt, f["prompt"])
    np.testing.assert_array_equal(tokens, f["tokens"])
    np.testing.assert_array_equal(logits, f["logits"])
    # reference src/generate.rs semantics at this config: 255 steps, the 7
    # forced prompt tokens then 248 generated ones
    assert len(tokens) == 255
    np.testing.assert_array_equal(tokens[:7], prompt[1:])
    assert np.all((prompt >= 1) & (prompt < 32000))


def test_c4_bf16kv_drift_fixture_states_what_the_gpu_test_relies_on():
    """The drift study (oracle against itself, one GEMV summation order
    changed) with a bf16 cache drifts ~100x more than with an fp32 cache and
    flips a greedy pick; with an fp32 cache it does not within the fixture's
    527 steps."""
    import make_bf16kv_drift
    f = np.load(os.path.join(HERE, "golden", "c4_bf16kv_drift.npz"))
    assert json.loads(str(f["config"])) == make_bf16kv_drift.C4
    prompt = make_bf16kv_drift.prompt_tokens()
    np.testing.assert_array_equal(prompt, f["prompt"])
    for kv in ("bf16", "f32"):
        ta, tb, first = f[f"{kv}_tokens_a"], f[f"{kv}_tokens_b"], int(f[f"{kv}_first_divergent"])
        np.testing.assert_array_equal(ta[:15], prompt[1:])
        agree = len(ta) if first < 0 else first
        np.testing.assert_array_equal(ta[:agree], tb[:agree])
        if first >= 0:
            assert first == len(ta) - 1 and ta[first] != tb[first]
            # the flipped pick is one of the few steps with a tiny top-2 margin
            m = f[f"{kv}_margins_a"]
            assert m[first] < np.percentile(m, 5)
    assert int(f["bf16_first_divergent"]) == 358
    assert int(f["f32_first_divergent"]) == -1 and len(f["f32_tokens_a"]) == 527
    bf, fp = f["bf16_drift"], f["f32_drift"]
    assert np.median(bf) > 30 * np.median(fp)
    assert bf[0] > 1e-3 and fp.max() < 1e-4


def test_c4_fixture_is_the_drift_study_fp32_run():
    """The C4 fixture (oracle, fp32 cache, seed-1004 prompt) and the drift
    study's run A with the fp32 cache are the same decode, written by two
    scripts: same prompt, same 527 tokens, same top-2 margins."""
    f = np.load(os.path.join(HERE, "golden", "c4_greedy.npz"))
    g = np.load(os.path.join(HERE, "golden", "c4_bf16kv_drift.npz"))
    assert json.loads(str(f["config"])) == json.loads(str(g["config"]))
    assert int(f["weight_seed"]) == int(g["weight_seed"])
    np.testing.assert_array_equal(f["prompt"], g["prompt"])
    np.testing.assert_array_equal(f["tokens"], g["f32_tokens_a"])
    np.testing.assert_array_equal(f["margins"], g["f32_margins_a"])
    # the largest |logit| per step is the scale of the 1e-4 normwise bar
    assert f["scales"].shape == f["margins"].shape and np.all(f["scales"] > 0)
