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
