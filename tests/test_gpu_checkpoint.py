"""GPU tests of llama2.c checkpoint loading: a model built from a loaded
checkpoint must give the same logits, bit for bit, as the model built from
the arrays the checkpoint was written from (fp32, or bf16 rounded to
nearest even on both sides), for both layouts and classifier kinds; the C1
golden generation runs from a checkpoint file."""
import json
import os

import numpy as np
import pytest

import oracle
from ammon_amd import AmmonError, LlamaModel
from ammon_amd._abi import BF16, F32
from oracle import llama2c

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))

CFG = oracle.LlamaConfig(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, hidden=520, vocab=611,
                         max_seq=40, theta=10000.0, w_dtype=F32, kv_dtype=F32)


@pytest.mark.parametrize("version", [0, 1])
@pytest.mark.parametrize("shared", [False, True])
@pytest.mark.parametrize("w_dtype", [F32, BF16])
def test_checkpoint_model_equals_direct_model(rt, tmp_path, version, shared, w_dtype):
    w = oracle.random_weights(CFG, seed=21, std=0.05)
    for i, name in enumerate(("rms_att", "rms_ffn", "rms_final")):
        w[name] = (1.0 + 0.1 * oracle.normal(w[name].size, 22, stream=i)).reshape(w[name].shape)
    if shared:
        w["wcls"] = w["tok_emb"].copy()
    path = tmp_path / "m.bin"
    llama2c.write(path, CFG, w, version=version, shared=shared)
    loaded = LlamaModel.from_checkpoint(rt, str(path), w_dtype=w_dtype)
    direct_w = {k: (v if k.startswith("rms") else oracle.storage(v, w_dtype)) for k, v in w.items()}
    cfg = oracle.LlamaConfig(**{**CFG.__dict__, "w_dtype": w_dtype})
    direct = LlamaModel.from_host(rt, cfg, direct_w)
    for pos, tok in enumerate([1, 610, 37, 37, 5]):
        np.testing.assert_array_equal(loaded.step(tok, pos), direct.step(tok, pos))
    loaded.close()
    direct.close()


def test_checkpoint_size_mismatch_is_rejected(rt, tmp_path):
    w = oracle.random_weights(CFG, seed=23)
    path = tmp_path / "m.bin"
    llama2c.write(path, CFG, w, version=0)
    with open(path, "ab") as f:
        f.write(b"\0" * 8)
    with pytest.raises(AmmonError, match="header's shape needs"):
        LlamaModel.from_checkpoint(rt, str(path))


def test_c1_generation_from_a_checkpoint_file(rt, tmp_path):
    f = np.load(os.path.join(HERE, "golden", "c1_greedy.npz"))
    cfg = oracle.LlamaConfig(**json.loads(str(f["config"])))
    weights = oracle.random_weights(cfg, seed=int(f["weight_seed"]), std=0.02)
    path = tmp_path / "c1.bin"
    llama2c.write(path, cfg, weights, version=0, shared=False)
    m = LlamaModel.from_checkpoint(rt, str(path))
    toks, logits, _ = m.generate_tokens_device(f["prompt"], int(f["max_new_tokens"]))
    np.testing.assert_array_equal(toks, f["tokens"])
    m.close()
