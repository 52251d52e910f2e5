"""The Llama-3-8B-shaped greedy decode as configured, against the oracle:
32 layers, dim 4096, 32 q / 8 kv heads of 128, SwiGLU hidden 14336, vocab
128256, RoPE theta 500000, bf16 weights N(0, 0.02), a KV cache sized 8192 in
fp32 (the reference's storage, src/modules.rs:53-54: greedy tokens are
compared bit for bit in fp32), a seeded 16-token prompt and max_new_tokens
528 -- 527 steps, 15 forced prompt tokens then 512 greedy picks (reference
src/generate.rs:43-91).

The expected tokens come from tests/golden/c4_greedy.npz, written once by
tests/golden/make_c4_fixture.py through the oracle on host-generated
weights.  Here the same weights are generated on the device by the same
seeded generator; every tensor's storage checksums must equal the fixture's
before any token is compared, so the comparison is between identical
models.  The greedy tokens must be identical; on a mismatch the message
names the first differing step and the oracle's top-2 logit margin there,
so a near tie can be told apart from a bug.  The last step's logits: the
two sides differ only in fp32 summation order (~4e-6 relative per
projection), compounded over 32 layers and 527 steps of cache: within 1e-4
normwise relative.  The same holds for the device and the host loop.
"""
import json
import os
import time

import numpy as np
import pytest

from ammon_amd import LlamaModel
from ammon_amd._abi import call
from ammon_amd.model import weight_shapes

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "c4_greedy.npz")
DEEP_FP32_TOL = 1e-4


class Cfg:
    def __init__(self, **kw):
        self.__dict__.update(kw)


def rel_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


def checksum(rt, buf, nbytes):
    """(wrapping sum, xor) of a device buffer's little-endian uint64 words,
    computed on the device (ammon_checksum)."""
    out = rt.alloc(16)
    call("ammon_checksum", rt.handle, None, buf, nbytes, out)
    s, x = out.download(2, np.uint64)
    return int(s), int(x)


@pytest.fixture(scope="module")
def c4(rt):
    f = np.load(FIXTURE)
    c = json.loads(str(f["config"]))
    cfg = Cfg(**c, w_dtype=int(f["w_dtype"]), kv_dtype=int(f["kv_dtype"]))
    t0 = time.time()
    model = LlamaModel.synthetic(rt, cfg, seed=int(f["weight_seed"]), std=0.02)
    print(f"c4: device weights in {time.time() - t0:.1f} s", flush=True)
    want = json.loads(str(f["checksums"]))
    for name, shape in weight_shapes(cfg).items():
        nbytes = int(np.prod(shape)) * (4 if name.startswith("rms") else 2)
        got = checksum(rt, model.weights[name], nbytes)
        assert got == tuple(int(v) for v in want[name]), \
            f"device weights {name} differ from the oracle's: {got} vs {want[name]}"
    print(f"c4: all weight checksums equal the fixture's ({time.time() - t0:.1f} s)", flush=True)
    yield model, f
    model.close()


def check_tokens(got, f):
    want = f["tokens"]
    margins = f["margins"]
    prompt_len = len(f["prompt"])
    gen = margins[prompt_len - 1:]
    print(f"c4: smallest top-2 margin over the generated steps {float(gen.min()):.3e} "
          f"(step {prompt_len - 1 + int(gen.argmin())})", flush=True)
    assert len(got) == len(want) == 527
    bad = np.nonzero(np.asarray(got) != want)[0]
    if bad.size:
        i = int(bad[0])
        raise AssertionError(
            f"first differing step {i} (position {i}): got {int(got[i])}, oracle {int(want[i])} "
            f"(oracle runner-up {int(f['runners'][i])}, top-2 margin {float(margins[i]):.3e}); "
            f"{bad.size} steps differ")


def test_c4_device_greedy_tokens_match_oracle(c4):
    model, f = c4
    t0 = time.time()
    toks, logits, tps = model.generate_tokens_device(f["prompt"], int(f["max_new_tokens"]))
    print(f"c4 device loop: {len(toks)} tokens in {time.time() - t0:.1f} s ({tps:.1f} tok/s)",
          flush=True)
    check_tokens(toks, f)
    err = rel_err(logits, f["logits"])
    print(f"c4 device loop: last-step logits rel err {err:.2e}", flush=True)
    assert err <= DEEP_FP32_TOL


def test_c4_host_greedy_tokens_match_oracle(c4):
    model, f = c4
    t0 = time.time()
    toks, logits, tps = model.generate_tokens(f["prompt"], int(f["max_new_tokens"]))
    print(f"c4 host loop: {len(toks)} tokens in {time.time() - t0:.1f} s ({tps:.1f} tok/s)",
          flush=True)
    check_tokens(toks, f)
    err = rel_err(logits, f["logits"])
    print(f"c4 host loop: last-step logits rel err {err:.2e}", flush=True)
    assert err <= DEEP_FP32_TOL
