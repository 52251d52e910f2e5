"""CPU tests of bench.py's contract pieces that need no GPU: the one-GPU
guard and the byte accounting behind `value` and `roofline`."""
import os
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_token_and_kernel_bytes_at_llama3_8b():
    c = bench.Cfg(**bench.LLAMA3_8B)
    # 32 x (wq 4096^2 + wk/wv 2 x 1024 x 4096 + wo 4096^2 + w1/w3/w2 3 x 14336 x 4096)
    # + LM head 128256 x 4096, bf16; K and V of 8 x 128 at 8192 positions, bf16
    weights = 2 * (32 * (4096 * 4096 + 2 * 1024 * 4096 + 4096 * 4096 + 3 * 14336 * 4096)
                   + 128256 * 4096)
    assert bench.token_bytes(c, 8192) == weights + 32 * 2 * 8192 * 1024 * 2
    kb = bench.kernel_bytes(c, 8192)
    assert kb["gate_up_swiglu"] == 234971136
    assert kb["lm_head"] == 128256 * 4096 * 2 + 4 * 4096 * 2 + 4 * 128256
    # every layer GEMV's weights are counted once across the per-kernel table
    gemv_w = sum(kb[k] for k in ("qkv_rope_store", "wo_residual", "gate_up_swiglu", "w2_residual"))
    assert 0 <= gemv_w - 2 * (4096 * 4096 + 2 * 1024 * 4096 + 4096 * 4096 + 3 * 14336 * 4096) < 1 << 20
