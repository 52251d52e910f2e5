"""Runs the C++ test programs of tests/cpp (built by __graft_entry__.build()).

generate_test checks ammon::generate_tokens / sample_argmax on the host with
a scripted model; kernels_test restates the reference's tests/kernels.rs
against the C++ recorder tier on the device.
"""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "_bin")


def run(name):
    path = os.path.join(BIN, name)
    if not os.path.exists(path):
        pytest.fail(f"{path} is not built (run __graft_entry__.build())")
    r = subprocess.run([path], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failed" in r.stdout, r.stdout


def test_cpp_generate_loop():
    run("generate_test")


@pytest.mark.gpu
def test_cpp_kernel_recorders():
    run("kernels_test")
