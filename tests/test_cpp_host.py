"""The C++20 host interface (qwen38-flash.cpp_amd/host/qwen38_verify.hpp) through its test
program tests/cpp/host_mirror_test.cpp, built with the library: host KATs and exception
types on the CPU, the device section (SparseMoe vs the C ABI, verify + commit lifecycle,
a greedy round, and the engine-side round driver with 3 requests sharing each batched
verification, every batch recomputed row by row in the same kernel family; the MTP draft head,
learned-draft rounds and the scheduler drafting with the head; the HyperConnection mixer,
the GatedDeltaNet and full-attention verify steps and the draft head on HC streams against
the C ABI) on the GPU."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "qwen38-flash.cpp_amd", "_build", "host_mirror_test")


def run(*args):
    assert os.path.exists(BIN), "host_mirror_test is not built (make -C qwen38-flash.cpp_amd)"
    p = subprocess.run([BIN, *args], capture_output=True, text=True, timeout=300)
    assert p.returncode == 0, p.stdout + p.stderr
    return p.stdout


def test_host_section():
    assert "host section: ok" in run()


@pytest.mark.gpu
def test_gpu_section():
    out = run("--gpu")
    assert "gpu section: ok" in out, out
    assert "batched slots: ok" in out, out
    assert "draft head: ok" in out, out
    assert "hyper connection: ok" in out, out
    assert "gated delta net: ok" in out, out
    assert "mtp streams: ok" in out, out
    assert "self attention: ok" in out, out
    assert "decoder layer: ok" in out, out
