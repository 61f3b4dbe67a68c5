"""Engine-side MTP round policy and the batched multi-slot round driver
(qwen38-flash.cpp_amd/host/qwen38_policy.hpp, qwen38_engine.hpp) through the CPU test program
tests/cpp/policy_test.cpp: the reference's known answers (tests/mtp_depth_policy_test.cpp,
tests/history_draft_test.cpp), random call sequences compared call by call with the reference's
own sources compiled into oracle/_ref, and scheduler invariants over an exact fake verifier."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "qwen38-flash.cpp_amd", "_build", "policy_test")
REF = os.path.join(ROOT, "oracle", "_ref", "libq38_ref.so")


def run(*args):
    assert os.path.exists(BIN), "policy_test is not built (make -C qwen38-flash.cpp_amd)"
    p = subprocess.run([BIN, *args], capture_output=True, text=True, timeout=300)
    assert p.returncode == 0, p.stdout + p.stderr
    return p.stdout


def test_policy_and_scheduler():
    out = run(REF) if os.path.exists(REF) else run()
    assert "0 failures" in out, out


def test_policy_matches_compiled_reference():
    """The differential part runs whenever the reference checkout was there to build oracle/_ref."""
    if not os.path.exists(REF):
        assert not os.path.exists("/root/reference/src/mtp_depth_policy.cpp"), "oracle/_ref was not built"
        return
    out = run(REF)
    assert "random cases against the reference's compiled policy" in out, out
