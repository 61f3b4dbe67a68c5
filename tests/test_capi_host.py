"""The C ABI library loads on a host without a GPU and exports every entry point that
include/q38.h declares (no compute calls)."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "q38.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(q38_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "q38_moe_forward" in names and "q38_head_greedy" in names and len(names) > 30


def test_every_declared_symbol_is_exported(q38):
    missing = [n for n in declared_symbols() if not hasattr(q38.lib, n)]
    assert not missing, missing


def test_version_and_error_strings(q38):
    assert q38.lib.q38_version().startswith(b"q38")
    out = C.c_void_p()
    assert q38.lib.q38_ctx_create(0, None) == q38.Q38_EINVAL
    assert b"null" in q38.lib.q38_last_error()


def test_workspace_sizes(q38):
    d = q38.desc()
    ws1 = q38.lib.q38_moe_workspace_size(C.byref(d), 1)
    ws4 = q38.lib.q38_moe_workspace_size(C.byref(d), 4)
    assert 0 < ws1 < ws4
    ws512 = q38.lib.q38_moe_workspace_size(C.byref(d), 512)
    assert ws4 < q38.lib.q38_moe_workspace_size(C.byref(d), 17) < ws512   # prefill widths
    assert q38.lib.q38_moe_workspace_size(C.byref(d), 2049) == 0
