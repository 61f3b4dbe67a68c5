import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "qwen38-flash.cpp_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libq38.so on cuda:0)")
    config.addinivalue_line("markers", "slow: full-size parity case")
    # torch carries its own HIP runtime. Importing torch before libq38.so is loaded makes the
    # library bind to that runtime (same soname), so the process has one HIP runtime
    # whichever test runs first.
    import torch  # noqa: F401
    if os.path.exists(os.path.join(PKG, "libq38.so")):
        import q38  # noqa: F401


@pytest.fixture(scope="session")
def orc():
    import oracle_lib
    return oracle_lib.load()


@pytest.fixture(scope="session")
def q38():
    import q38 as mod
    return mod


@pytest.fixture(scope="session")
def gpu():
    """torch on cuda:0 plus a q38 context; skips nothing: a gpu-marked test without a GPU fails."""
    import torch
    import q38 as mod
    assert torch.cuda.is_available(), "gpu tests need a HIP device"
    ctx = mod.Ctx(0)
    yield ctx
    ctx.close()
