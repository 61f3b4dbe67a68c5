"""q38_moe_forward_static (the allocation-free forward) against q38_moe_forward: the same
kernels on the library's fixed per-GPU scratch instead of a caller workspace, so outputs,
routes and plans are bit-identical; two calls in a row, the second with fewer rows (the
scratch keeps the first call's contents); sizes beyond the scratch are rejected."""
import ctypes as C

import numpy as np
import pytest

import gpu_util as G
from moe_cases import SEED

pytestmark = pytest.mark.gpu


def forward(q38, L, d, x_np, static):
    M = x_np.shape[0]
    x = G.to_dev(x_np)
    y = G.empty(x_np.shape, np.uint16)
    MK = M * d.top_k
    ex, wt, plan = G.empty(MK, np.int32), G.empty(MK, np.float32), G.empty(2 + 4 * MK, np.int32)
    r = q38.routes(ex, wt, None, plan)
    if static:
        q38.check(q38.lib.q38_moe_forward_static(L.h, x.data_ptr(), M, y.data_ptr(), C.byref(r), G.stream()))
    else:
        ws = G.workspace(q38.lib.q38_moe_workspace_size(C.byref(d), M))
        q38.check(q38.lib.q38_moe_forward(L.h, x.data_ptr(), M, y.data_ptr(), C.byref(r), ws.data_ptr(), ws.numel(),
                                          G.stream()))
    return [G.to_host(t) for t in (y, ex, wt, plan)]


@pytest.mark.parametrize("kind", ["uniform", "mixed"])
def test_static_forward_matches_workspace_forward(gpu, q38, orc, kind):
    d = q38.desc() if kind == "uniform" else q38.desc(mixed=1)
    L = q38.MoeLayer(gpu, d, seed=SEED, layer=5)
    try:
        for M in ((4, 1) if kind == "uniform" else (16, 3)):  # the second call is smaller
            x = orc.rmsnorm(orc.embed(SEED, list(range(60 + M, 60 + 2 * M)), 2048))
            a = forward(q38, L, d, x, static=True)
            b = forward(q38, L, d, x, static=False)
            for u, v in zip(a, b):
                assert np.array_equal(u, v), (kind, M)
    finally:
        L.close()


def test_static_forward_rejects_sizes(gpu, q38):
    d = q38.desc()
    L = q38.MoeLayer(gpu, d, seed=SEED, layer=6)
    try:
        x = G.empty((17, 2048), np.uint16)
        y = G.empty((17, 2048), np.uint16)
        for rows in (0, 17, 2048):
            assert q38.lib.q38_moe_forward_static(L.h, x.data_ptr(), rows, y.data_ptr(), None, G.stream()) == \
                q38.Q38_EINVAL
        assert q38.lib.q38_moe_forward_static(L.h, x.data_ptr(), 4, x.data_ptr(), None, G.stream()) == q38.Q38_EINVAL
    finally:
        L.close()
    # a layer whose workspace for 16 rows exceeds the fixed 8 MiB scratch (hidden 2560,
    # intermediate 640, top-16): 16 rows are rejected, 4 rows fit and match the workspace call
    d = q38.desc(hidden=2560, inter=640, top_k=16)
    assert q38.lib.q38_moe_workspace_size(C.byref(d), 16) > 8 << 20 >= q38.lib.q38_moe_workspace_size(C.byref(d), 4)
    L = q38.MoeLayer(gpu, d, seed=SEED, layer=7)
    try:
        x = G.empty((16, 2560), np.uint16)
        y = G.empty((16, 2560), np.uint16)
        assert q38.lib.q38_moe_forward_static(L.h, x.data_ptr(), 16, y.data_ptr(), None, G.stream()) == \
            q38.Q38_ESPACE
        assert b"scratch" in q38.lib.q38_last_error()
    finally:
        L.close()
