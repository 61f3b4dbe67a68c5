"""The fused verify layer kernel (gate/up, down and combine in one launch; values cross
workgroups by agent-coherent stores and loads polled for a reset pattern) is deterministic:
repeated calls, replays of a captured HIP graph with eager work between them, a workspace
that starts out holding arbitrary bytes, and calls of other widths on the same workspace in
between all give the same bits."""
import ctypes as C

import numpy as np
import pytest

import gpu_util as G
from moe_cases import SEED

pytestmark = pytest.mark.gpu

N_LAYERS = 3


@pytest.fixture(scope="module")
def stack(gpu, q38):
    layers = [q38.MoeLayer(gpu, q38.desc(), seed=SEED, layer=l) for l in range(N_LAYERS)]
    yield layers
    for L in layers:
        L.close()


def chain(q38, layers, h, ws, M):
    arr = (C.c_void_p * len(layers))(*[L.h.value for L in layers])
    q38.check(q38.lib.q38_verify_chain(arr, len(layers), h.data_ptr(), M, C.c_float(1e-6), None, ws.data_ptr(),
                                       ws.numel(), G.stream()))


@pytest.mark.parametrize("M", [4, 1])
def test_repeat_and_workspace_contents(q38, orc, stack, M):
    import torch
    d = stack[0].desc
    h0 = orc.embed(SEED, list(range(300, 300 + M)), 2048)
    ws = G.workspace(q38.lib.q38_moe_workspace_size(C.byref(d), 4))
    outs = []
    for rep in range(4):
        if rep == 2:  # arbitrary prior contents (bytes that are not the reset pattern)
            ws.copy_(torch.randint(0, 255, (ws.numel(),), dtype=torch.uint8, device=ws.device))
        if rep == 3:  # a call of the other width in between on the same workspace
            other = 1 if M == 4 else 4
            h1 = G.to_dev(orc.embed(SEED, list(range(400, 400 + other)), 2048))
            chain(q38, stack, h1, ws, other)
        h = G.to_dev(h0)
        chain(q38, stack, h, ws, M)
        outs.append(G.to_host(h, np.uint16))
    assert np.all(np.isfinite((outs[0].astype(np.uint32) << 16).view(np.float32)))
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])


def test_graph_replays(q38, orc, stack):
    import torch
    M = 4
    d = stack[0].desc
    h0 = G.to_dev(orc.embed(SEED, list(range(500, 500 + M)), 2048))
    ws = G.workspace(q38.lib.q38_moe_workspace_size(C.byref(d), M))
    h = h0.clone()
    chain(q38, stack, h, ws, M)
    torch.cuda.synchronize()
    eager = G.to_host(h, np.uint16)
    hg = h0.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        arr = (C.c_void_p * len(stack))(*[L.h.value for L in stack])
        q38.check(q38.lib.q38_verify_chain(arr, len(stack), hg.data_ptr(), M, C.c_float(1e-6), None,
                                           ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream))
    for rep in range(3):
        hg.copy_(h0)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(G.to_host(hg, np.uint16), eager), rep
        # eager work between the replays on the same workspace
        h = h0.clone()
        chain(q38, stack, h, ws, M)
        torch.cuda.synchronize()
        assert np.array_equal(G.to_host(h, np.uint16), eager), rep
