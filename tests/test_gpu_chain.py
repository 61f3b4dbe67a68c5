"""The k+1 verify pass through 48 MoE layers (config 1): per layer, with the GPU's own
layer input (teacher forcing), routing (logits, experts, weights) is bit-exact at every
one of the 48 layers, the layer output is within tolerance on a subset of them (the
oracle's expert arithmetic is the slow part), and the fused 48-layer call equals the
layer-by-layer result bit for bit."""
import ctypes as C

import numpy as np
import pytest

import gpu_util as G
import oracle_lib
from moe_cases import SEED, bf16_ulps, tol_check

pytestmark = pytest.mark.gpu

N_LAYERS = 48


@pytest.fixture(scope="module")
def stack(gpu, q38):
    layers = [q38.MoeLayer(gpu, q38.desc(), seed=SEED, layer=l) for l in range(N_LAYERS)]
    yield layers
    for L in layers:
        L.close()


def run_chain(q38, layers, h_np, traces=False):
    M = h_np.shape[0]
    h = G.to_dev(h_np)
    d = layers[0].desc
    ws = G.workspace(q38.lib.q38_moe_workspace_size(C.byref(d), M))
    arr = (C.c_void_p * len(layers))(*[L.h.value for L in layers])
    bufs = None
    tr = None
    if traces:
        bufs = [(G.empty((M, 2048), np.uint16), G.empty(M * 10, np.int32), G.empty(M * 10, np.float32),
                 G.empty(M * 512, np.float32)) for _ in layers]
        tr = (q38.RouteOut * len(layers))(*[q38.routes(experts=e, weights=w, logits=g, x_norm=x)
                                            for x, e, w, g in bufs])
    q38.check(q38.lib.q38_verify_chain(arr, len(layers), h.data_ptr(), M, 1e-6, tr, ws.data_ptr(), ws.numel(),
                                       G.stream()))
    out = G.to_host(h, np.uint16)
    if not traces:
        return out, None
    return out, [(G.to_host(x, np.uint16), G.to_host(e).reshape(M, 10), G.to_host(w).reshape(M, 10),
                  G.to_host(g).reshape(M, 512)) for x, e, w, g in bufs]


@pytest.mark.parametrize("M", [4, 3, 2, 1])
def test_chain_teacher_forced(stack, q38, orc, M):
    tokens = [11, 22, 33, 44][:M]
    h0 = orc.embed(SEED, tokens, 2048)
    check_layers = {0, 1, 2, 23, 46, 47} if M == 4 else {0, 47}
    h = h0
    d = oracle_lib.make_desc()
    per_layer = []
    for l in range(N_LAYERS):
        h_next, tr = run_chain(q38, stack[l:l + 1], h, traces=True)
        xg, exg, wtg, lgg = tr[0]
        # RMSNorm within one bf16 ulp (per element) of the float64 oracle
        xo = orc.rmsnorm(h)
        assert bf16_ulps(orc, xg, xo).max() <= 1
        # routing of every layer, bit for bit, on the x the GPU used
        ex, wt, lg = orc.route_synth(d, SEED, l, xg)
        assert np.array_equal(lgg.view(np.uint32), lg.view(np.uint32)), f"layer {l} logits"
        assert np.array_equal(exg, ex), f"layer {l} experts"
        assert np.array_equal(wtg.view(np.uint32), wt.view(np.uint32)), f"layer {l} weights"
        if l in check_layers:
            y, ex2, _, _ = orc.moe_layer_synth(d, SEED, l, xg)
            assert np.array_equal(ex2, ex)
            tol_check(orc, h_next, orc.residual_add(h, y))
        per_layer.append(h_next)
        h = h_next
    fused, _ = run_chain(q38, stack, h0)
    assert np.array_equal(fused, per_layer[-1])
    assert np.isfinite(orc.bf16_to_f32(fused)).all()
