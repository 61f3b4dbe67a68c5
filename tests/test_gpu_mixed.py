"""Config 4: the mixed VQ v2 layout (even experts d4/8-bit fp16 books, odd experts
d8/14-bit INT8 books with one fp16 scale per book), four request slots of k+1 = 4 rows
(16 rows) through a 48-layer stack, and independent per-slot commit / rollback.

Per layer, on the GPU's own layer input (teacher forcing), the RMSNorm is within one bf16
ulp of the float64 oracle and routing (experts, weights) is bit-exact at all 48 layers, and
the output is within tolerance on the first and last layer; the fused 48-layer call equals its
layer-by-layer replay bit for bit; each slot commits its own accepted length (drawn from
{0..3} with a seeded generator) or rolls back, and the others are untouched."""
import ctypes as C

import numpy as np
import pytest

import gpu_util as G
import oracle_lib
from moe_cases import SEED, bf16_ulps, run_forward, tol_check

pytestmark = pytest.mark.gpu

N_LAYERS = 48


def mixed_desc(q38):
    return q38.desc(mixed=1)


@pytest.fixture(scope="module")
def mixed_stack(gpu, q38):
    layers = [q38.MoeLayer(gpu, mixed_desc(q38), seed=SEED, layer=l) for l in range(N_LAYERS)]
    yield layers
    for L in layers:
        L.close()


@pytest.mark.parametrize("M", [1, 4, 16])
def test_mixed_layer_vs_oracle(mixed_stack, q38, orc, M):
    d = mixed_desc(q38)
    x = orc.rmsnorm(orc.embed(SEED, list(range(100, 100 + M)), 2048))
    y, ex, wt, lg, plan = run_forward(q38, mixed_stack[0], d, x)
    wy, wex, wwt, wlg = orc.moe_layer_synth(oracle_lib.make_desc(mixed=1), SEED, 0, x)
    assert np.array_equal(ex, wex)
    assert np.array_equal(wt, wwt)
    assert {int(e) % 2 for e in ex.reshape(-1)} == {0, 1}
    tol_check(orc, y, wy)


def run_chain(q38, layers, h_np):
    M = h_np.shape[0]
    h = G.to_dev(h_np)
    d = mixed_desc(q38)
    ws = G.workspace(q38.lib.q38_moe_workspace_size(C.byref(d), M))
    arr = (C.c_void_p * len(layers))(*[L.h.value for L in layers])
    xs = [G.empty((M, 2048), np.uint16) for _ in layers]
    exs = [G.empty(M * 10, np.int32) for _ in layers]
    wts = [G.empty(M * 10, np.float32) for _ in layers]
    tr = (q38.RouteOut * len(layers))(*[q38.routes(experts=e, weights=w, x_norm=x) for x, e, w in zip(xs, exs, wts)])
    q38.check(q38.lib.q38_verify_chain(arr, len(layers), h.data_ptr(), M, 1e-6, tr, ws.data_ptr(), ws.numel(),
                                       G.stream()))
    return G.to_host(h, np.uint16), [(G.to_host(x, np.uint16), G.to_host(e).reshape(M, 10),
                                      G.to_host(w).reshape(M, 10)) for x, e, w in zip(xs, exs, wts)]


def test_four_slots_chain_and_commit(mixed_stack, gpu, q38, orc):
    rng = np.random.default_rng(SEED)
    tokens = [int(t) for t in rng.integers(0, 151936, 16)]     # 4 slots x (current + 3 drafts)
    h0 = orc.embed(SEED, tokens, 2048)
    # fused 48-layer pass, then its layer-by-layer replay with per-layer oracle checks
    fused, _ = run_chain(q38, mixed_stack, h0)
    h = h0
    d = oracle_lib.make_desc(mixed=1)
    for l in range(N_LAYERS):
        h_next, tr = run_chain(q38, mixed_stack[l:l + 1], h)
        xg, exg, wtg = tr[0]
        # RMSNorm within one bf16 ulp (per element) of the float64 oracle, every layer
        assert bf16_ulps(orc, xg, orc.rmsnorm(h)).max() <= 1, f"layer {l} norm"
        # routing of every layer, bit for bit, on the x the GPU used
        ex, wt, _ = orc.route_synth(d, SEED, l, xg)
        assert np.array_equal(exg, ex), f"layer {l} experts"
        assert np.array_equal(wtg.view(np.uint32), wt.view(np.uint32)), f"layer {l} weights"
        if l in (0, N_LAYERS - 1):
            y, _, _, _ = orc.moe_layer_synth(d, SEED, l, xg)
            tol_check(orc, h_next, orc.residual_add(h, y))
        h = h_next
    assert np.array_equal(fused, h)
    assert np.isfinite(orc.bf16_to_f32(fused)).all()

    # per-slot checkpoints: each slot stages its 4 rows, then commits accepted in {0..3}
    # or rolls back; the other slots are unaffected
    final = orc.rmsnorm(fused)
    slots = []
    for s in range(4):
        p = C.c_void_p()
        q38.check(q38.lib.q38_slot_create(gpu.h, 2048, 4, 1000 + 10 * s, C.byref(p)))
        slots.append(p)
    try:
        accepted = [int(a) for a in rng.integers(0, 4, 4)]
        rollback = [False, False, True, False]
        rows_dev = [G.to_dev(np.ascontiguousarray(final[4 * s:4 * s + 4])) for s in range(4)]
        for s in range(4):
            q38.check(q38.lib.q38_slot_stage(slots[s], 3, rows_dev[s].data_ptr(), G.stream()))
        for s in range(4):
            if rollback[s]:
                q38.check(q38.lib.q38_slot_rollback(slots[s]))
            else:
                q38.check(q38.lib.q38_slot_commit(slots[s], accepted[s], G.stream()))
        G.hip().hipDeviceSynchronize()
        for s in range(4):
            tc, sr, dc = C.c_uint64(), C.c_int32(), C.c_int32()
            q38.check(q38.lib.q38_slot_info(slots[s], C.byref(tc), C.byref(sr), C.byref(dc)))
            assert sr.value == 0
            if rollback[s]:
                assert tc.value == 1000 + 10 * s
            else:
                assert tc.value == 1000 + 10 * s + accepted[s] + 1
                row = G.d2h(q38.lib.q38_slot_hidden(slots[s]), 2048, np.uint16)
                assert np.array_equal(row, final[4 * s + accepted[s]])
    finally:
        for p in slots:
            q38.lib.q38_slot_destroy(p)


@pytest.mark.parametrize("M", [4, 16])
def test_explicit_mixed_layer_equals_synthetic(gpu, q38, mixed_stack, M):
    """q38_moe_layer_create_mixed over caller-owned tensors: a layer built from the bank tensors
    of a synthetic mixed layer (the generator the oracle reproduces, pinned by
    test_mixed_layer_vs_oracle) gives the same routing and outputs bit for bit."""
    src = mixed_stack[5]
    w = q38.MoeMixedWeights()
    q38.check(q38.lib.q38_moe_layer_mixed_weights(src.h, C.byref(w)))
    assert all(w.codes_d4[p] and w.codes_d8[p] and w.books_d8[p] for p in range(3))
    d = mixed_desc(q38)
    h = C.c_void_p()
    q38.check(q38.lib.q38_moe_layer_create_mixed(gpu.h, C.byref(d), C.byref(w), C.byref(h)))

    class Explicit:
        pass

    ex_layer = Explicit()
    ex_layer.h = h
    try:
        x = G.to_host(G.to_dev(np.random.default_rng(M).normal(0, 1, (M, 2048)).astype(np.float32)))
        xb = (x.view(np.uint32) >> 16).astype(np.uint16)
        a = run_forward(q38, src, d, xb)
        b = run_forward(q38, ex_layer, d, xb)
        for u, v in zip(a, b):
            assert np.array_equal(u, v)
        # the uniform-layer accessor refuses a mixed layer, and creation refuses a missing bank tensor
        assert q38.lib.q38_moe_layer_weights(h, C.byref(q38.MoeWeights())) == q38.Q38_EINVAL
        w.books_d8[1] = None
        h2 = C.c_void_p()
        assert q38.lib.q38_moe_layer_create_mixed(gpu.h, C.byref(d), C.byref(w), C.byref(h2)) == q38.Q38_EINVAL
    finally:
        q38.lib.q38_moe_layer_destroy(h)
