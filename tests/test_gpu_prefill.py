"""Config 3, prefill width: 17..2048 token rows through one MoE layer of config-0 shapes
(SparseMoe::forward_prefill_impl's segmented path, src/sparse_moe.cpp:2252-2505), on the
segmented-GEMM kernels, with the router logits skewed like Zipf(1.1).

- router logits bit-exact with the oracle on sampled rows, and with the verify-width router
  on the same rows;
- top-k bit-exact with the oracle's top-k of the GPU's logits, for every row;
- the route plan bit-exact with a stable sort of the routes by expert (numpy) and with the
  oracle's plan;
- layer outputs within the MoE tolerance of the oracle on sampled rows;
- the workload itself: hot experts receive 60-200 of 512 rows, a third of the experts 0-4."""
import ctypes as C

import numpy as np
import pytest

import gpu_util as G
import oracle_lib
from moe_cases import SEED, ExplicitLayer, plan_check, run_forward, tol_check
from workloads import zipf_router_bias

pytestmark = pytest.mark.gpu

LAYER = 3


@pytest.fixture(scope="module")
def zipf_layer(gpu, q38):
    L = q38.MoeLayer(gpu, q38.desc(), seed=SEED, layer=LAYER)
    bias = zipf_router_bias(512, SEED)
    bias_dev = G.to_dev(bias)
    q38.check(q38.lib.q38_moe_layer_set_router_bias(L.h, bias_dev.data_ptr()))
    yield L, bias
    L.close()


def tokens(n, seed=SEED):
    return [int(t) for t in np.random.default_rng(seed + n).integers(0, 151936, n)]


def stable_plan_check(orc, plan, ex, E):
    MK = ex.size
    order = np.argsort(ex.reshape(-1), kind="stable")
    assert np.array_equal(plan[2 + 2 * MK:2 + 3 * MK], order)
    plan_check(orc, plan, ex, E)


def sampled_rows(M, n, seed):
    rows = np.random.default_rng(seed).choice(M, size=n - 2, replace=False)
    return np.unique(np.concatenate([[0, M - 1], rows]))


def check_rows_vs_oracle(orc, d, x, y, ex, wt, lg, rows, bias):
    wy, wex, wwt, wlg = orc.moe_layer_synth(d, SEED, LAYER, x[rows], bias=bias)
    assert np.array_equal(lg[rows].view(np.uint32), wlg.view(np.uint32)), "router logits"
    assert np.array_equal(ex[rows], wex)
    assert np.array_equal(wt[rows].view(np.uint32), wwt.view(np.uint32))
    tol_check(orc, y[rows], wy)


def test_prefill_512_zipf(zipf_layer, q38, orc):
    L, bias = zipf_layer
    d, od = q38.desc(), oracle_lib.make_desc()
    M = 512
    x = orc.rmsnorm(orc.embed(SEED, tokens(M), 2048))
    y, ex, wt, lg, plan = run_forward(q38, L, d, x)
    # top-k of every row from the GPU's logits
    oex, owt = orc.route(lg, 10)
    assert np.array_equal(ex, oex) and np.array_equal(wt.view(np.uint32), owt.view(np.uint32))
    stable_plan_check(orc, plan, ex, 512)
    counts = np.bincount(ex.reshape(-1), minlength=512)
    assert 60 <= counts.max() <= 200, counts.max()
    assert (counts >= 60).sum() >= 4 and (counts <= 4).sum() >= 120
    check_rows_vs_oracle(orc, od, x, y, ex, wt, lg, sampled_rows(M, 24, 1), bias)
    # the verify-width router gives the same logits on a 16-row slice
    ws = G.workspace(q38.lib.q38_moe_workspace_size(C.byref(d), 16))
    lg16 = G.empty(16 * 512, np.float32)
    xs = G.to_dev(np.ascontiguousarray(x[100:116]))
    q38.check(q38.lib.q38_moe_route(L.h, xs.data_ptr(), 16, C.byref(q38.routes(logits=lg16)), ws.data_ptr(),
                                    ws.numel(), G.stream()))
    assert np.array_equal(G.to_host(lg16).reshape(16, 512).view(np.uint32), lg[100:116].view(np.uint32))


def test_prefill_profiled_equals_forward(zipf_layer, q38, orc):
    L, _ = zipf_layer
    d = q38.desc()
    M = 512
    x_np = orc.rmsnorm(orc.embed(SEED, tokens(M), 2048))
    y_ref = run_forward(q38, L, d, x_np)[0]
    x = G.to_dev(x_np)
    y = G.empty(x_np.shape, np.uint16)
    ws = G.workspace(q38.lib.q38_moe_workspace_size(C.byref(d), M))
    ms = (C.c_float * 7)()
    q38.check(q38.lib.q38_moe_forward_prefill_profiled(L.h, x.data_ptr(), M, y.data_ptr(), None, ws.data_ptr(),
                                                       ws.numel(), ms, G.stream()))
    assert np.array_equal(G.to_host(y, np.uint16), y_ref)
    assert all(v > 0 for v in ms), list(ms)


def test_prefill_2048_multi_pass(zipf_layer, q38, orc):
    """The widest call: a hot expert's routes span several 256-route passes."""
    L, bias = zipf_layer
    d, od = q38.desc(), oracle_lib.make_desc()
    M = 2048
    x = orc.rmsnorm(orc.embed(SEED, tokens(M), 2048))
    y, ex, wt, lg, plan = run_forward(q38, L, d, x)
    oex, _ = orc.route(lg, 10)
    assert np.array_equal(ex, oex)
    stable_plan_check(orc, plan, ex, 512)
    assert np.bincount(ex.reshape(-1), minlength=512).max() > 256
    check_rows_vs_oracle(orc, od, x, y, ex, wt, lg, sampled_rows(M, 10, 2), bias)
    assert np.isfinite(orc.bf16_to_f32(y)).all()


def test_prefill_17_rows_unbiased(gpu, q38, orc):
    """The narrowest prefill call, no bias: every row against the oracle."""
    L = q38.MoeLayer(gpu, q38.desc(), seed=SEED, layer=LAYER)
    try:
        M = 17
        x = orc.rmsnorm(orc.embed(SEED, tokens(M), 2048))
        y, ex, wt, lg, plan = run_forward(q38, L, q38.desc(), x)
        wy, wex, wwt, wlg = orc.moe_layer_synth(oracle_lib.make_desc(), SEED, LAYER, x)
        assert np.array_equal(lg.view(np.uint32), wlg.view(np.uint32))
        assert np.array_equal(ex, wex)
        stable_plan_check(orc, plan, ex, 512)
        tol_check(orc, y, wy)
        # the verify kernels on the first 16 rows agree within the same tolerance
        y16 = run_forward(q38, L, q38.desc(), x[:16])[0]
        tol_check(orc, y[:16], y16)
    finally:
        L.close()


def test_prefill_explicit_small_layer(gpu, q38, orc):
    """A small explicit layer (E = 64, k = 4, H = 512, I = 256): the generic top-k path."""
    lay = ExplicitLayer(q38, gpu, orc, H=512, I=256, E=64, k=4, seed=11)
    try:
        x = orc.rmsnorm(orc.embed(SEED, tokens(96), 512))
        y, ex, wt, lg, plan = run_forward(q38, lay.layer, lay.qdesc, x)
        wy, wex, wwt, wlg = lay.oracle(orc, x)
        assert np.array_equal(ex, wex)
        stable_plan_check(orc, plan, ex, 64)
        tol_check(orc, y, wy)
    finally:
        lay.close()


def test_prefill_rejects(gpu, q38, orc):
    d = q38.desc()
    L = q38.MoeLayer(gpu, d, seed=SEED, layer=LAYER)
    mixed = q38.MoeLayer(gpu, q38.desc(mixed=1), seed=SEED, layer=0)
    try:
        ws = G.workspace(q38.lib.q38_moe_workspace_size(C.byref(d), 64))
        x = G.empty((2049, 2048), np.uint16)
        y = G.empty((2049, 2048), np.uint16)
        assert q38.lib.q38_moe_forward(L.h, x.data_ptr(), 2049, y.data_ptr(), None, ws.data_ptr(), ws.numel(),
                                       G.stream()) == q38.Q38_EINVAL
        assert q38.lib.q38_moe_forward(L.h, x.data_ptr(), 64, y.data_ptr(), None, ws.data_ptr(), 1024,
                                       G.stream()) == q38.Q38_ESPACE
        # the mixed VQ v2 layout has no prefill kernels
        assert q38.lib.q38_moe_forward(mixed.h, x.data_ptr(), 32, y.data_ptr(), None, ws.data_ptr(), ws.numel(),
                                       G.stream()) == q38.Q38_EINVAL
        assert b"prefill" in q38.lib.q38_last_error()
    finally:
        L.close()
        mixed.close()


# ---------------------------------------------------------------- grouped-scale layouts
# Layouts the segmented MFMA kernels do not take run at prefill widths on the grouped VALU
# kernels, in passes of up to 16 of a slot's routes (hot experts take many passes).

def test_prefill_512_zipf_group64(gpu, q38, orc):
    """The reference checkpoints' layout (d8/14-bit, one FP16 scale per 64 inputs) at 512 rows
    with Zipf-skewed routing: logits, top-k, weights and the stable plan bit-exact, outputs
    within the MoE tolerance of the oracle on sampled rows."""
    M = 512
    d = q38.desc(gu_group=64, down_group=64)
    od = oracle_lib.make_desc(gu_group=64, down_group=64)
    L = q38.MoeLayer(gpu, d, seed=SEED, layer=LAYER)
    try:
        bias = zipf_router_bias(512, SEED)
        bias_dev = G.to_dev(bias)
        q38.check(q38.lib.q38_moe_layer_set_router_bias(L.h, bias_dev.data_ptr()))
        x = orc.rmsnorm(orc.embed(SEED, tokens(M), 2048))
        y, ex, wt, lg, plan = run_forward(q38, L, d, x)
        oex, owt = orc.route(lg, 10)
        assert np.array_equal(ex, oex) and np.array_equal(wt.view(np.uint32), owt.view(np.uint32))
        stable_plan_check(orc, plan, ex, 512)
        counts = np.bincount(ex.reshape(-1), minlength=512)
        assert counts.max() > 32  # some slots take several 16-route passes
        check_rows_vs_oracle(orc, od, x, y, ex, wt, lg, sampled_rows(M, 16, 3), bias)
        assert np.isfinite(orc.bf16_to_f32(y)).all()
    finally:
        L.close()


@pytest.mark.parametrize("geo,M", [(dict(gu=(4, 8), down=(4, 8)), 40), (dict(gu=(2, 8), down=(2, 8), gu_group=64,
                                                                            down_group=64), 100),
                                   (dict(gu=(8, 14), down=(4, 8), gu_group=64, down_group=64), 33)])
def test_prefill_grouped_small_layers(gpu, q38, orc, geo, M):
    """d4/8 with row scales, d2/8 byte codes with 64-input groups, and d8 gate/up over a d4
    down, at prefill widths on a small explicit layer (E = 64, k = 4: slots with up to ~M/4
    routes, several passes each): every row against the oracle."""
    lay = ExplicitLayer(q38, gpu, orc, H=512, I=256, E=64, k=4, seed=13 + M, **geo)
    try:
        x = orc.rmsnorm(orc.embed(SEED, tokens(M), 512))
        y, ex, wt, lg, plan = run_forward(q38, lay.layer, lay.qdesc, x)
        wy, wex, wwt, wlg = lay.oracle(orc, x)
        assert np.array_equal(lg.view(np.uint32), wlg.view(np.uint32)) and np.array_equal(ex, wex)
        assert np.array_equal(wt.view(np.uint32), wwt.view(np.uint32))
        stable_plan_check(orc, plan, ex, 64)
        tol_check(orc, y, wy)
    finally:
        lay.close()


def test_prefill_grouped_matches_verify_rows(gpu, q38, orc):
    """The same rows through the grouped kernels at prefill width (40 rows) and at verify
    width (the first 16 rows alone): outputs within the MoE tolerance of each other, routing
    identical."""
    d = q38.desc(gu_group=64, down_group=64)
    L = q38.MoeLayer(gpu, d, seed=SEED, layer=5)
    try:
        x = orc.rmsnorm(orc.embed(SEED, tokens(40), 2048))
        y, ex, wt, lg, _ = run_forward(q38, L, d, x)
        y16, ex16, wt16, lg16, _ = run_forward(q38, L, d, x[:16])
        assert np.array_equal(ex[:16], ex16) and np.array_equal(wt[:16].view(np.uint32), wt16.view(np.uint32))
        tol_check(orc, y[:16], y16)
    finally:
        L.close()
