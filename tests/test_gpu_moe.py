"""Sparse-MoE layer on the GPU vs the CPU oracle: routing, plans and greedy-relevant
integer outputs bit-exact; MoE outputs within relative L2 <= 1e-2 and max-abs <= 2e-2."""
import ctypes as C

import numpy as np
import pytest

import gpu_util as G
import oracle_lib
from moe_cases import SEED, ExplicitLayer, plan_check, run_forward, tol_check

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def layer0(gpu, q38):
    L = q38.MoeLayer(gpu, q38.desc(), seed=SEED, layer=0)
    yield L
    L.close()


@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_config0_layer(layer0, q38, orc, M):
    x = orc.normal(orc.key(SEED, 0, 20), 1000 * M, M * 2048, 1.0).reshape(M, 2048)
    y, ex, wt, lg, plan = run_forward(q38, layer0, layer0.desc, x)
    wy, wex, wwt, wlg = orc.moe_layer_synth(oracle_lib.make_desc(), SEED, 0, x)
    assert np.array_equal(lg, wlg), "router logits"
    assert np.array_equal(ex, wex), "routed experts"
    assert np.array_equal(wt, wwt), "route weights"
    plan_check(orc, plan, ex, 512)
    tol_check(orc, y, wy)


@pytest.fixture(scope="module")
def layer_g64(gpu, q38):
    L = q38.MoeLayer(gpu, q38.desc(gu_group=64, down_group=64), seed=SEED, layer=5)
    yield L
    L.close()


@pytest.mark.parametrize("M", [1, 2, 3, 4, 16])
def test_group64_layer(layer_g64, q38, orc, M):
    """One fp16 scale per 64 inputs (the reference checkpoints' layout) on the config-0
    geometry: rows 1-4 take the four-row MFMA kernels, which scale each K slice's four group
    partial sums; 16 rows take the grouped VALU kernels. Routing bit-exact, outputs within
    the MoE tolerance of the oracle."""
    x = orc.normal(orc.key(SEED, 5, 20), 31 * M, M * 2048, 1.0).reshape(M, 2048)
    y, ex, wt, lg, plan = run_forward(q38, layer_g64, layer_g64.desc, x)
    wy, wex, wwt, wlg = orc.moe_layer_synth(oracle_lib.make_desc(gu_group=64, down_group=64), SEED, 5, x)
    assert np.array_equal(lg, wlg) and np.array_equal(ex, wex) and np.array_equal(wt, wwt)
    plan_check(orc, plan, ex, 512)
    tol_check(orc, y, wy)


def test_group64_narrow_matches_grouped_kernels(layer_g64, q38, orc):
    """The same four rows through the four-row kernels (a 4-row call) and the grouped VALU
    kernels (rows 0-3 of a 5-row call) agree within the MoE tolerance."""
    x = orc.normal(orc.key(SEED, 5, 21), 3, 5 * 2048, 1.0).reshape(5, 2048)
    y4 = run_forward(q38, layer_g64, layer_g64.desc, x[:4])[0]
    y5 = run_forward(q38, layer_g64, layer_g64.desc, x)[0]
    tol_check(orc, y4, y5[:4])


@pytest.mark.parametrize("M", [4, 16])
def test_fp16_operand_extremes(layer0, q38, orc, M):
    """The expert kernels take x as an fp16 MFMA operand. RMSNorm outputs with one spike
    per row reach sqrt(H) ~ 45 in one element and put the rest below fp16's normal range
    (2^-14); the layer output stays within the MoE tolerance of the oracle, whose products
    are in float."""
    rng = np.random.default_rng(M)
    h = rng.normal(0, 1e-4, (M, 2048))
    h[np.arange(M), rng.integers(0, 2048, M)] = 1e3
    x = orc.rmsnorm(orc.bf16(h))
    xf = orc.bf16_to_f32(x)
    assert np.abs(xf).max() > 40 and (np.abs(xf) < 2.0 ** -14).mean() > 0.9
    y, ex, wt, lg, plan = run_forward(q38, layer0, layer0.desc, x)
    wy, wex, wwt, wlg = orc.moe_layer_synth(oracle_lib.make_desc(), SEED, 0, x)
    assert np.array_equal(ex, wex) and np.array_equal(wt, wwt)
    tol_check(orc, y, wy)


def test_sixteen_rows(layer0, q38, orc):
    x = orc.normal(orc.key(SEED, 0, 20), 7, 16 * 2048, 1.0).reshape(16, 2048)
    y, ex, wt, lg, plan = run_forward(q38, layer0, layer0.desc, x)
    wy, wex, wwt, wlg = orc.moe_layer_synth(oracle_lib.make_desc(), SEED, 0, x)
    assert np.array_equal(ex, wex) and np.array_equal(wt, wwt)
    plan_check(orc, plan, ex, 512)
    tol_check(orc, y, wy)


def test_repeated_rows_share_experts(layer0, q38, orc):
    """Identical rows route identically; each expert's code rows are applied to both."""
    x1 = orc.normal(orc.key(SEED, 0, 20), 99, 2048, 1.0)
    x = np.stack([x1, x1, x1, x1])
    y, ex, wt, lg, plan = run_forward(q38, layer0, layer0.desc, x)
    assert plan[0] == 10 and (ex == ex[0]).all()
    assert (y == y[0]).all()


@pytest.mark.parametrize("geo", [dict(gu=(8, 14), down=(8, 14)), dict(gu=(4, 8), down=(4, 8)),
                                 dict(gu=(8, 14), down=(4, 8), gu_group=64, down_group=64),
                                 dict(gu=(4, 8), down=(8, 14), gu_group=64, down_group=64)])
@pytest.mark.parametrize("M", [1, 4, 16])
def test_explicit_small_layers(gpu, q38, orc, geo, M):
    L = ExplicitLayer(q38, gpu, orc, seed=M, **geo)
    try:
        x = orc.bf16(np.random.default_rng(M).normal(0, 1, (M, 512)))
        y, ex, wt, lg, plan = run_forward(q38, L.layer, L.qdesc, x)
        wy, wex, wwt, wlg = L.oracle(orc, x)
        assert np.array_equal(lg, wlg) and np.array_equal(ex, wex) and np.array_equal(wt, wwt)
        plan_check(orc, plan, ex, 64)
        tol_check(orc, y, wy)
    finally:
        L.close()


def test_router_contract_order_and_ties(gpu, q38, orc):
    """Logit order pin (a sequential sum gives 0, the contract 1) and lower-index ties."""
    H, E = 512, 64
    router = np.zeros((E, H), np.float32)
    router[0, 0], router[0, 8], router[0, 264] = 1.0, 2.0 ** 24, -(2.0 ** 24)
    rng = np.random.default_rng(9)
    router[1:] = rng.normal(0, 0.02, (E - 1, H))
    router[5] = router[3] = 0.5     # duplicated rows -> equal logits
    x = np.zeros((2, H), np.float32)
    x[:, [0, 8, 264]] = 1.0
    x[1] = rng.normal(0, 1, H)
    x[1, [0, 8, 264]] = 0.0
    L = ExplicitLayer(q38, gpu, orc, H=H, E=E, router=orc.bf16(router))
    try:
        xb = orc.bf16(x)
        y, ex, wt, lg, plan = run_forward(q38, L.layer, L.qdesc, xb)
        wy, wex, wwt, wlg = L.oracle(orc, xb)
        assert lg[0, 0] == 1.0 == wlg[0, 0]
        assert np.array_equal(lg, wlg) and np.array_equal(ex, wex)
        r3, r5 = list(ex[1]).index(3) if 3 in ex[1] else None, list(ex[1]).index(5) if 5 in ex[1] else None
        assert lg[1, 3] == lg[1, 5]
        if r3 is not None and r5 is not None:
            assert r3 < r5
    finally:
        L.close()


def test_invalid_shapes_rejected(layer0, q38):
    ws = G.workspace(1 << 20)
    x = G.empty((17, 2048), np.uint16)
    y = G.empty((17, 2048), np.uint16)
    # 17 rows is a prefill width: valid, but it needs a larger workspace
    rc = q38.lib.q38_moe_forward(layer0.h, x.data_ptr(), 17, y.data_ptr(), None, ws.data_ptr(), ws.numel(), G.stream())
    assert rc == q38.Q38_ESPACE
    for rows in (0, -1, 2049):
        rc = q38.lib.q38_moe_forward(layer0.h, x.data_ptr(), rows, y.data_ptr(), None, ws.data_ptr(), ws.numel(),
                                     G.stream())
        assert rc == q38.Q38_EINVAL
    rc = q38.lib.q38_moe_forward(layer0.h, x.data_ptr(), 4, y.data_ptr(), None, ws.data_ptr(), 16, G.stream())
    assert rc == q38.Q38_ESPACE
    rc = q38.lib.q38_moe_forward(layer0.h, x.data_ptr(), 4, x.data_ptr(), None, ws.data_ptr(), ws.numel(), G.stream())
    assert rc == q38.Q38_EINVAL


def test_mixed_desc_rejected_by_uniform_create(gpu, q38):
    """q38_moe_layer_create takes uniform-geometry tensors only: a mixed description is an
    argument error (it would otherwise read per-bank geometry fields it does not have)."""
    d = q38.desc(mixed=1)
    d.gu_dim = d.down_dim = 0
    w = q38.MoeWeights()
    h = C.c_void_p()
    assert q38.lib.q38_moe_layer_create(gpu.h, C.byref(d), C.byref(w), C.byref(h)) == q38.Q38_EINVAL
    assert b"q38_moe_layer_create_mixed" in q38.lib.q38_last_error()


@pytest.mark.parametrize("H,I,M", [(2560, 512, 4), (2560, 512, 1), (2560, 640, 4)])
def test_hidden_2560_layers(gpu, q38, orc, H, I, M):
    """The reference family's hidden size: 2560 x 512 takes the four-row MFMA kernels with
    320-subvector K slices (10 waves), 2560 x 640 the general path; both against the oracle."""
    L = q38.MoeLayer(gpu, q38.desc(hidden=H, inter=I), seed=SEED, layer=7)
    try:
        x = orc.normal(orc.key(SEED, 7, 20), 31 * M, M * H, 1.0).reshape(M, H)
        y, ex, wt, lg, plan = run_forward(q38, L, L.desc, x)
        wy, wex, wwt, wlg = orc.moe_layer_synth(oracle_lib.make_desc(hidden=H, inter=I), SEED, 7, x)
        assert np.array_equal(lg, wlg), "router logits"
        assert np.array_equal(ex, wex) and np.array_equal(wt, wwt), "routing"
        plan_check(orc, plan, ex, 512)
        tol_check(orc, y, wy)
    finally:
        L.close()


@pytest.mark.parametrize("M", [1, 4])
def test_d8_gate_up_over_d4_down(gpu, q38, orc, M):
    """A full-size layer whose gate/up (d8/14-bit, 256 KiB book) and down (d4/8-bit, 2 KiB
    book) geometries differ takes the four-row kernels; the gate/up kernel's warm-up of the
    down book stays inside the down book's own lines."""
    d = q38.desc(gu=(8, 14), down=(4, 8))
    L = q38.MoeLayer(gpu, d, seed=SEED, layer=9)
    try:
        x = orc.normal(orc.key(SEED, 9, 21), 29 * M, M * 2048, 1.0).reshape(M, 2048)
        y, ex, wt, lg, plan = run_forward(q38, L, L.desc, x)
        wy, wex, wwt, wlg = orc.moe_layer_synth(oracle_lib.make_desc(gu=(8, 14), down=(4, 8)), SEED, 9, x)
        assert np.array_equal(lg, wlg), "router logits"
        assert np.array_equal(ex, wex) and np.array_equal(wt, wwt), "routing"
        plan_check(orc, plan, ex, 512)
        tol_check(orc, y, wy)
    finally:
        L.close()
