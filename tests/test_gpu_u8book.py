"""Per-dimension INT8/U8 codebooks (R6, Q38_CB_U8_PERDIM) on the GPU: the tables the device
derives at layer creation equal the oracle's restatement of SparseMoe::prepare_u8_codebook
(src/sparse_moe.cpp:750-804) bit for bit, and layers using them match the oracle at verify
widths (1, 4, 16 rows), prefill width and with per-64-input scale groups.

At 1-16 rows such layers run on the kernels that read the U8 books themselves (the reference's
verify-width decode, src/vq_metal_kernels.hpp:564-579): checked against the oracle's float
decode and against the decoded-fp16-book kernels (q38_set_u8_native(0)) on the same rows
(mode 2 takes them at 1-4 rows too; the default takes them at 5-16)."""
import ctypes as C

import numpy as np
import pytest

import gpu_util as G
import oracle_lib
from moe_cases import SEED, ExplicitLayer, run_forward, tol_check

pytestmark = pytest.mark.gpu

K, D = 16384, 8


@pytest.fixture(scope="module")
def u8layer(gpu, q38):
    L = q38.MoeLayer(gpu, q38.desc(book_format=q38.Q38_CB_U8_PERDIM), seed=SEED, layer=9)
    yield L
    L.close()


def test_device_tables_match_oracle(u8layer, orc):
    for p in range(3):
        book, q, s, b = u8layer.codebook(p)
        raw = orc.normal(orc.key(SEED, 9, 3 + p), 0, K * D, 1.0, f16=True)
        wq, ws, wb, wv = orc.prepare_u8_book(raw, K, D, p == 0)
        gq = G.d2h(q, K * D, np.int8 if p == 0 else np.uint8).astype(np.int32)
        assert np.array_equal(gq, wq), p
        assert np.array_equal(G.d2h(s, D, np.uint16), ws) and np.array_equal(G.d2h(b, D, np.uint16), wb), p
        # the book the kernels read: the float decode rounded to fp16
        assert np.array_equal(G.d2h(book, K * D, np.uint16), wv.astype(np.float16).view(np.uint16)), p


@pytest.mark.parametrize("M", [1, 4, 16, 64])
def test_u8book_layer_vs_oracle(u8layer, q38, orc, M):
    x = orc.rmsnorm(orc.embed(SEED, [300 + 13 * i for i in range(M)], 2048))
    y, ex, wt, lg, plan = run_forward(q38, u8layer, u8layer.desc, x)
    wy, wex, wwt, wlg = orc.moe_layer_synth(oracle_lib.make_desc(book_format=2), SEED, 9, x)
    assert np.array_equal(ex, wex) and np.array_equal(wt, wwt), "routing"
    tol_check(orc, y, wy)
    # the FP16-book layer differs (the derived books are in effect)
    y16, _, _, _ = orc.moe_layer_synth(oracle_lib.make_desc(), SEED, 9, x)
    assert not np.array_equal(wy, y16)


@pytest.mark.parametrize("M", [1, 4])
def test_u8book_group64_explicit(gpu, q38, orc, M):
    L = ExplicitLayer(q38, gpu, orc, gu_group=64, down_group=64, seed=21, book_format=2)
    try:
        x = orc.bf16(np.random.default_rng(M).normal(0, 1, (M, L.H)))
        y, ex, wt, lg, plan = run_forward(q38, L.layer, L.qdesc, x)
        wy, wex, wwt, wlg = L.oracle(orc, x)
        assert np.array_equal(ex, wex)
        tol_check(orc, y, wy)
    finally:
        L.close()


def test_book_format_validation(gpu, q38):
    h = C.c_void_p()
    d = q38.desc(mixed=1, book_format=2)
    assert q38.lib.q38_moe_layer_create_synthetic(gpu.h, C.byref(d), SEED, 0, C.byref(h)) == q38.Q38_EINVAL
    d = q38.desc(book_format=5)
    assert q38.lib.q38_moe_layer_create_synthetic(gpu.h, C.byref(d), SEED, 0, C.byref(h)) == q38.Q38_EINVAL


@pytest.fixture
def restore_u8_native(q38):
    yield
    q38.lib.q38_set_u8_native(1)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 9, 16])
def test_u8_kernels_vs_decoded_book(u8layer, q38, orc, restore_u8_native, M):
    """Routing identical on both paths; both within the MoE tolerance of the oracle's float
    decode; the outputs differ (the U8 kernels' arithmetic, not the decoded book, ran)."""
    x = orc.rmsnorm(orc.embed(SEED, [900 + 7 * i for i in range(M)], 2048))
    q38.lib.q38_set_u8_native(2)
    y1, ex1, wt1, lg1, plan1 = run_forward(q38, u8layer, u8layer.desc, x)
    q38.lib.q38_set_u8_native(0)
    y0, ex0, wt0, lg0, plan0 = run_forward(q38, u8layer, u8layer.desc, x)
    wy, wex, wwt, wlg = orc.moe_layer_synth(oracle_lib.make_desc(book_format=2), SEED, 9, x)
    assert np.array_equal(ex1, wex) and np.array_equal(wt1, wwt) and np.array_equal(plan1, plan0)
    assert np.array_equal(ex0, wex) and np.array_equal(wt0, wwt)
    r1 = tol_check(orc, y1, wy)
    r0 = tol_check(orc, y0, wy)
    print(f"M={M}: U8 kernels rel {r1[0]:.2e} max {r1[1]:.2e}; decoded book rel {r0[0]:.2e} max {r0[1]:.2e}")
    assert not np.array_equal(y1, y0)


def test_u8_kernels_repeat_and_width_change(u8layer, q38, orc, restore_u8_native):
    """The same call twice gives the same bits; a 16-row call in between (other staging and
    passes) leaves no state behind."""
    q38.lib.q38_set_u8_native(2)
    x4 = orc.rmsnorm(orc.embed(SEED, [11, 12, 13, 14], 2048))
    x16 = orc.rmsnorm(orc.embed(SEED, list(range(500, 516)), 2048))
    a = run_forward(q38, u8layer, u8layer.desc, x4)[0]
    run_forward(q38, u8layer, u8layer.desc, x16)
    b = run_forward(q38, u8layer, u8layer.desc, x4)[0]
    assert np.array_equal(a, b)
