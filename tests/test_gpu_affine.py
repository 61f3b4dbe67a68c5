"""Layers whose shared expert is in MLX affine form (the reference checkpoints' shared-expert
format, q38_moe_layer_create_affine_shared): routing bit-exact with the oracle and outputs within
the MoE tolerance at verify widths (the one-launch experts with a separate combine at 1-4 rows,
the 16-row kernels) and at a prefill width; the shared kernels alone against the oracle's
affine expert; scale groups 32 / 64 / 128, 2 / 4 / 8 bits, bf16 and fp16 scales, and a shared
intermediate size other than the routed experts'."""
import ctypes as C

import numpy as np
import pytest

import gpu_util as G
import oracle_lib
from affine_cases import random_affine, to16
from moe_cases import run_forward, tol_check

pytestmark = pytest.mark.gpu


class AffineLayer:
    """A config-0-shaped layer (H 2048, I 512, 512 experts, top-10, d8/14 codes, per-row scales)
    with random routed tensors and an affine shared expert."""

    def __init__(self, q38, ctx, orc, seed, bits, group, fmt, Is=512, H=2048, I=512, E=512, k=10):
        rng = np.random.default_rng(seed)
        self.qdesc = q38.desc(hidden=H, inter=I, experts=E, top_k=k)
        self.odesc = oracle_lib.make_desc(hidden=H, inter=I, experts=E, top_k=k)
        self.router = orc.bf16(rng.normal(0, 0.02, (E, H)))
        self.wsg = orc.bf16(rng.normal(0, 0.02, H))
        self.books, self.codes, self.scales = [], [], []
        for IN, OUT in ((H, I), (H, I), (I, H)):
            self.books.append(to16(rng.normal(0, 1, 16384 * 8), 1))
            self.codes.append(rng.integers(0, 2 ** 32, E * OUT * (IN // 8 // 32) * 14, dtype=np.uint64).astype(np.uint32))
            self.scales.append(to16(rng.uniform(0.005, 0.02, E * OUT), 1))
        self.sa = random_affine(rng, H, Is, bits, group, fmt)
        self.dev = [G.to_dev(a) for a in [self.router, self.wsg, *self.codes, *self.scales, *self.books]]
        self.sdev = [G.to_dev(a) for a in (*self.sa["w"], *self.sa["s"], *self.sa["b"])]
        w = q38.MoeWeights()
        w.router, w.shared_gate = self.dev[0].data_ptr(), self.dev[1].data_ptr()
        for p in range(3):
            w.codes[p] = self.dev[2 + p].data_ptr()
            w.scales[p] = self.dev[5 + p].data_ptr()
            w.books[p] = self.dev[8 + p].data_ptr()
        a = q38.AffineShared()
        for p in range(3):
            a.weight[p] = self.sdev[p].data_ptr()
            a.scales[p] = self.sdev[3 + p].data_ptr()
            a.biases[p] = self.sdev[6 + p].data_ptr()
        a.bits, a.group, a.inter, a.scale_dtype = bits, group, Is, fmt
        self.h = C.c_void_p()
        q38.check(q38.lib.q38_moe_layer_create_affine_shared(ctx.h, C.byref(self.qdesc), C.byref(w), C.byref(a),
                                                             C.byref(self.h)))
        self.q38 = q38

    def oracle(self, orc, x):
        return orc.moe_layer_dense_affine_shared(self.odesc, self.router, self.wsg, self.codes, self.scales,
                                                 self.books, self.sa, x)

    def close(self):
        self.q38.lib.q38_moe_layer_destroy(self.h)


@pytest.fixture(scope="module")
def layers(gpu, q38, orc):
    ls = {(4, 64, 0): AffineLayer(q38, gpu, orc, 1, 4, 64, 0),
          (8, 32, 1): AffineLayer(q38, gpu, orc, 2, 8, 32, 1, Is=1024),
          (2, 128, 0): AffineLayer(q38, gpu, orc, 3, 2, 128, 0, Is=256)}
    yield ls
    for L in ls.values():
        L.close()


@pytest.mark.parametrize("key", [(4, 64, 0), (8, 32, 1), (2, 128, 0)])
@pytest.mark.parametrize("M", [1, 4, 16])
def test_affine_shared_layer_vs_oracle(layers, q38, orc, key, M):
    L = layers[key]
    x = orc.rmsnorm(orc.embed(0x5EED + M, list(range(7, 7 + M)), 2048))
    y, ex, wt, lg, plan = run_forward(q38, L, L.qdesc, x)
    wy, wex, wwt, wlg = L.oracle(orc, x)
    assert np.array_equal(ex, wex) and np.array_equal(wt, wwt)
    r, m = tol_check(orc, y, wy)
    print(f"affine shared {key} M={M}: rel L2 {r:.2e}, max abs {m:.2e}")


def test_affine_shared_prefill_width(layers, q38, orc):
    L = layers[(4, 64, 0)]
    M = 40
    x = orc.rmsnorm(orc.embed(0x5EED, list(range(300, 300 + M)), 2048))
    y, ex, wt, _, _ = run_forward(q38, L, L.qdesc, x)
    wy, wex, wwt, _ = L.oracle(orc, x)
    assert np.array_equal(ex, wex) and np.array_equal(wt, wwt)
    tol_check(orc, y, wy)


def test_affine_shared_part_alone(gpu, layers, q38, orc):
    """A layer whose router sends every route to expert 0 with all-zero codebooks computes only
    the shared part: y = T(T(down_shared) * sgate); compared with the oracle's affine expert."""
    L = layers[(8, 32, 1)]
    x = orc.rmsnorm(orc.embed(0x5EED, [1, 2, 3], 2048))
    zero_books = [G.to_dev(np.zeros(16384 * 8, np.uint16)) for _ in range(3)]
    w = q38.MoeWeights()
    w.router, w.shared_gate = L.dev[0].data_ptr(), L.dev[1].data_ptr()
    for p in range(3):
        w.codes[p] = L.dev[2 + p].data_ptr()
        w.scales[p] = L.dev[5 + p].data_ptr()
        w.books[p] = zero_books[p].data_ptr()
    a = q38.AffineShared()
    for p in range(3):
        a.weight[p], a.scales[p], a.biases[p] = L.sdev[p].data_ptr(), L.sdev[3 + p].data_ptr(), L.sdev[6 + p].data_ptr()
    a.bits, a.group, a.inter, a.scale_dtype = 8, 32, 1024, 1
    h = C.c_void_p()
    q38.check(q38.lib.q38_moe_layer_create_affine_shared(gpu.h, C.byref(L.qdesc), C.byref(w), C.byref(a),
                                                         C.byref(h)))

    class H:
        pass

    lay = H()
    lay.h = h
    try:
        y, _, _, _, _ = run_forward(q38, lay, L.qdesc, x)
    finally:
        q38.lib.q38_moe_layer_destroy(h)
    d = orc.affine_expert(L.sa, x).astype(np.float64)
    lg = orc.router_logits(x, L.wsg[None, :]).astype(np.float64)[:, 0]
    sg = orc.bf16_to_f32(orc.bf16((1.0 / (1.0 + np.exp(-lg))).astype(np.float32))).astype(np.float64)
    want = orc.bf16((d * sg[:, None]).astype(np.float32))
    tol_check(orc, y, want, rel=2e-3, mx=2e-3)
    assert np.mean(y == want) > 0.95, np.mean(y == want)


def test_affine_shared_rejects_bad_geometry(gpu, q38):
    d = q38.desc()
    w = q38.MoeWeights()
    a = q38.AffineShared()
    a.bits, a.group, a.inter, a.scale_dtype = 3, 64, 512, 0
    h = C.c_void_p()
    assert q38.lib.q38_moe_layer_create_affine_shared(gpu.h, C.byref(d), C.byref(w), C.byref(a), C.byref(h)) == \
        q38.Q38_EINVAL
    a.bits, a.group = 4, 48
    assert q38.lib.q38_moe_layer_create_affine_shared(gpu.h, C.byref(d), C.byref(w), C.byref(a), C.byref(h)) == \
        q38.Q38_EINVAL
