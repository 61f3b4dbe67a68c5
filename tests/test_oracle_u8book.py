"""Per-dimension INT8/U8 codebooks (R6): the reference's verify-width codebook derivation
SparseMoe::prepare_u8_codebook (src/sparse_moe.cpp:750-804) and its float decode
(src/vq_metal_kernels.hpp:564-579), restated by the oracle. Pinned by closed forms (min/max
round trip, lround ties away from zero, clamps, a constant dimension) and by a float64 numpy
recomputation of a whole layer whose d8 projections use the format (gate centred INT8,
up/down affine U8, src/sparse_moe.cpp:528-544)."""
import numpy as np
import pytest

import oracle_lib
from test_oracle_moe import np_expert, rb

K, D = 16384, 8


def f16(v):
    return np.asarray(v, np.float32).astype(np.float16).view(np.uint16)


def np_prepare(book16, centered):
    """Independent restatement (numpy): per-dim min/max, float scale, lround = half away."""
    v = book16.view(np.float16).astype(np.float32).reshape(-1, D)
    mn, mx = v.min(0), v.max(0)
    sc = ((mx - mn) / np.float32(255.0)).astype(np.float32)
    sc = np.where(sc > 0, sc, np.float32(1.0)).astype(np.float32)
    t = (v / sc) if centered else ((v - mn) / sc)
    r = np.sign(t) * np.floor(np.abs(t).astype(np.float64) + 0.5)  # lround: ties away from zero
    q = np.clip(r, -128, 127) if centered else np.clip(r, 0, 255)
    s16, b16 = f16(sc), f16(mn)
    w = q.astype(np.float32) * s16.view(np.float16).astype(np.float32)
    if not centered:
        w = (w + b16.view(np.float16).astype(np.float32)).astype(np.float32)
    return q.astype(np.int32).reshape(-1), s16, b16, w.reshape(-1)


@pytest.mark.parametrize("centered", [True, False])
def test_u8_book_vs_numpy(orc, centered):
    rng = np.random.default_rng(7 + centered)
    book = f16(rng.normal(0, 1, K * D) * np.repeat(rng.uniform(0.2, 3, D)[None], K, 0).reshape(-1))
    q, s16, b16, vals = orc.prepare_u8_book(book, K, D, centered)
    nq, ns, nb, nw = np_prepare(book, centered)
    assert np.array_equal(q, nq) and np.array_equal(s16, ns) and np.array_equal(b16, nb)
    assert np.array_equal(vals, nw)
    assert q.min() >= (-128 if centered else 0) and q.max() <= (127 if centered else 255)


def test_u8_book_closed_forms(orc):
    # dim 0 spans [0, 255] with step 0.5 around: scale 1 exactly, so v = k + 0.5 rounds away
    # from zero (lround, not rint); dim 1 is constant (scale 0 -> 1); dim 2 spans
    # [-127.5, 127.5] (centred: q = lround(v), clamped at 127); dims 3..7 are random.
    rng = np.random.default_rng(3)
    v = rng.normal(0, 1, (K, D)).astype(np.float32)
    v[:, 0] = np.tile(np.arange(0, 255.5, 0.5, dtype=np.float32), K // 511 + 1)[:K]
    v[:2, 0] = [0.0, 255.0]
    v[:, 1] = 0.75
    v[:, 2] = np.tile(np.arange(-127.5, 128.0, 0.5, dtype=np.float32), K // 511 + 1)[:K]
    v[:2, 2] = [-127.5, 127.5]
    book = f16(v)
    vf = book.view(np.float16).astype(np.float32).reshape(K, D)
    qa, sa, ba, wa = orc.prepare_u8_book(book, K, D, False)
    qa, wa = qa.reshape(K, D), wa.reshape(K, D)
    s0 = sa.view(np.float16).astype(np.float32)
    assert s0[0] == 1.0 and s0[1] == 1.0                          # (255 - 0) / 255; constant dim
    half = (vf[:, 0] % 1) == 0.5
    assert np.array_equal(qa[half, 0], (vf[half, 0] + 0.5).astype(np.int32))   # 2.5 -> 3, not 2
    assert np.all(qa[:, 1] == 0) and np.all(wa[:, 1] == np.float32(0.75))      # affine: q 0, w = min
    for d in range(D):                                            # min -> q 0 (w = f16(min)), max -> q 255
        lo, hi = np.argmin(vf[:, d]), np.argmax(vf[:, d])
        assert qa[lo, d] == 0 and wa[lo, d] == ba.view(np.float16).astype(np.float32)[d]
        if d != 1:
            assert qa[hi, d] == 255
    qc, sc, bc, wc = orc.prepare_u8_book(book, K, D, True)
    qc = qc.reshape(K, D)
    assert sc.view(np.float16).astype(np.float32)[2] == 1.0
    h2 = (vf[:, 2] % 1) == 0.5
    want = np.clip(np.sign(vf[h2, 2]) * np.floor(np.abs(vf[h2, 2]) + 0.5), -128, 127)
    assert np.array_equal(qc[h2, 2], want.astype(np.int32))       # -2.5 -> -3, 127.5 -> 127 (clamp)
    assert qc[:, 2].max() == 127 and qc[:, 2].min() == -128
    assert np.all(qc[:, 1] == 1)                                  # centred constant dim: lround(0.75) = 1


def test_layer_with_u8_books_vs_numpy(orc):
    """A whole layer (dense tensors) with book_format 2: the oracle against float64 numpy with
    the numpy-derived books (gate centred, up and down affine)."""
    H, I, E, k = 512, 128, 64, 4
    desc = oracle_lib.make_desc(hidden=H, inter=I, experts=E, top_k=k, book_format=2)
    rng = np.random.default_rng(11)
    router = orc.bf16(rng.normal(0, 0.02, (E, H)))
    wsg = orc.bf16(rng.normal(0, 0.02, H))
    bk = [f16(rng.normal(0, 1, K * D)) for _ in range(3)]
    nsub, outs = (H // 8, H // 8, I // 8), (I, I, H)
    raw = [rng.integers(0, K, ((E + 1) * outs[p], nsub[p])).astype(np.uint32) for p in range(3)]
    codes = [np.stack([orc.pack_row(r, 14) for r in raw[p]]).reshape(-1) for p in range(3)]
    scl = [f16(rng.uniform(0.005, 0.02, (E + 1) * outs[p])) for p in range(3)]
    x = orc.bf16(rng.normal(0, 1, (3, H)))
    y, ex, wt, lg = orc.moe_layer_dense(desc, router, wsg, codes, scl, bk, x)
    books = [np_prepare(bk[p], p == 0)[3].astype(np.float64).reshape(K, D) for p in range(3)]

    def dense(p, e):
        s = scl[p].view(np.float16).astype(np.float64).reshape(E + 1, outs[p])[e]
        return books[p][raw[p][e * outs[p]:(e + 1) * outs[p]]].reshape(outs[p], -1) * s[:, None]

    xf = orc.bf16_to_f32(x).astype(np.float64)
    want = np.zeros((3, H))
    for r in range(3):
        routed = sum(wt[r, s] * np_expert(orc, dense(0, ex[r, s]), dense(1, ex[r, s]), dense(2, ex[r, s]), xf[r])
                     for s in range(k))
        sh_out = np_expert(orc, dense(0, E), dense(1, E), dense(2, E), xf[r])
        g = rb(orc, 1 / (1 + np.exp(-rb(orc, xf[r] @ orc.bf16_to_f32(wsg)))))
        want[r] = rb(orc, rb(orc, routed) + rb(orc, sh_out * g))
    got = orc.bf16_to_f32(y).astype(np.float64)
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel < 2e-3 and np.abs(got - want).max() < 2e-3, rel
    # the per-dim book changes the layer against the FP16 books (the format is in effect)
    y16, _, _, _ = orc.moe_layer_dense(oracle_lib.make_desc(hidden=H, inter=I, experts=E, top_k=k), router, wsg,
                                       codes, scl, bk, x)
    assert not np.array_equal(y16, y)
