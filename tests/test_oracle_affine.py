"""The oracle's affine shared expert (SparseMoe::forward_shared over MLX affine weights,
src/sparse_moe.cpp:662-700, 1306-1313), pinned by an independent float64 numpy restatement
over dequantized weights, by closed forms that fix the packing order (LSB-first values), the
scale / bias roles and the group index, and by the composition of a layer with an affine shared
expert from the same layer without one."""
import numpy as np
import pytest

import oracle_lib
from affine_cases import dequant, np_affine_expert, pack_affine, random_affine, to16
from moe_cases import bf16_ulps


@pytest.mark.parametrize("bits,group,fmt", [(4, 64, 0), (8, 64, 1), (2, 32, 0), (4, 128, 1)])
def test_affine_expert_vs_numpy(orc, bits, group, fmt):
    rng = np.random.default_rng(bits * 100 + group + fmt)
    H, Is = 512, 256
    sa = random_affine(rng, H, Is, bits, group, fmt)
    x = orc.bf16(rng.normal(0, 1, (3, H)))
    got = orc.affine_expert(sa, x)
    want = np_affine_expert(orc, sa, x)
    gb, wb = orc.bf16(got), orc.bf16(want)
    ulps = bf16_ulps(orc, gb, wb)
    assert ulps.max() <= 1 and np.mean(ulps == 0) > 0.99, (ulps.max(), np.mean(ulps == 0))


def test_affine_closed_forms(orc):
    """Down projection set to the identity-like map below reads the SwiGLU row back, so the
    gate / up rows can be fixed value by value."""
    rng = np.random.default_rng(5)
    H, Is, bits, group, fmt = 256, 128, 4, 64, 0
    sa = random_affine(rng, H, Is, bits, group, fmt)
    x = orc.bf16(rng.normal(0, 1, (2, H)))
    xf = orc.bf16_to_f32(x).astype(np.float64)
    # gate row o: one value q = 1 at input 2o + 1 (the second value of its word), scale 1, bias 0
    # -> g = x[2o + 1]; up row o: all values 0, bias 1 in group 0 only -> u = sum of x[0:64]
    qg = np.zeros((Is, H), np.int64)
    qg[np.arange(Is), 2 * np.arange(Is) + 1] = 1
    sa["q"][0] = qg
    sa["w"][0] = pack_affine(qg, bits)
    sa["s"][0] = to16(np.ones((Is, H // group)), fmt)
    sa["b"][0] = to16(np.zeros((Is, H // group)), fmt)
    sa["q"][1] = np.zeros((Is, H), np.int64)
    sa["w"][1] = pack_affine(sa["q"][1], bits)
    sa["s"][1] = to16(rng.uniform(1, 2, (Is, H // group)), fmt)
    bias = np.zeros((Is, H // group))
    bias[:, 0] = 1.0
    sa["b"][1] = to16(bias, fmt)
    # down: row o takes h[o mod Is] with q = 1, scale 1 (value 1), bias 0
    qd = np.zeros((H, Is), np.int64)
    qd[np.arange(H), np.arange(H) % Is] = 1
    sa["q"][2] = qd
    sa["w"][2] = pack_affine(qd, bits)
    sa["s"][2] = to16(np.ones((H, Is // group)), fmt)
    sa["b"][2] = to16(np.zeros((H, Is // group)), fmt)
    got = orc.affine_expert(sa, x).astype(np.float64)
    T = lambda v: orc.bf16_to_f32(orc.bf16(np.asarray(v, np.float32))).astype(np.float64)
    g = T(xf[:, 1::2][:, :Is])
    u = T(np.repeat(xf[:, :64].sum(1, keepdims=True), Is, 1))
    h = T(T(g / (1 + np.exp(-g))) * u)
    want = T(h[:, np.arange(H) % Is])
    assert np.array_equal(got, want)
    # a planted nibble-order mistake (value j at bit 28 - 4j) moves every gate input
    bad = np.zeros_like(sa["w"][0])
    for j in range(8):
        bad |= ((sa["w"][0] >> np.uint32(4 * j)) & np.uint32(0xF)) << np.uint32(28 - 4 * j)
    sa["w"][0] = bad
    assert not np.array_equal(orc.affine_expert(sa, x).astype(np.float64), want)


def test_affine_dequant_matches_formula(orc):
    rng = np.random.default_rng(6)
    sa = random_affine(rng, 128, 64, 8, 32, 1)
    W = dequant(sa, 0)
    o, c = 7, 45
    want = float(np.float16(sa["s"][0].view(np.float16)[o, c // 32])) * sa["q"][0][o, c] + \
        float(sa["b"][0].view(np.float16)[o, c // 32])
    assert W[o, c] == want


def test_layer_with_affine_shared_composes(orc):
    """y(affine-shared layer) = T(T(routed) + T(T(down_shared) * sgate)): the routed part from the
    same layer without a shared expert, the shared part from the affine expert alone, the gate
    T(sigmoid(T(x . w_sg)))."""
    rng = np.random.default_rng(7)
    H, I, E, k = 512, 128, 64, 4
    d_sh = oracle_lib.make_desc(hidden=H, inter=I, experts=E, top_k=k)
    d_no = oracle_lib.make_desc(hidden=H, inter=I, experts=E, top_k=k, shared=0)
    router = orc.bf16(rng.normal(0, 0.02, (E, H)))
    wsg = orc.bf16(rng.normal(0, 0.5, H))
    books, codes, scales = [], [], []
    for p, (IN, OUT) in enumerate(((H, I), (H, I), (I, H))):
        books.append(to16(rng.normal(0, 1, 16384 * 8), 1))
        raw = rng.integers(0, 1 << 14, (E * OUT, IN // 8)).astype(np.uint32)
        codes.append(np.stack([orc.pack_row(r, 14) for r in raw]).reshape(-1))
        scales.append(to16(rng.uniform(0.005, 0.02, E * OUT), 1))
    sa = random_affine(rng, H, 192, 4, 64, 0)
    x = orc.bf16(rng.normal(0, 1, (4, H)))
    y, ex, wt, _ = orc.moe_layer_dense_affine_shared(d_sh, router, wsg, codes, scales, books, sa, x)
    y0, ex0, wt0, _ = orc.moe_layer_dense(d_no, router, wsg, codes, scales, books, x)
    assert np.array_equal(ex, ex0) and np.array_equal(wt, wt0)
    dsh = orc.affine_expert(sa, x).astype(np.float64)
    lg = orc.router_logits(x, wsg[None, :]).astype(np.float64)[:, 0]
    sg = orc.bf16_to_f32(orc.bf16((1.0 / (1.0 + np.exp(-lg))).astype(np.float32))).astype(np.float64)
    T = lambda v: orc.bf16(np.asarray(v, np.float64).astype(np.float32))
    sh = orc.bf16_to_f32(T(dsh * sg[:, None])).astype(np.float64)
    want = T(orc.bf16_to_f32(y0).astype(np.float64) + sh)
    assert np.array_equal(y, want)
