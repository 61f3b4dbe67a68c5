"""VQ decode + expert SwiGLU + MoE layer (R5-R11) of the CPU oracle against closed-form
banks restated from tests/vq_geometry_gpu_test.cpp:24-57 and an independent float64 numpy
recomputation."""
import numpy as np

import oracle_lib


def rb(orc, v):
    return orc.bf16_to_f32(orc.bf16(np.asarray(v, np.float32)))


def f16(v):
    return np.asarray(v, np.float32).astype(np.float16).view(np.uint16)


def closed_bank(orc, n_in, n_out, experts, d, bits, seed, group):
    # book[i] = ((i*17+seed)%31-15)/64, scale = (1+(i*7+seed)%4)/16, code = (r*73+s*251+seed)%K
    K = 1 << bits
    nsub = n_in // d
    book = np.array([((i * 17 + seed) % 31 - 15) / 64 for i in range(K * d)], np.float32)
    ngrp = n_in // group
    scales = np.array([(1 + (i * 7 + seed) % 4) / 16 for i in range(experts * n_out * ngrp)], np.float32)
    codes = np.array([[(r * 73 + s * 251 + seed) % K for s in range(nsub)] for r in range(experts * n_out)],
                     np.uint32)
    words = np.stack([orc.pack_row(c, bits) for c in codes])
    dense = np.zeros((experts * n_out, n_in))
    for r in range(experts * n_out):
        w = book.reshape(K, d)[codes[r]].reshape(-1).astype(np.float64)
        dense[r] = w * np.repeat(scales.reshape(-1, ngrp)[r], group)
    return f16(book), words.reshape(-1), f16(scales), dense


def np_expert(orc, dense_g, dense_u, dense_d, x):
    g = rb(orc, dense_g @ x)
    u = rb(orc, dense_u @ x)
    s = rb(orc, g / (1 + np.exp(-g.astype(np.float64))))
    h = rb(orc, s.astype(np.float64) * u)
    return rb(orc, dense_d @ h.astype(np.float64))


def test_expert_closed_form_banks(orc):
    for (d, bits), group in [((8, 14), 64), ((4, 8), 64), ((8, 14), 512)]:
        H, I, E = 512, 128, 3
        desc = oracle_lib.make_desc(hidden=H, inter=I, experts=64, top_k=4, gu=(d, bits), down=(d, bits),
                                    gu_group=group, down_group=min(group, I))
        gb, gw, gs, gd = closed_bank(orc, H, I, E, d, bits, 3, group)
        ub, uw, us, ud = closed_bank(orc, H, I, E, d, bits, 11, group)
        db, dw, ds, dd = closed_bank(orc, I, H, E, d, bits, 19, min(group, I))
        x = orc.bf16(np.array([((i * 13) % 17 - 8) / 32 for i in range(2 * H)], np.float32).reshape(2, H))
        import ctypes as C
        keep = [gw, uw, dw, gs, us, ds, gb, ub, db]
        arr = lambda xs: (C.c_void_p * 3)(*[a.ctypes.data for a in xs])
        for e in range(E):
            out = np.zeros((2, H), np.float32)
            rc = orc.lib.orc_expert_dense(C.byref(desc), arr(keep[0:3]), arr(keep[3:6]), arr(keep[6:9]), e,
                                          x.ctypes.data, 2, out.ctypes.data)
            assert rc == 0
            for r in range(2):
                xr = orc.bf16_to_f32(x[r]).astype(np.float64)
                want = np_expert(orc, gd[e * I:(e + 1) * I], ud[e * I:(e + 1) * I], dd[e * H:(e + 1) * H], xr)
                assert np.array_equal(out[r], want), (d, bits, group, e, r)


def test_zero_codebook_gives_zero(orc):
    H, I, E = 512, 128, 64
    desc = oracle_lib.make_desc(hidden=H, inter=I, experts=E, top_k=4)
    rng = np.random.default_rng(0)
    router = orc.bf16(rng.normal(0, 0.02, (E, H)))
    wsg = orc.bf16(rng.normal(0, 0.02, H))
    codes = [rng.integers(0, 2**32, (E + 1) * n_out * w, dtype=np.uint64).astype(np.uint32)
             for n_out, w in ((I, 28), (I, 28), (H, 14))]  # 16 codes per down row fill one 14-word block
    scales = [f16(rng.uniform(0.005, 0.02, (E + 1) * n)) for n in (I, I, H)]
    books = [np.zeros(16384 * 8, np.uint16)] * 3
    x = orc.bf16(rng.normal(0, 1, (3, H)))
    y, ex, wt, lg = orc.moe_layer_dense(desc, router, wsg, codes, scales, books, x)
    assert (orc.bf16_to_f32(y) == 0).all()
    assert ex.shape == (3, 4) and np.allclose(wt.sum(1), 1, atol=1e-6)


def test_moe_layer_vs_numpy(orc):
    H, I, E, k = 512, 128, 64, 4
    desc = oracle_lib.make_desc(hidden=H, inter=I, experts=E, top_k=k)
    rng = np.random.default_rng(5)
    router = orc.bf16(rng.normal(0, 0.02, (E, H)))
    wsg = orc.bf16(rng.normal(0, 0.02, H))
    bk = [f16(rng.normal(0, 1, 16384 * 8)) for _ in range(3)]
    nsub = (H // 8, H // 8, I // 8)
    outs = (I, I, H)
    raw = [rng.integers(0, 16384, ((E + 1) * outs[p], nsub[p])).astype(np.uint32) for p in range(3)]
    codes = [np.stack([orc.pack_row(r, 14) for r in raw[p]]).reshape(-1) for p in range(3)]
    scl = [f16(rng.uniform(0.005, 0.02, (E + 1) * outs[p])) for p in range(3)]
    x = orc.bf16(rng.normal(0, 1, (4, H)))
    y, ex, wt, lg = orc.moe_layer_dense(desc, router, wsg, codes, scl, bk, x)

    def dense(p, e):
        book = bk[p].view(np.float16).astype(np.float64).reshape(16384, 8)
        s = scl[p].view(np.float16).astype(np.float64).reshape(E + 1, outs[p])[e]
        w = book[raw[p][e * outs[p]:(e + 1) * outs[p]]].reshape(outs[p], -1)
        return w * s[:, None]

    xf = orc.bf16_to_f32(x).astype(np.float64)
    want = np.zeros((4, H))
    for r in range(4):
        routed = sum(wt[r, s] * np_expert(orc, dense(0, ex[r, s]), dense(1, ex[r, s]), dense(2, ex[r, s]), xf[r])
                     for s in range(k))
        sh_out = np_expert(orc, dense(0, E), dense(1, E), dense(2, E), xf[r])
        g = rb(orc, 1 / (1 + np.exp(-rb(orc, xf[r] @ orc.bf16_to_f32(wsg)))))
        want[r] = rb(orc, rb(orc, routed) + rb(orc, sh_out * g))
    got = orc.bf16_to_f32(y).astype(np.float64)
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel < 2e-3 and np.abs(got - want).max() < 2e-3, rel


def test_mixed_layer_vs_numpy(orc):
    """Mixed geometry (config 4): even experts (and the shared expert E) d4/8-bit with an
    fp16 [256, 4] book, odd experts d8/14-bit with an INT8 [16384, 8] book and one fp16
    scale per book (q = clamp(rint(v / s), -127, 127), value q * s). The oracle's synthetic
    layer against a float64 numpy recomputation from the generator streams."""
    H, I, E, k, seed, layer = 512, 128, 64, 4, 77, 3
    desc = oracle_lib.make_desc(hidden=H, inter=I, experts=E, top_k=k, mixed=1)
    K = lambda t: orc.key(seed, layer, t)
    x = orc.bf16(np.random.default_rng(9).normal(0, 1, (2, H)))
    y, ex, wt, lg = orc.moe_layer_synth(desc, seed, layer, x)
    outs, ins = (I, I, H), (H, H, I)
    book4 = [orc.normal(K(12 + p), 0, 256 * 4, 1.0, f16=True).view(np.float16).astype(np.float64).reshape(256, 4)
             for p in range(3)]
    book8 = []
    for p in range(3):
        v = orc.normal(K(3 + p), 0, 16384 * 8, 1.0, f16=True).view(np.float16).astype(np.float32)
        s = np.float32(np.float16(np.abs(v).max() / np.float32(127)))
        q = np.clip(np.rint(v / s), -127, 127)
        assert q.min() >= -127 and q.max() <= 127 and np.abs(q).max() == 127
        book8.append((q.astype(np.float64) * np.float64(s)).reshape(16384, 8))

    def unpack_rows(words, n, bits):  # LSB-first 32-code blocks of `bits` words
        i = np.arange(n)
        bit = (i % 32) * bits
        w = (i // 32) * bits + bit // 32
        sh = (bit % 32).astype(np.uint64)
        wp = np.concatenate([words, np.zeros((words.shape[0], 1), np.uint32)], 1).astype(np.uint64)
        v = (wp[:, w] >> sh) | (wp[:, w + 1] << (np.uint64(32) - sh))
        return (v & np.uint64((1 << bits) - 1)).astype(np.int64)

    def dense(p, e):
        d4 = e % 2 == 0
        dim, bits, book = (4, 8, book4[p]) if d4 else (8, 14, book8[p])
        codes = unpack_rows(orc.code_rows(K(6 + p), e, outs[p], 0, outs[p], ins[p] // dim, bits), ins[p] // dim, bits)
        sc = orc.uniform_f16(K(9 + p), e * outs[p], outs[p], 0.005, 0.02).view(np.float16).astype(np.float64)
        return book[codes].reshape(outs[p], -1) * sc[:, None]

    wsg = orc.bf16_to_f32(orc.normal(K(2), 0, H, 0.02))
    xf = orc.bf16_to_f32(x).astype(np.float64)
    want = np.zeros((2, H))
    for r in range(2):
        routed = sum(wt[r, s] * np_expert(orc, dense(0, ex[r, s]), dense(1, ex[r, s]), dense(2, ex[r, s]), xf[r])
                     for s in range(k))
        sh_out = np_expert(orc, dense(0, E), dense(1, E), dense(2, E), xf[r])
        g = rb(orc, 1 / (1 + np.exp(-rb(orc, xf[r] @ wsg))))
        want[r] = rb(orc, rb(orc, routed) + rb(orc, sh_out * g))
    assert {e % 2 for e in ex.reshape(-1)} == {0, 1}  # both geometries routed
    got = orc.bf16_to_f32(y).astype(np.float64)
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel < 2e-3 and np.abs(got - want).max() < 2e-3, rel


def test_thread_pool_is_deterministic(orc):
    """The pooled oracle gives the same bits on 1, 3 and 8 threads, and repeated timed passes
    reproduce the single-pass result (routes are independent items; the route reduce is serial)."""
    desc = oracle_lib.make_desc(hidden=512, inter=128, experts=64, top_k=4)
    x = orc.bf16(np.random.default_rng(9).normal(0, 1, (4, 512)))
    ref = orc.moe_layer_synth(desc, 7, 2, x, threads=1)[0]
    for t in (3, 8):
        assert np.array_equal(orc.moe_layer_synth(desc, 7, 2, x, threads=t)[0], ref)
    y, sec = orc.moe_layer_synth_reps(desc, 7, 2, x, threads=(8, 1), warm=1, reps=3)
    assert np.array_equal(y, ref)
    assert sec.shape == (2, 3) and (sec > 0).all()
