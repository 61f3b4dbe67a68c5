"""Device-generated synthetic tensors equal the oracle's generator bit for bit."""
import numpy as np
import pytest

import gpu_util as G

SEED = 0x51A5EED

pytestmark = pytest.mark.gpu


def test_layer_tensors_match_oracle(gpu, q38, orc):
    d = q38.desc()
    L = q38.MoeLayer(gpu, d, seed=SEED, layer=3)
    w = L.weights()
    try:
        H, I, E = 2048, 512, 512
        router = G.d2h(w.router, (E, H), np.uint16)
        assert np.array_equal(router, orc.normal(orc.key(SEED, 3, 1), 0, E * H, 0.02).reshape(E, H))
        assert np.array_equal(G.d2h(w.shared_gate, H, np.uint16), orc.normal(orc.key(SEED, 3, 2), 0, H, 0.02))
        for p, tb in enumerate((3, 4, 5)):
            book = G.d2h(w.books[p], 16384 * 8, np.uint16)
            assert np.array_equal(book, orc.normal(orc.key(SEED, 3, tb), 0, 16384 * 8, 1.0, f16=True))
        for p, (tc, ts, n_in, n_out) in enumerate(((6, 9, H, I), (7, 10, H, I), (8, 11, I, H))):
            words = ((n_in // 8 + 31) // 32) * 14
            for e in (0, 17, 511, 512):
                got = G.d2h(w.codes[p] + (e * n_out) * words * 4, (4, words), np.uint32)
                want = orc.code_rows(orc.key(SEED, 3, tc), e, n_out, 0, 4, n_in // 8, 14)
                assert np.array_equal(got, want), (p, e)
            sc = G.d2h(w.scales[p], (E + 1) * n_out, np.uint16)
            assert np.array_equal(sc, orc.uniform_f16(orc.key(SEED, 3, ts), 0, (E + 1) * n_out, 0.005, 0.02))
    finally:
        L.close()


def test_embed_matches_oracle(gpu, q38, orc):
    import ctypes as C
    toks = [0, 5, 151935, 77]
    h = G.empty((4, 2048), np.uint16)
    arr = (C.c_uint32 * 4)(*toks)
    q38.check(q38.lib.q38_embed_synthetic(SEED, arr, 4, 2048, h.data_ptr(), G.stream()))
    assert np.array_equal(G.to_host(h, np.uint16), orc.embed(SEED, toks, 2048))
    h2 = G.empty((4, 2048), np.uint16)
    td = G.to_dev(np.array(toks, np.uint32))
    q38.check(q38.lib.q38_embed_synthetic_dev(SEED, td.data_ptr(), 4, 2048, h2.data_ptr(), G.stream()))
    assert np.array_equal(G.to_host(h2, np.uint16), orc.embed(SEED, toks, 2048))


def test_head_tensors_match_oracle(gpu, q38, orc):
    hd = q38.Head(gpu, q38.Q38_HEAD_Q8, 151936, 2048, seed=SEED)
    try:
        wp, sp = hd.device_weights()
        rows = [0, 1, 77777, 151935]
        for v in rows:
            got = G.d2h(wp + v * 2048, 2048, np.int8)
            want = np.empty(2048, np.int8)
            orc.lib.orc_gen_int8(orc.key(SEED, 0xFFFE, 30), v * 2048, 2048, want.ctypes.data)
            assert np.array_equal(got, want)
        s = G.d2h(sp, 151936, np.uint16)
        assert np.array_equal(s, orc.uniform_f16(orc.key(SEED, 0xFFFE, 31), 0, 151936, 1e-4, 1e-3))
    finally:
        hd.close()
