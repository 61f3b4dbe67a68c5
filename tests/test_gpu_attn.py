"""The full-attention verify step on the GPU (q38_attn_verify; the dense path of
SelfAttention::forward_verify, src/self_attention.cpp:1450-1720) against the oracle on the
same weights, rows and cache:
- outputs within the MoE tolerance (rel L2 <= 1e-2, max-abs <= 2e-2);
- the new keys and values in the cache within two bf16 steps of the larger of the element and
  its head vector's RMS, and within one step on almost every element;
- the rest of the cache untouched, bit for bit; unused cache slots hold 65536.0 and are never
  read (a read would show in the outputs);
- S rows in one call equal S one-row calls through the cache, bit for bit (the checkpoint of
  row r is the cache prefix);
- the closed form of the oracle's tests (a one-hot query reading one cached key) exactly;
- the reference's geometry check and the capacity and row limits."""
import ctypes as C

import numpy as np
import pytest

import gpu_util as G
from affine_cases import pack_affine, to16
from attn_cases import AttnLayer, bf, rel_l2
from moe_cases import tol_check
from test_oracle_attn import D_ID, H_ID, HQ_ID, identity_layer
from test_oracle_hc import ulp_diff

pytestmark = pytest.mark.gpu


class DevAttn:
    def __init__(self, q38, gpu, L: AttnLayer, cap, max_rows=64):
        self.q38, self.L, self.cap = q38, L, cap
        self.keep = []
        w = q38.AttnWeights()
        for p in range(4):
            t = [G.to_dev(L.proj["w"][p]), G.to_dev(L.proj["s"][p]), G.to_dev(L.proj["b"][p])]
            self.keep += t
            w.weight[p], w.scales[p], w.biases[p] = t[0].data_ptr(), t[1].data_ptr(), t[2].data_ptr()
        t = [G.to_dev(L.q_norm), G.to_dev(L.k_norm)]
        self.keep += t
        w.q_norm, w.k_norm = t[0].data_ptr(), t[1].data_ptr()
        d = q38.AttnDesc(L.hidden, L.hq, L.hkv, L.d, L.rot, L.bits, L.group, L.fmt, L.norm_offset, L.eps, L.theta)
        self.h = C.c_void_p()
        q38.check(q38.lib.q38_attn_create(gpu.h, C.byref(d), C.byref(w), C.byref(self.h)))
        assert q38.lib.q38_attn_cache_bytes(self.h, cap) == 2 * L.hkv * cap * L.d * 2
        self.ws = G.workspace(q38.lib.q38_attn_workspace_size(self.h, min(max_rows, cap), cap))

    def cache_dev(self, keys, values):
        return G.to_dev(np.concatenate([keys.reshape(-1), values.reshape(-1)]))

    def cache_host(self, dev):
        a = G.to_host(dev, np.uint16)
        n = self.L.hkv * self.cap * self.L.d
        shape = (self.L.hkv, self.cap, self.L.d)
        return a[:n].reshape(shape), a[n:].reshape(shape)

    def verify(self, x, cache, T0, position):
        S = x.shape[0]
        xd = G.to_dev(x)
        out = G.empty((S, self.L.hidden), np.uint16)
        self.q38.check(self.q38.lib.q38_attn_verify(self.h, xd.data_ptr(), S, cache.data_ptr(), self.cap, T0,
                                                    position, out.data_ptr(), self.ws.data_ptr(), self.ws.numel(),
                                                    G.stream()))
        return G.to_host(out, np.uint16)

    def close(self):
        self.q38.lib.q38_attn_destroy(self.h)


def check_cache(keys, values, k2, v2, wk, wv, T0, S):
    """New rows within two bf16 steps of the larger of the element and its head vector's RMS
    (an element much smaller than its vector carries the absolute error of the vector's sums),
    one step or less on almost all elements; the rest of the cache bit for bit."""
    for got, want, old in ((k2, wk, keys), (v2, wv, values)):
        g, wnt = bf(got[:, T0:T0 + S]).astype(np.float64), bf(want[:, T0:T0 + S]).astype(np.float64)
        rms = np.sqrt((wnt * wnt).mean(-1, keepdims=True))
        scale = np.maximum(np.abs(wnt), rms)
        assert (np.abs(g - wnt) <= scale * 2.0 ** -7).all(), np.abs(g - wnt).max()
        u = ulp_diff(got[:, T0:T0 + S], want[:, T0:T0 + S])
        assert (u > 1).mean() <= 1e-3, (u > 1).mean()
        assert np.array_equal(got[:, :T0], old[:, :T0]) and np.array_equal(got[:, T0 + S:], old[:, T0 + S:])


GEOS = {
    "q8_g64": dict(),
    "q4_g32_f16_offset": dict(bits=4, group=32, fmt=1, norm_offset=1, seed=1),
    "mqa_d64_full_rotary": dict(q_heads=8, kv_heads=1, head_dim=64, rotary_dim=64, seed=2, theta=1e4),
    "d256_gqa8": dict(hidden=1024, q_heads=16, kv_heads=2, head_dim=256, rotary_dim=64, seed=3),
}


@pytest.mark.parametrize("geo", list(GEOS))
@pytest.mark.parametrize("S,T0", [(1, 0), (4, 37), (16, 300), (4, 1000)])
def test_verify_vs_oracle(gpu, q38, orc, geo, S, T0):
    L = AttnLayer(**GEOS[geo])
    rng = np.random.default_rng(S * 1000 + T0)
    cap = T0 + S + 5
    keys, values = L.random_cache(rng, cap, T0)
    x = to16(rng.normal(0, 1, (S, L.hidden)), 0)
    dev = DevAttn(q38, gpu, L, cap)
    try:
        cache = dev.cache_dev(keys, values)
        out = dev.verify(x, cache, T0, 9000 + T0)
        k2, v2 = dev.cache_host(cache)
    finally:
        dev.close()
    wout, wk, wv = orc.attn_verify(L, x, keys, values, T0, 9000 + T0)
    tol_check(orc, out, wout)
    check_cache(keys, values, k2, v2, wk, wv, T0, S)


def test_full_size_layer(gpu, q38, orc):
    """H 2048, 16 query heads and 2 kv heads of 256, rotary 64, 8-bit g64, 4 rows over 4000
    cached tokens."""
    L = AttnLayer(hidden=2048, q_heads=16, kv_heads=2, head_dim=256, rotary_dim=64, seed=7)
    rng = np.random.default_rng(7)
    T0, S = 4000, 4
    cap = 4100
    keys, values = L.random_cache(rng, cap, T0)
    x = to16(rng.normal(0, 1, (S, L.hidden)), 0)
    dev = DevAttn(q38, gpu, L, cap)
    try:
        cache = dev.cache_dev(keys, values)
        out = dev.verify(x, cache, T0, 123456)
        k2, v2 = dev.cache_host(cache)
    finally:
        dev.close()
    wout, wk, wv = orc.attn_verify(L, x, keys, values, T0, 123456)
    tol_check(orc, out, wout)
    check_cache(keys, values, k2, v2, wk, wv, T0, S)


def test_rows_chain_through_the_cache(gpu, q38):
    L = AttnLayer(seed=5)
    rng = np.random.default_rng(5)
    T0, S, cap = 380, 6, 390   # the rows cross a 128-token P.V tile and a 64-token score tile
    keys, values = L.random_cache(rng, cap, T0)
    x = to16(rng.normal(0, 1, (S, L.hidden)), 0)
    dev = DevAttn(q38, gpu, L, cap)
    try:
        c1 = dev.cache_dev(keys, values)
        out = dev.verify(x, c1, T0, 50)
        c2 = dev.cache_dev(keys, values)
        for r in range(S):
            o1 = dev.verify(x[r:r + 1], c2, T0 + r, 50 + r)
            assert np.array_equal(o1[0], out[r]), r
        assert np.array_equal(G.to_host(c1, np.uint16), G.to_host(c2, np.uint16))
        # a rejected suffix is overwritten: verify two other rows from T0 + 2 (accepted 1)
        x2 = to16(rng.normal(0, 1, (2, L.hidden)), 0)
        o2 = dev.verify(x2, c1, T0 + 2, 52)
        c3 = dev.cache_dev(*dev.cache_host(c2))
        o3 = dev.verify(x2, c3, T0 + 2, 52)
        assert np.array_equal(o2, o3)
    finally:
        dev.close()


def test_one_hot_query_reads_its_key_exactly(gpu, q38, orc):
    j = 40
    L = identity_layer(q_rows={j: (0, 3)})
    rng = np.random.default_rng(2)
    T0, cap = 12, 16
    keys, values = L.random_cache(rng, cap, T0)
    keys[:, :T0] = 0
    keys[0, 5, j] = to16(np.array([64.0]), 0)[0]
    x = np.zeros((1, H_ID), np.uint16)
    x[0, 0] = to16(np.array([1.0]), 0)[0]
    dev = DevAttn(q38, gpu, L, cap)
    try:
        out = dev.verify(x, dev.cache_dev(keys, values), T0, 3)
    finally:
        dev.close()
    got = bf(out[0]).reshape(HQ_ID, D_ID)
    want = bf(orc.bf16((bf(values[0, 5]) * 0.5).astype(np.float32)))
    assert np.array_equal(got[0], want)
    wout, _, _ = orc.attn_verify(L, x, keys, values, T0, 3)
    assert np.array_equal(out, wout)


def test_limits_and_geometry(gpu, q38):
    L = AttnLayer(seed=6)
    dev = DevAttn(q38, gpu, L, 32)
    lib = q38.lib
    try:
        cache = G.workspace(lib.q38_attn_cache_bytes(dev.h, 32))
        x = G.to_dev(np.zeros((65, L.hidden), np.uint16))
        out = G.empty((65, L.hidden), np.uint16)
        assert lib.q38_attn_verify(dev.h, x.data_ptr(), 65, cache.data_ptr(), 32, 0, 0, out.data_ptr(),
                                   dev.ws.data_ptr(), dev.ws.numel(), G.stream()) == q38.Q38_EINVAL
        assert b"S=1..64" in lib.q38_last_error()
        assert lib.q38_attn_verify(dev.h, x.data_ptr(), 4, cache.data_ptr(), 32, 29, 0, out.data_ptr(),
                                   dev.ws.data_ptr(), dev.ws.numel(), G.stream()) == q38.Q38_ERANGE
        assert lib.q38_attn_verify(dev.h, x.data_ptr(), 4, cache.data_ptr(), 32, 8, 0, out.data_ptr(),
                                   dev.ws.data_ptr(), 1024, G.stream()) == q38.Q38_ESPACE
    finally:
        dev.close()
    assert lib.q38_attn_workspace_size(None, 4, 100) == 0
    for bad, msg in ((dict(q_heads=3, kv_heads=2), b"unsupported attention head/rotary configuration"),
                     (dict(rotary_dim=31), b"unsupported attention head/rotary configuration"),
                     (dict(rotary_dim=256), b"unsupported attention head/rotary configuration"),
                     (dict(head_dim=96, rotary_dim=32), b"64, 128 or 256")):
        g = dict(hidden=512, q_heads=4, kv_heads=2, head_dim=128, rotary_dim=32)
        g.update(bad)
        d = q38.AttnDesc(g["hidden"], g["q_heads"], g["kv_heads"], g["head_dim"], g["rotary_dim"], 8, 64, 0, 0,
                         1e-6, 1e6)
        w = q38.AttnWeights()
        for p in range(4):
            w.weight[p] = w.scales[p] = w.biases[p] = dev.keep[0].data_ptr()
        w.q_norm = w.k_norm = dev.keep[0].data_ptr()
        h = C.c_void_p()
        assert lib.q38_attn_create(gpu.h, C.byref(d), C.byref(w), C.byref(h)) == q38.Q38_EINVAL
        assert msg in lib.q38_last_error(), (bad, lib.q38_last_error())
