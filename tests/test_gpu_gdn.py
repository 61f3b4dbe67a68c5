"""The GatedDeltaNet verify step on the GPU (q38_gdn_verify; GatedDeltaNet::forward_verify,
src/gated_delta_net.cpp:657-834) against the oracle on the same weights and rows: outputs within
the MoE tolerance (rel L2 <= 1e-2, max-abs <= 2e-2), the checkpoint states (convolution rows and
recurrent state after every row) within 1e-2 rel L2; S rows in one call equal S one-row calls
chained through q38_gdn_commit, bit for bit; and the reference's geometry checks."""
import ctypes as C

import numpy as np
import pytest

import gpu_util as G
from gdn_cases import GdnLayer, bf, rel_l2
from moe_cases import tol_check

pytestmark = pytest.mark.gpu


class DevGdn:
    def __init__(self, q38, gpu, L: GdnLayer):
        self.q38, self.L = q38, L
        self.keep = []
        w = q38.GdnWeights()
        for p in range(5):
            t = [G.to_dev(L.proj["w"][p]), G.to_dev(L.proj["s"][p]), G.to_dev(L.proj["b"][p])]
            self.keep += t
            w.weight[p], w.scales[p], w.biases[p] = t[0].data_ptr(), t[1].data_ptr(), t[2].data_ptr()
        t = [G.to_dev(L.conv_w), G.to_dev(L.a_log), G.to_dev(L.dt_bias), G.to_dev(L.norm_w)]
        self.keep += t
        w.conv, w.a_log, w.dt_bias, w.norm = (a.data_ptr() for a in t)
        d = q38.GdnDesc(L.hidden, L.hk, L.hv, L.dk, L.dv, 4, L.bits, L.group, L.fmt, L.gate_silu, L.eps)
        self.h = C.c_void_p()
        q38.check(q38.lib.q38_gdn_create(gpu.h, C.byref(d), C.byref(w), C.byref(self.h)))
        assert q38.lib.q38_gdn_state_bytes(self.h) == 2 * L.state_elems
        self.ws = G.workspace(q38.lib.q38_gdn_workspace_size(self.h, 64))

    def verify(self, x, origin=None, state_dev=None):
        """-> (out [S, H] bf16 bits, checkpoints [S, state_elems] bf16 bits, checkpoint device buffer)."""
        q38, L = self.q38, self.L
        S = x.shape[0]
        xd = G.to_dev(x)
        od = state_dev if state_dev is not None else (None if origin is None else G.to_dev(origin))
        ck = G.empty((S, L.state_elems), np.uint16)
        out = G.empty((S, L.hidden), np.uint16)
        q38.check(q38.lib.q38_gdn_verify(self.h, xd.data_ptr(), S, None if od is None else od.data_ptr(),
                                         ck.data_ptr(), out.data_ptr(), self.ws.data_ptr(), self.ws.numel(),
                                         G.stream()))
        return G.to_host(out, np.uint16), G.to_host(ck, np.uint16), ck

    def close(self):
        self.q38.lib.q38_gdn_destroy(self.h)


def compare(orc, L, out, ck, wout, wck):
    tol_check(orc, out, wout)
    C3 = 3 * L.C
    assert rel_l2(bf(ck[:, :C3]), bf(wck[:, :C3])) < 1e-2
    assert rel_l2(bf(ck[:, C3:]), bf(wck[:, C3:])) < 1e-2, rel_l2(bf(ck[:, C3:]), bf(wck[:, C3:]))


GEOS = {
    "q8_g64_sigmoid": dict(),
    "q4_g32_f16_silu": dict(bits=4, group=32, fmt=1, gate_silu=1, seed=1),
    "one_value_head_per_key": dict(hk=4, hv=4, seed=2),
    "dk64": dict(dk=64, dv=64, hk=2, hv=8, seed=3),
}


@pytest.mark.parametrize("geo", list(GEOS))
@pytest.mark.parametrize("S", [1, 4, 16])
def test_verify_vs_oracle(gpu, q38, orc, geo, S):
    L = GdnLayer(**GEOS[geo])
    dev = DevGdn(q38, gpu, L)
    try:
        rng = np.random.default_rng(10 + S)
        x = orc.bf16(rng.normal(0, 1, (S, L.hidden)).astype(np.float32))
        for origin in (None, L.random_state(rng)):
            out, ck, _ = dev.verify(x, origin)
            wout, wck = orc.gdn_verify(L, x, origin)
            compare(orc, L, out, ck, wout, wck)
    finally:
        dev.close()


def test_full_size_layer(gpu, q38, orc):
    """The family's geometry: hidden 2048, 16 key and 32 value heads of 128, Q8/g64."""
    L = GdnLayer(hidden=2048, hk=16, hv=32, seed=4)
    dev = DevGdn(q38, gpu, L)
    try:
        rng = np.random.default_rng(4)
        x = orc.bf16(rng.normal(0, 1, (4, L.hidden)).astype(np.float32))
        origin = L.random_state(rng)
        out, ck, _ = dev.verify(x, origin)
        wout, wck = orc.gdn_verify(L, x, origin)
        compare(orc, L, out, ck, wout, wck)
    finally:
        dev.close()


def test_rows_chain_through_commit(gpu, q38, orc):
    """S rows in one call equal S one-row calls, each from the state q38_gdn_commit made of the
    previous call's checkpoint, bit for bit (outputs and checkpoints)."""
    L = GdnLayer(seed=5)
    dev = DevGdn(q38, gpu, L)
    try:
        rng = np.random.default_rng(5)
        x = orc.bf16(rng.normal(0, 1, (5, L.hidden)).astype(np.float32))
        origin = L.random_state(rng)
        out, ck, _ = dev.verify(x, origin)
        state = G.to_dev(origin)
        for t in range(5):
            o1, c1, cdev = dev.verify(x[t:t + 1], state_dev=state)
            assert np.array_equal(o1[0], out[t]) and np.array_equal(c1[0], ck[t]), t
            q38.check(q38.lib.q38_gdn_commit(dev.h, cdev.data_ptr(), 0, state.data_ptr(), G.stream()))
        # a commit of an earlier row: the state equals that row's checkpoint
        _, ck2, cdev2 = dev.verify(x[:3], origin)
        q38.check(q38.lib.q38_gdn_commit(dev.h, cdev2.data_ptr(), 1, state.data_ptr(), G.stream()))
        assert np.array_equal(G.to_host(state, np.uint16), ck2[1])
    finally:
        dev.close()


def test_geometry_checks(gpu, q38):
    L = GdnLayer()
    dev = DevGdn(q38, gpu, L)
    try:
        w = q38.GdnWeights()
        for p in range(5):
            w.weight[p] = w.scales[p] = w.biases[p] = 1
        w.conv = w.a_log = w.dt_bias = w.norm = 1
        h = C.c_void_p()
        for bad, msg in ((dict(conv_kernel=3), b"convolution width 4"), (dict(value_heads=3), b"divisible by key heads"),
                         (dict(bits=3), b"bits must be"), (dict(key_dim=96, value_dim=96), b"key_dim = value_dim")):
            f = dict(hidden=512, key_heads=2, value_heads=4, key_dim=128, value_dim=128, conv_kernel=4, bits=8, group=64,
                     scale_dtype=0, gate_silu=0, eps=1e-6)
            f.update(bad)
            d = q38.GdnDesc(**f)
            assert q38.lib.q38_gdn_create(gpu.h, C.byref(d), C.byref(w), C.byref(h)) == q38.Q38_EINVAL
            assert msg in q38.lib.q38_last_error(), (bad, q38.lib.q38_last_error())
        x = G.empty((65, L.hidden), np.uint16)
        out = G.empty((65, L.hidden), np.uint16)
        assert q38.lib.q38_gdn_verify(dev.h, x.data_ptr(), 65, None, None, out.data_ptr(), dev.ws.data_ptr(),
                                      dev.ws.numel(), G.stream()) == q38.Q38_EINVAL
        assert b"S=1..64" in q38.lib.q38_last_error()
    finally:
        dev.close()
