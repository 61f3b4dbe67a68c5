"""Shared builders for the GPU MoE parity tests."""
from __future__ import annotations

import ctypes as C

import numpy as np

import gpu_util as G

SEED = 0x51A5EED


def f16(v):
    return np.asarray(v, np.float32).astype(np.float16).view(np.uint16)


def pack_q4(w):
    """[V, H] ints in [-8, 7] -> [V, H/2] bytes: input 2i in the low nibble, 2i + 1 in the
    high nibble (the Q4/g64 head's tensor contract)."""
    u = (np.asarray(w, np.int64) & 0xF).astype(np.uint8)
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)


def bf16_ulps(orc, got, want):
    """Per-element distance in bf16 units in the last place (bit patterns of finite values,
    ordered across zero)."""
    def key(u):
        u = np.asarray(u, np.uint16).astype(np.int32)
        return np.where(u & 0x8000, -(u & 0x7FFF), u)
    return np.abs(key(got) - key(want))


class ExplicitLayer:
    """A layer whose tensors are numpy arrays uploaded to the device (q38_moe_layer_create)."""

    def __init__(self, q38, ctx, orc, H=512, I=128, E=64, k=4, gu=(8, 14), down=(8, 14), gu_group=None,
                 down_group=None, seed=0, router=None, book_format=0):
        rng = np.random.default_rng(seed)
        self.H, self.I, self.E, self.k = H, I, E, k
        self.qdesc = q38.desc(hidden=H, inter=I, experts=E, top_k=k, gu=gu, down=down, gu_group=gu_group,
                              down_group=down_group, book_format=book_format)
        import oracle_lib
        self.odesc = oracle_lib.make_desc(hidden=H, inter=I, experts=E, top_k=k, gu=gu, down=down,
                                          gu_group=gu_group, down_group=down_group, book_format=book_format)
        self.router = router if router is not None else orc.bf16(rng.normal(0, 0.02, (E, H)))
        self.wsg = orc.bf16(rng.normal(0, 0.02, H))
        geo = (gu, gu, down)
        ins, outs = (H, H, I), (I, I, H)
        grp = (gu_group or H, gu_group or H, down_group or I)
        self.books, self.codes, self.scales = [], [], []
        for p in range(3):
            dim, bits = geo[p]
            self.books.append(f16(rng.normal(0, 1, (1 << bits) * dim)))
            raw = rng.integers(0, 1 << bits, ((E + 1) * outs[p], ins[p] // dim)).astype(np.uint32)
            self.codes.append(np.stack([orc.pack_row(r, bits) for r in raw]).reshape(-1))
            self.scales.append(f16(rng.uniform(0.005, 0.02, (E + 1) * outs[p] * (ins[p] // grp[p]))))
        self.dev = [G.to_dev(a) for a in [self.router, self.wsg, *self.codes, *self.scales, *self.books]]
        w = q38.MoeWeights()
        w.router, w.shared_gate = self.dev[0].data_ptr(), self.dev[1].data_ptr()
        for p in range(3):
            w.codes[p] = self.dev[2 + p].data_ptr()
            w.scales[p] = self.dev[5 + p].data_ptr()
            w.books[p] = self.dev[8 + p].data_ptr()
        self.layer = q38.MoeLayer(ctx, self.qdesc, weights=w)

    def oracle(self, orc, x):
        return orc.moe_layer_dense(self.odesc, self.router, self.wsg, self.codes, self.scales, self.books, x)

    def close(self):
        self.layer.close()


def run_forward(q38, layer, desc, x_np):
    """q38_moe_forward on x (numpy bf16 bits) -> (y, experts, weights, logits, plan)."""
    M = x_np.shape[0]
    x = G.to_dev(x_np)
    y = G.empty(x_np.shape, np.uint16)
    MK = M * desc.top_k
    ex = G.empty(MK, np.int32)
    wt = G.empty(MK, np.float32)
    lg = G.empty(M * desc.experts, np.float32)
    plan = G.empty(2 + 4 * MK, np.int32)
    ws = G.workspace(q38.lib.q38_moe_workspace_size(C.byref(desc), M))
    r = q38.routes(ex, wt, lg, plan)
    q38.check(q38.lib.q38_moe_forward(layer.h, x.data_ptr(), M, y.data_ptr(), C.byref(r), ws.data_ptr(),
                                      ws.numel(), G.stream()))
    return (G.to_host(y, np.uint16), G.to_host(ex).reshape(M, -1), G.to_host(wt).reshape(M, -1),
            G.to_host(lg).reshape(M, -1), G.to_host(plan))


def tol_check(orc, got, want, rel=1e-2, mx=2e-2):
    g = orc.bf16_to_f32(got).astype(np.float64)
    w = orc.bf16_to_f32(want).astype(np.float64)
    r = np.linalg.norm(g - w) / max(np.linalg.norm(w), 1e-30)
    m = np.abs(g - w).max()
    assert r <= rel and m <= mx, (r, m)
    return r, m


def plan_check(orc, plan, experts, E):
    n, uexp, uoff, rl, rp = orc.plan(experts, E)
    MK = experts.size
    assert plan[0] == n
    assert np.array_equal(plan[1:1 + n], uexp)
    assert np.array_equal(plan[1 + MK:1 + MK + n + 1], uoff)
    assert np.array_equal(plan[2 + 2 * MK:2 + 3 * MK], rl)
    assert np.array_equal(plan[2 + 3 * MK:2 + 4 * MK], rp)
