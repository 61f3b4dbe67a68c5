"""GatedDeltaNet verify layers for the tests: random tensors in the reference checkpoint's
layout (in_proj_qkv / in_proj_z / in_proj_b / in_proj_a / out_proj affine-quantized,
conv1d.weight [C, 4] bf16, A_log fp32, dt_bias and norm.weight bf16; src/gated_delta_net.cpp:
138-178), and an independent float64 numpy restatement of GatedDeltaNet::forward_verify
(src/gated_delta_net.cpp:657-834) over the dequantized weights: vectorised per head, the
state and every intermediate kept in float64 (no bf16 rounding inside), so it agrees with the
oracle's bf16 contract within tolerance and differs from it by O(1) on a wrong index."""
from __future__ import annotations

import numpy as np

import oracle_lib
from affine_cases import from16, pack_affine, to16


class GdnLayer:
    def __init__(self, hidden=512, hk=2, hv=4, dk=128, dv=128, bits=8, group=64, fmt=0, gate_silu=0, seed=0,
                 eps=1e-6, wscale=0.02):
        rng = np.random.default_rng(seed)
        self.hidden, self.hk, self.hv, self.dk, self.dv = hidden, hk, hv, dk, dv
        self.bits, self.group, self.fmt, self.gate_silu, self.eps = bits, group, fmt, gate_silu, eps
        self.KW, self.VW = hk * dk, hv * dv
        self.C = 2 * self.KW + self.VW
        self.state_elems = 3 * self.C + hv * dv * dk
        self.odesc = oracle_lib.GdnDesc(hidden, hk, hv, dk, dv, 4, bits, group, fmt, gate_silu, eps)
        shapes = [(self.C, hidden), (self.VW, hidden), (hv, hidden), (hv, hidden), (hidden, self.VW)]
        self.proj = {"w": [], "s": [], "b": [], "q": []}
        for O, IN in shapes:
            q = rng.integers(0, 1 << bits, (O, IN))
            sc = rng.uniform(0.5, 1.5, (O, IN // group)) * wscale * 4 / (1 << bits)
            bi = -sc * ((1 << bits) - 1) / 2 + rng.normal(0, wscale * 0.05, (O, IN // group))
            self.proj["q"].append(q)
            self.proj["w"].append(pack_affine(q, bits))
            self.proj["s"].append(to16(sc, fmt))
            self.proj["b"].append(to16(bi, fmt))
        self.conv_w = to16(rng.normal(0, 0.5, (self.C, 4)), 0)
        self.a_log = np.log(rng.uniform(1.0, 16.0, hv)).astype(np.float32)
        self.dt_bias = to16(rng.normal(0, 0.5, hv), 0)
        self.norm_w = to16(rng.uniform(0.5, 1.5, dv), 0)

    def dequant(self, p):
        q = self.proj["q"][p].astype(np.float64)
        s = np.repeat(from16(self.proj["s"][p], self.fmt), self.group, axis=1)
        b = np.repeat(from16(self.proj["b"][p], self.fmt), self.group, axis=1)
        return s * q + b

    def random_state(self, rng, scale=0.05):
        st = rng.normal(0, scale, self.state_elems)
        return to16(st, 0)


def bf(u):
    return from16(np.asarray(u, np.uint16), 0)


def np_gdn_verify(L: GdnLayer, x, origin=None, fault_hk_mod=False):
    """float64 restatement: returns (out [S, hidden] float64, conv checkpoints [S, 3, C],
    recurrent checkpoints [S, HV, DV, DK])."""
    xf = bf(x)
    S = xf.shape[0]
    HK, HV, DK, DV, C, KW, VW = L.hk, L.hv, L.dk, L.dv, L.C, L.KW, L.VW
    sig = lambda a: 1.0 / (1.0 + np.exp(-a))
    qkv = xf @ L.dequant(0).T
    z = xf @ L.dequant(1).T
    b = xf @ L.dequant(2).T
    a = xf @ L.dequant(3).T
    if origin is None:
        conv0 = np.zeros((3, C))
        st = np.zeros((HV, DV, DK))
    else:
        o = bf(origin)
        conv0 = o[:3 * C].reshape(3, C)
        st = o[3 * C:].reshape(HV, DV, DK).copy()
    cin = np.concatenate([conv0, qkv], 0)                   # [S + 3, C]
    w = bf(L.conv_w)                                        # [C, 4]
    conv = sum(w[:, j] * cin[j:j + S] for j in range(4))    # [S, C]
    act = conv * sig(conv)
    q = act[:, :KW].reshape(S, HK, DK)
    k = act[:, KW:2 * KW].reshape(S, HK, DK)
    v = act[:, 2 * KW:].reshape(S, HV, DV)
    rms = lambda t: t / np.sqrt((t * t).mean(-1, keepdims=True) + 1e-6)
    q = rms(q) / DK
    k = rms(k) / np.sqrt(DK)
    head = (np.arange(HV) % HK) if fault_hk_mod else (np.arange(HV) // (HV // HK))
    q, k = q[:, head], k[:, head]                            # [S, HV, DK]
    beta = sig(b)
    decay = np.exp(-np.exp(L.a_log.astype(np.float64)) * np.log1p(np.exp(a + bf(L.dt_bias))))
    ys, states = [], []
    for t in range(S):
        st = st * decay[t][:, None, None]
        recalled = np.einsum("hvk,hk->hv", st, k[t])
        delta = (v[t] - recalled) * beta[t][:, None]
        st = st + delta[:, :, None] * k[t][:, None, :]
        ys.append(np.einsum("hvk,hk->hv", st, q[t]))
        states.append(st.copy())
    y = np.stack(ys)                                         # [S, HV, DV]
    yn = y / np.sqrt((y * y).mean(-1, keepdims=True) + L.eps) * bf(L.norm_w)
    zz = z.reshape(S, HV, DV)
    gate = zz * sig(zz) if L.gate_silu else sig(zz)
    out = (yn * gate).reshape(S, VW) @ L.dequant(4).T
    conv_ck = np.stack([cin[t + 1:t + 4] for t in range(S)])
    return out, conv_ck, np.stack(states)


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)
