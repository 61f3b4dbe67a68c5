"""Full-attention verify layers for the tests: random tensors in the reference checkpoint's
layout (q_proj [HQ * 2D, H] with each head's D query rows followed by its D gate rows, k_proj /
v_proj [HKV * D, H], o_proj [H, HQ * D], MLX affine-quantized; q_norm / k_norm [D] bf16;
src/self_attention.cpp:460-521), random KV caches, and an independent float64 numpy
restatement of SelfAttention::forward_verify on the dense path (src/self_attention.cpp:
1450-1720, the explicit decode arithmetic of :1240-1305) over the dequantized weights. The
restatement keeps every intermediate in float64 (no bf16 rounding inside), computes RoPE
with numpy's own cos / sin and writes the rotation as a 2 x 2 matrix per pair, so it agrees
with the oracle's bf16 contract within tolerance and differs from it by O(1) on a wrong
pairing, position or mask."""
from __future__ import annotations

import numpy as np

import oracle_lib
from affine_cases import from16, pack_affine, to16


class AttnLayer:
    def __init__(self, hidden=512, q_heads=4, kv_heads=2, head_dim=128, rotary_dim=32, bits=8, group=64, fmt=0,
                 norm_offset=0, seed=0, eps=1e-6, theta=1e7, wscale=0.02):
        rng = np.random.default_rng(seed)
        self.hidden, self.hq, self.hkv, self.d, self.rot = hidden, q_heads, kv_heads, head_dim, rotary_dim
        self.bits, self.group, self.fmt, self.norm_offset, self.eps, self.theta = bits, group, fmt, norm_offset, eps, theta
        self.QW, self.KW = q_heads * head_dim, kv_heads * head_dim
        self.odesc = oracle_lib.AttnDesc(hidden, q_heads, kv_heads, head_dim, rotary_dim, bits, group, fmt,
                                         norm_offset, eps, theta)
        shapes = [(2 * self.QW, hidden), (self.KW, hidden), (self.KW, hidden), (hidden, self.QW)]
        self.proj = {"w": [], "s": [], "b": [], "q": []}
        for O, IN in shapes:
            q = rng.integers(0, 1 << bits, (O, IN))
            sc = rng.uniform(0.5, 1.5, (O, IN // group)) * wscale * 4 / (1 << bits)
            bi = -sc * ((1 << bits) - 1) / 2 + rng.normal(0, wscale * 0.05, (O, IN // group))
            self.proj["q"].append(q)
            self.proj["w"].append(pack_affine(q, bits))
            self.proj["s"].append(to16(sc, fmt))
            self.proj["b"].append(to16(bi, fmt))
        base = 0.0 if norm_offset else 1.0
        self.q_norm = to16(base + rng.normal(0, 0.2, head_dim), 0)
        self.k_norm = to16(base + rng.normal(0, 0.2, head_dim), 0)

    def dequant(self, p):
        q = self.proj["q"][p].astype(np.float64)
        s = np.repeat(from16(self.proj["s"][p], self.fmt), self.group, axis=1)
        b = np.repeat(from16(self.proj["b"][p], self.fmt), self.group, axis=1)
        return s * q + b

    def random_cache(self, rng, cap, T0, scale=1.0):
        """keys / values [HKV, cap, D] bf16 bits: T0 valid tokens (keys of unit RMS like normed
        keys), the rest filled with a large value that must never be read."""
        k = np.full((self.hkv, cap, self.d), 0x4780, np.uint16)   # 65536.0 in the unused slots
        v = np.full((self.hkv, cap, self.d), 0x4780, np.uint16)
        k[:, :T0] = to16(rng.normal(0, scale, (self.hkv, T0, self.d)), 0)
        v[:, :T0] = to16(rng.normal(0, scale, (self.hkv, T0, self.d)), 0)
        return k, v


def bf(u):
    return from16(np.asarray(u, np.uint16), 0)


def np_rope(x, pos, R, theta, interleaved=False):
    """x [..., D] at positions pos (broadcast over the leading axes) -> rotated copy."""
    out = np.array(x, np.float64, copy=True)
    half = R // 2
    inv = theta ** (-2.0 * np.arange(half) / R)
    ang = np.asarray(pos, np.float64)[..., None] * inv       # [..., half]
    c, s = np.cos(ang), np.sin(ang)
    if interleaved:
        a, b = x[..., 0:R:2], x[..., 1:R:2]
        out[..., 0:R:2] = a * c - b * s
        out[..., 1:R:2] = a * s + b * c
    else:
        a, b = x[..., :half], x[..., half:R]
        out[..., :half] = a * c - b * s
        out[..., half:R] = a * s + b * c
    return out


def np_attn_verify(L: AttnLayer, x, keys, values, T0, position, interleaved=False, causal=True):
    """float64 restatement -> (out [S, hidden] float64, new keys [HKV, S, D], new values)."""
    xf = bf(x)
    S = xf.shape[0]
    HQ, HKV, D, R = L.hq, L.hkv, L.d, L.rot
    qg = (xf @ L.dequant(0).T).reshape(S, HQ, 2 * D)
    q, gate = qg[..., :D], qg[..., D:]
    k = (xf @ L.dequant(1).T).reshape(S, HKV, D)
    v = (xf @ L.dequant(2).T).reshape(S, HKV, D)
    wq, wk = bf(L.q_norm), bf(L.k_norm)
    if L.norm_offset:
        wq, wk = 1.0 + wq, 1.0 + wk
    rms = lambda t: t / np.sqrt((t * t).mean(-1, keepdims=True) + L.eps)
    pos = position + np.arange(S)
    q = np_rope(rms(q) * wq, pos[:, None], R, L.theta, interleaved)
    k = np_rope(rms(k) * wk, pos[:, None], R, L.theta, interleaved)
    K = np.concatenate([bf(keys[:, :T0]), k.transpose(1, 0, 2)], 1)   # [HKV, T0 + S, D]
    V = np.concatenate([bf(values[:, :T0]), v.transpose(1, 0, 2)], 1)
    grp = HQ // HKV
    att = np.empty((S, HQ, D))
    for r in range(S):
        T = T0 + r + 1 if causal else T0 + S
        for h in range(HQ):
            sc = K[h // grp, :T] @ q[r, h] / np.sqrt(D)
            p = np.exp(sc - sc.max())
            p /= p.sum()
            att[r, h] = p @ V[h // grp, :T]
    gated = att * (1.0 / (1.0 + np.exp(-gate)))
    out = gated.reshape(S, HQ * D) @ L.dequant(3).T
    return out, k.transpose(1, 0, 2), v.transpose(1, 0, 2)


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)
