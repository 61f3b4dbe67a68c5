"""Pins of the oracle's HyperConnection mixer (read / write), CPU only.

Reference: HyperConnection::read / write (src/hyper_connection.cpp:309-493, 692-709), the
rounding points of its fused read kernels (src/hc_metal_kernels.hpp:10-36, 85-128,
270-308) and the MLX graph's injection (src/hyper_connection.cpp:481-493). MLX itself is not
in this image, so the oracle is pinned by an independent vectorised numpy restatement and by
closed forms that a dropped term, a wrong rounding point, a transposed operand or a wrong
packed-value order would break.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle_lib import HcDesc, Oracle


@pytest.fixture(scope="module")
def orc():
    return Oracle()


def rbf(x):
    """Round float32 values to bf16 (nearest even), returned as float32."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def to_bf16_bits(x):
    return (rbf(x).view(np.uint32) >> 16).astype(np.uint16)


def bf(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def rbf_scalar(v: float) -> float:
    return float(rbf(np.float32(v)))


def unpack(words, n, bits):
    vpw = 32 // bits
    k = np.arange(n)
    return ((words[:, k // vpw] >> (bits * (k % vpw)).astype(np.uint32)) & ((1 << bits) - 1)).astype(np.float64)


def dequant(words, s, b, n, bits, group):
    q = unpack(words, n, bits)
    g = np.arange(n) // group
    return q * bf(s)[:, g].astype(np.float64) + bf(b)[:, g].astype(np.float64)


def sigmoid64(v):
    with np.errstate(over="ignore"):
        return (1.0 / (1.0 + np.exp(-np.asarray(v, np.float64)))).astype(np.float32)


def np_hc_read(d: HcDesc, w, stream):
    """Independent vectorised restatement (float64 dots rounded to float32, float32 steps)."""
    H, HC, R, bits, G = d.hidden, d.streams, d.rank, d.bits, d.group
    K = HC * H
    Wd = dequant(w["down_w"], w["down_s"], w["down_b"], K, bits, G)
    Wu = dequant(w["up_w"], w["up_s"], w["up_b"], R, bits, G)
    x = bf(stream).reshape(-1, HC, H)
    ss = (x.astype(np.float64) ** 2).sum(axis=2).astype(np.float32)
    inv = (1.0 / np.sqrt(ss.astype(np.float64) / H + np.float64(np.float32(d.eps)))).astype(np.float32)
    t = rbf(x * inv[:, :, None])
    wn = rbf(bf(w["norm"]).reshape(HC, H) + np.float32(1.0))
    xn = rbf(t * wn[None]).reshape(-1, K)
    dot = (xn.astype(np.float64) @ Wd.T).astype(np.float32)
    v = rbf(dot / np.float32(HC))
    sg = rbf(sigmoid64(v))
    act = rbf(v * sg)
    inj = None
    if d.with_injection:
        Wi = dequant(w["inj_w"], w["inj_s"], w["inj_b"], K, bits, G)
        di = rbf((xn.astype(np.float64) @ Wi.T).astype(np.float32))
        vi = rbf(di * rbf(np.float32(1.0) / np.float32(HC)))
        gi = rbf(sigmoid64(vi))
        inj = to_bf16_bits(gi * np.float32(2.0))
    u = rbf((act.astype(np.float64) @ Wu.T).astype(np.float32))          # [M, HC*H]
    gate = rbf(sigmoid64(u))
    terms = rbf(gate * xn).reshape(-1, HC, H)
    s = np.zeros(terms.shape[::2], np.float32)
    for h in range(HC):  # float32 additions in stream order
        s = (s + terms[:, h]).astype(np.float32)
    mixed = to_bf16_bits(rbf(s) / np.float32(HC))
    return mixed, inj, to_bf16_bits(xn), act


def random_case(rng, H=256, HC=4, R=64, bits=4, G=32, inj=True, M=3):
    K = HC * H
    vpw = 32 // bits
    d = HcDesc(H, HC, R, bits, G, 1 if inj else 0, 1e-6)

    def proj(out, n):
        # centred affine groups, as a quantiser makes them: bias ~ -scale * (2^bits - 1) / 2
        scale = rbf(np.abs(rng.normal(0, 0.05, (out, n // G))).astype(np.float32) / (1 << (bits - 1)))
        bias = -scale * np.float32(((1 << bits) - 1) / 2) + rng.normal(0, 0.002, scale.shape).astype(np.float32)
        return (rng.integers(0, 2**32, size=(out, n // vpw), dtype=np.uint64).astype(np.uint32),
                to_bf16_bits(scale), to_bf16_bits(bias))

    w = {"norm": to_bf16_bits(rng.normal(0, 0.1, K).astype(np.float32))}
    w["down_w"], w["down_s"], w["down_b"] = proj(R, K)
    w["up_w"], w["up_s"], w["up_b"] = proj(K, R)
    if inj:
        w["inj_w"], w["inj_s"], w["inj_b"] = proj(HC, K)
    stream = to_bf16_bits(rng.normal(0, 1.0, (M, K)).astype(np.float32))
    return d, w, stream


def ulp_diff(a_bits, b_bits):
    a = a_bits.astype(np.int32)
    b = b_bits.astype(np.int32)
    sa = np.where(a & 0x8000, -(a & 0x7FFF), a & 0x7FFF)
    sb = np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)
    return np.abs(sa - sb)


@pytest.mark.parametrize("bits,G,inj", [(4, 32, True), (4, 64, True), (8, 64, False), (8, 128, True)])
def test_oracle_matches_numpy_restatement(orc, bits, G, inj):
    rng = np.random.default_rng(100 + bits + G)
    d, w, stream = random_case(rng, H=256, HC=4, R=128, bits=bits, G=G, inj=inj)
    mixed, injv, xn, act = orc.hc_read(d, w, stream)
    m2, i2, xn2, act2 = np_hc_read(d, w, stream)
    # the dots differ only in double summation order: float results agree except, rarely, one
    # bf16 step at a rounding boundary
    for a, b in ((xn, xn2), (mixed, m2)):
        u = ulp_diff(a, b)
        assert u.max() <= 1 and (u > 0).mean() <= 2e-3
    u = ulp_diff(to_bf16_bits(act), to_bf16_bits(act2))
    assert u.max() <= 1 and (u > 0).mean() <= 2e-3
    if inj:
        assert ulp_diff(injv, i2).max() <= 1


def test_zero_projections_and_sign_streams_closed_form(orc):
    """Zero weights: act = T(0 * T(sigmoid(0))) = 0, every gate is T(sigmoid(0)) = 0.5 and the
    injection is T(2 * 0.5) = 1. Streams held at constants |c| >= 1 normalise to sign(c)
    (c / sqrt(c^2 + eps) rounds to +-1 in bf16), so mixed = T(sum_s 0.5 sign_s / HC)."""
    H, HC, R, bits, G = 256, 4, 64, 4, 64
    K = HC * H
    d = HcDesc(H, HC, R, bits, G, 1, 1e-6)
    z = lambda o, n: (np.zeros((o, n * bits // 32), np.uint32), np.zeros((o, n // G), np.uint16),
                      np.zeros((o, n // G), np.uint16))
    w = {"norm": np.zeros(K, np.uint16)}
    w["down_w"], w["down_s"], w["down_b"] = z(R, K)
    w["up_w"], w["up_s"], w["up_b"] = z(K, R)
    w["inj_w"], w["inj_s"], w["inj_b"] = z(HC, K)
    signs = np.array([[1, 1, 1, -1], [-1, -1, 1, -1], [1, -1, 1, -1]], np.float32)
    mags = np.array([1.0, 3.0, 7.5, 100.0], np.float32)
    stream = to_bf16_bits(np.repeat(signs * mags, H, axis=1))
    mixed, inj, xn, act = orc.hc_read(d, w, stream)
    assert np.all(act == 0.0)
    assert np.all(bf(xn).reshape(3, HC, H) == signs[:, :, None])
    assert np.all(bf(inj) == 1.0)
    expect = signs.sum(axis=1) * 0.5 / HC
    assert np.all(bf(mixed) == expect[:, None])


def test_packed_order_and_norm_weight_closed_form(orc):
    """One packed value q = 1 (scale 1, bias 0) at input j of rank row r: act[r] =
    T(v * T(sigmoid(v))) with v = T(xn[j] / HC). A constant unit stream with norm weight
    raw[k] = k / 64 gives xn[k] = 1 + k / 64 exactly, so the result names the input the value
    was read from (LSB-first packing) and the norm weight's 1 + w."""
    H, HC, R, G = 256, 4, 64, 64
    K = HC * H
    for bits in (4, 8):
        vpw = 32 // bits
        d = HcDesc(H, HC, R, bits, G, 0, 1e-6)
        w = {"norm": to_bf16_bits((np.arange(K) % 64 / 64.0).astype(np.float32))}
        dw = np.zeros((R, K // vpw), np.uint32)
        js = [(r * 7 + 3) % 64 for r in range(R)]  # input j of row r, within the first group
        for r, j in enumerate(js):
            dw[r, j // vpw] = np.uint32(1) << np.uint32(bits * (j % vpw))
        w["down_w"] = dw
        w["down_s"] = np.full((R, K // G), to_bf16_bits(np.float32(1.0)), np.uint16)
        w["down_b"] = np.zeros((R, K // G), np.uint16)
        w["up_w"] = np.zeros((K, R // vpw), np.uint32)
        w["up_s"] = np.zeros((K, R // G), np.uint16)
        w["up_b"] = np.zeros((K, R // G), np.uint16)
        stream = to_bf16_bits(np.ones((1, K), np.float32))
        _, _, xn, act = orc.hc_read(d, w, stream)
        assert np.all(bf(xn)[0] == 1.0 + (np.arange(K) % 64) / 64.0)
        for r, j in enumerate(js):
            v = rbf_scalar((1.0 + j / 64.0) / HC)
            sg = rbf_scalar(1.0 / (1.0 + math.exp(-v)))
            assert act[0, r] == rbf_scalar(v * sg), (bits, r, j)


def test_bias_only_injection_closed_form(orc):
    """Injection rows with q = 0, scale 0 and bias beta: dot = beta * sum_k xn[k]. With sign
    streams the sum is H * sum_s sign_s; inj = T(2 T(sigmoid(T(T(dot) * 0.25))))."""
    H, HC, R, bits, G = 256, 4, 64, 8, 32
    K = HC * H
    d = HcDesc(H, HC, R, bits, G, 1, 1e-6)
    z = lambda o, n: (np.zeros((o, n * bits // 32), np.uint32), np.zeros((o, n // G), np.uint16),
                      np.zeros((o, n // G), np.uint16))
    w = {"norm": np.zeros(K, np.uint16)}
    w["down_w"], w["down_s"], w["down_b"] = z(R, K)
    w["up_w"], w["up_s"], w["up_b"] = z(K, R)
    betas = np.array([0.0, 1.0 / 512, -1.0 / 256, 1.0 / 128], np.float32)
    w["inj_w"] = np.zeros((HC, K // 4), np.uint32)
    w["inj_s"] = np.zeros((HC, K // G), np.uint16)
    w["inj_b"] = np.repeat(to_bf16_bits(betas)[:, None], K // G, axis=1)
    signs = np.array([[1, 1, -1, 1], [-1, -1, -1, -1]], np.float32)
    stream = to_bf16_bits(np.repeat(signs * 2.0, H, axis=1))
    _, inj, _, _ = orc.hc_read(d, w, stream)
    for m in range(2):
        total = H * signs[m].sum()
        for c in range(HC):
            dot = rbf_scalar(betas[c] * total)
            v = rbf_scalar(dot * 0.25)
            g = rbf_scalar(1.0 / (1.0 + math.exp(-v)))
            assert bf(inj[m, c]) == rbf_scalar(2.0 * g), (m, c)


def test_write_closed_forms(orc):
    """write: out = T(stream + T(block * inj[s])): injection 1 with a zero block returns the
    stream; injection 2 gives T(stream + 2 block) (the doubling is exact)."""
    rng = np.random.default_rng(7)
    H, HC, M = 64, 4, 3
    stream = to_bf16_bits(rng.normal(0, 1, (M, HC * H)).astype(np.float32))
    block = to_bf16_bits(rng.normal(0, 1, (M, H)).astype(np.float32))
    one = np.full((M, HC), to_bf16_bits(np.float32(1.0)), np.uint16)
    two = np.full((M, HC), to_bf16_bits(np.float32(2.0)), np.uint16)
    out = orc.hc_write(H, HC, stream, np.zeros_like(block), one)
    assert np.array_equal(out, stream)
    out = orc.hc_write(H, HC, stream, block, two)
    expect = to_bf16_bits(bf(stream).reshape(M, HC, H) + 2.0 * bf(block)[:, None, :]).reshape(M, HC * H)
    assert np.array_equal(out, expect)
    # per-stream injection: stream s takes its own gate
    gates = to_bf16_bits(np.array([[0.5, 1.0, 1.5, 2.0]] * M, np.float32))
    out = orc.hc_write(H, HC, stream, block, gates)
    g = bf(gates)[:, :, None]
    expect = to_bf16_bits(bf(stream).reshape(M, HC, H) + rbf(bf(block)[:, None, :] * g)).reshape(M, HC * H)
    assert np.array_equal(out, expect)


def test_planted_mistake_is_caught(orc):
    """The numpy restatement is sensitive: dropping the 1 + w of the norm weight, or the / HC
    of the rank projection, moves the outputs far beyond the comparison bound."""
    rng = np.random.default_rng(3)
    d, w, stream = random_case(rng, H=256, HC=4, R=64, bits=4, G=64, inj=False, M=2)
    mixed, _, _, _ = orc.hc_read(d, w, stream)
    w_bad = dict(w)
    w_bad["norm"] = to_bf16_bits(bf(w["norm"]) - 1.0)  # the restatement adds 1 to this
    m_bad, _, _, _ = np_hc_read(d, w_bad, stream)
    assert (ulp_diff(mixed, m_bad) > 1).mean() > 0.1
