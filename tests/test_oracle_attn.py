"""The full-attention verify oracle (orc_attn_verify, the dense path of
SelfAttention::forward_verify, src/self_attention.cpp:1450-1720) pinned without the oracle's
own formulas:
- closed forms:
  - a zero query (zero q_proj rows) attends uniformly, so the output is the mean of the
    visible values;
  - a one-hot query in a dimension RoPE leaves alone, matched by one large cached key, attends
    that token alone;
  - with an identity o_proj and zero gate rows (sigmoid 0 = 1/2) both are exact;
  - the RoPE table at position 0 and at R = 2 (frequency 1) against math.cos / math.sin;
- an independent float64 numpy restatement (tests/attn_cases.py) on three geometries;
- two planted faults that the restatement must catch: RoPE on interleaved pairs, and no causal
  mask within the verify rows;
- S rows = S one-row calls chained through the cache, bit for bit (which also pins the causal
  mask: a row must not see later rows)."""
import math

import numpy as np
import pytest

from affine_cases import pack_affine, to16
from attn_cases import AttnLayer, bf, np_attn_verify, rel_l2

H_ID, HQ_ID, HKV_ID, D_ID, R_ID = 128, 2, 1, 64, 16  # hidden = HQ * D: o_proj can be the identity


def identity_layer(q_rows=None, k_rows=None):
    """8-bit layer with scales 1 and biases 0 (weight = q exactly): o_proj the identity, the
    gate rows zero, q_proj / k_proj rows as given (dicts row -> (input column, integer value))."""
    L = AttnLayer(hidden=H_ID, q_heads=HQ_ID, kv_heads=HKV_ID, head_dim=D_ID, rotary_dim=R_ID, bits=8, group=64)

    def set_proj(p, rows_out, entries):
        O, IN = rows_out, L.proj["q"][p].shape[1]
        q = np.zeros((O, IN), np.int64)
        for o, (c, val) in (entries or {}).items():
            q[o, c] = val
        L.proj["q"][p] = q
        L.proj["w"][p] = pack_affine(q, 8)
        L.proj["s"][p] = to16(np.ones((O, IN // 64)), 0)
        L.proj["b"][p] = to16(np.zeros((O, IN // 64)), 0)

    set_proj(0, 2 * L.QW, q_rows)
    set_proj(1, L.KW, k_rows)
    set_proj(2, L.KW, {})
    set_proj(3, H_ID, {o: (o, 1) for o in range(H_ID)})
    L.q_norm = to16(np.ones(D_ID), 0)
    L.k_norm = to16(np.ones(D_ID), 0)
    return L


def test_rope_table_closed_forms(orc):
    c, s = orc.rope_table(1e6, 8, 0)
    assert np.array_equal(c, np.ones(4, np.float32)) and np.array_equal(s, np.zeros(4, np.float32))
    for pos in (1, 7, 1000, 123457):
        c, s = orc.rope_table(1e6, 2, pos)
        assert c[0] == bf(orc.bf16(np.float32(math.cos(pos)))) and s[0] == bf(orc.bf16(np.float32(math.sin(pos))))
        c, s = orc.rope_table(1e4, 4, pos)
        f = 1e4 ** -0.5
        assert c[1] == bf(orc.bf16(np.float32(math.cos(pos * f)))) and s[1] == bf(orc.bf16(np.float32(math.sin(pos * f))))


def test_zero_query_attends_uniformly(orc):
    rng = np.random.default_rng(1)
    L = identity_layer()
    T0, cap = 7, 16
    keys, values = L.random_cache(rng, cap, T0)
    x = to16(rng.normal(0, 1, (1, H_ID)), 0)
    out, k2, v2 = orc.attn_verify(L, x, keys, values, T0, 40)
    # the new row: zero k and v (zero projections); 8 visible tokens, p = 1/8 exactly
    assert not bf(k2[:, T0]).any() and not bf(v2[:, T0]).any()  # (signed zeros: 0 * cos < 0 is -0)
    mean = bf(v2[0, :T0 + 1]).astype(np.float64).mean(0)
    want = bf(orc.bf16((bf(orc.bf16(mean.astype(np.float32))) * 0.5).astype(np.float32)))
    got = bf(out[0]).reshape(HQ_ID, D_ID)
    assert np.array_equal(got[0], want) and np.array_equal(got[1], want)


def test_one_hot_query_attends_its_key(orc):
    """Query row = sqrt(D) e_j (j >= R, untouched by RoPE) for head 0 from input column 0; the
    cached key t* = 64 e_j: scores 64 at t*, 0 elsewhere, so the row reads v_t* alone."""
    j = 40
    L = identity_layer(q_rows={j: (0, 3)})
    rng = np.random.default_rng(2)
    T0, cap = 12, 16
    keys, values = L.random_cache(rng, cap, T0)
    keys[:, :T0] = 0
    tstar = 5
    keys[0, tstar, j] = to16(np.array([64.0]), 0)[0]
    x = np.zeros((1, H_ID), np.uint16)
    x[0, 0] = to16(np.array([1.0]), 0)[0]
    out, _, v2 = orc.attn_verify(L, x, keys, values, T0, 3)
    got = bf(out[0]).reshape(HQ_ID, D_ID)
    want = bf(orc.bf16((bf(v2[0, tstar]) * 0.5).astype(np.float32)))
    assert np.array_equal(got[0], want)
    # head 1 has a zero query: uniform over the 13 visible tokens
    assert not np.array_equal(got[1], want)


GEOS = [dict(), dict(bits=4, group=32, fmt=1, norm_offset=1, seed=1),
        dict(q_heads=8, kv_heads=1, head_dim=64, rotary_dim=64, seed=2, theta=1e4)]


@pytest.mark.parametrize("geo", GEOS)
def test_verify_matches_numpy(orc, geo):
    L = AttnLayer(**geo)
    rng = np.random.default_rng(10)
    T0, S, cap = 37, 4, 48
    keys, values = L.random_cache(rng, cap, T0)
    x = to16(rng.normal(0, 1, (S, L.hidden)), 0)
    out, k2, v2 = orc.attn_verify(L, x, keys, values, T0, 1000)
    wout, wk, wv = np_attn_verify(L, x, keys, values, T0, 1000)
    assert rel_l2(bf(k2[:, T0:T0 + S]), wk) < 1e-2 and rel_l2(bf(v2[:, T0:T0 + S]), wv) < 1e-2
    assert rel_l2(bf(out), wout) < 2e-2, rel_l2(bf(out), wout)
    # the cache outside the new rows is untouched
    assert np.array_equal(k2[:, :T0], keys[:, :T0]) and np.array_equal(k2[:, T0 + S:], keys[:, T0 + S:])


@pytest.mark.parametrize("fault", [1, 2])
def test_planted_faults_fail(orc, fault):
    L = AttnLayer(seed=3)
    rng = np.random.default_rng(11)
    T0, S, cap = 9, 4, 16
    keys, values = L.random_cache(rng, cap, T0, scale=0.2)
    x = to16(rng.normal(0, 1, (S, L.hidden)), 0)
    orc.attn_plant_fault(fault)
    try:
        out, _, _ = orc.attn_verify(L, x, keys, values, T0, 5000)
    finally:
        orc.attn_plant_fault(0)
    wout, _, _ = np_attn_verify(L, x, keys, values, T0, 5000)
    assert rel_l2(bf(out), wout) > 0.05, rel_l2(bf(out), wout)
    fout, _, _ = np_attn_verify(L, x, keys, values, T0, 5000, interleaved=fault == 1, causal=fault != 2)
    assert rel_l2(bf(out), fout) < 2e-2  # (the fault is the planted one, nothing else)


def test_rows_chain_through_the_cache(orc):
    L = AttnLayer(seed=4)
    rng = np.random.default_rng(12)
    T0, S, cap = 20, 5, 32
    keys, values = L.random_cache(rng, cap, T0)
    x = to16(rng.normal(0, 1, (S, L.hidden)), 0)
    out, k2, v2 = orc.attn_verify(L, x, keys, values, T0, 77)
    kc, vc = keys, values
    for r in range(S):
        o1, kc, vc = orc.attn_verify(L, x[r:r + 1], kc, vc, T0 + r, 77 + r)
        assert np.array_equal(o1[0], out[r]), r
    assert np.array_equal(kc, k2) and np.array_equal(vc, v2)
