"""Pins of the oracle's GatedDeltaNet verify step (GatedDeltaNet::forward_verify,
src/gated_delta_net.cpp:657-834; the bf16-sum recurrence, src/gdn_metal_kernels.hpp:498-562):
closed forms of the recurrence, an independent float64 numpy restatement of the recurrence
and of the whole step, the chaining of single-row calls through the checkpoints, and planted
faults (a wrong key-head mapping) that those checks catch."""
import numpy as np
import pytest

from gdn_cases import GdnLayer, bf, np_gdn_verify, rel_l2
from affine_cases import to16


def bf16v(orc, a):
    """Round float values to bf16 and return them as float32."""
    return orc.bf16_to_f32(orc.bf16(np.asarray(a, np.float32)))


def test_recurrence_one_row_from_zero(orc):
    """From a zero state one row writes beta * v * k^T and reads beta * v * (k . q)."""
    S, HK, HV, DK, DV = 1, 1, 2, 128, 8
    q = np.full((S, HK, DK), 2.0 ** -4, np.float32)
    k = np.full((S, HK, DK), 2.0 ** -3, np.float32)
    v = np.ones((S, HV, DV), np.float32)
    v[0, 1] = 2.0
    beta = np.full((S, HV), 0.5, np.float32)
    decay = np.full((S, HV), 0.75, np.float32)
    y, st = orc.gdn_recurrence(HK, q, k, v, decay, beta)
    # y = beta * v * (k . q) = 0.5 * v * 128 * 2^-7
    assert np.array_equal(y[0, 0], np.full(DV, 0.5, np.float32))
    assert np.array_equal(y[0, 1], np.full(DV, 1.0, np.float32))
    sf = orc.bf16_to_f32(st)
    assert np.array_equal(sf[0, 0], np.full((DV, DK), 2.0 ** -4, np.float32))
    assert np.array_equal(sf[0, 1], np.full((DV, DK), 2.0 ** -3, np.float32))


def test_recurrence_decay_only(orc):
    """beta = 0: no update; the state decays by g every row, y_t = (g^(t+1) s) . q."""
    S, HK, HV, DK, DV = 4, 1, 1, 32, 4
    q = np.full((S, HK, DK), 2.0 ** -5, np.float32)
    k = np.full((S, HK, DK), 1.0, np.float32)
    v = np.ones((S, HV, DV), np.float32)
    beta = np.zeros((S, HV), np.float32)
    decay = np.full((S, HV), 0.5, np.float32)
    state = to16(np.ones((HV, DV, DK)), 0)
    y, st = orc.gdn_recurrence(HK, q, k, v, decay, beta, state)
    for t in range(S):
        g = 0.5 ** (t + 1)
        assert np.array_equal(orc.bf16_to_f32(st[t]), np.full((HV, DV, DK), g, np.float32))
        assert np.array_equal(y[t], np.full((HV, DV), g * DK * 2.0 ** -5, np.float32))


def test_recurrence_delta_rule_writes_the_value(orc):
    """g = 1, beta = 1, k = e_j: the delta rule replaces column j of the state by v and leaves
    the other columns; y reads column j when q = e_j (exact small dyadic values)."""
    rng = np.random.default_rng(0)
    HK, HV, DK, DV = 1, 2, 64, 8
    j = 37
    s0 = rng.integers(-2, 3, (HV, DV, DK)) / 8.0
    v = (rng.integers(-2, 3, (1, HV, DV)) / 8.0).astype(np.float32)
    k = np.zeros((1, HK, DK), np.float32)
    k[0, 0, j] = 1.0
    y, st = orc.gdn_recurrence(HK, k, k, v, np.ones((1, HV), np.float32), np.ones((1, HV), np.float32),
                               to16(s0, 0))
    sf = orc.bf16_to_f32(st[0]).astype(np.float64)
    want = s0.copy()
    want[:, :, j] = v[0]
    assert np.array_equal(sf, want)
    assert np.array_equal(y[0], v[0])


def np_recurrence(HK, q, k, v, decay, beta, s0, fault=False):
    S, HV, DV = v.shape
    head = (np.arange(HV) % HK) if fault else (np.arange(HV) // (HV // HK))
    q, k = q[:, head].astype(np.float64), k[:, head].astype(np.float64)
    st = s0.astype(np.float64).copy()
    ys, sts = [], []
    for t in range(S):
        st = st * decay[t][:, None, None]
        delta = (v[t] - np.einsum("hvk,hk->hv", st, k[t])) * beta[t][:, None]
        st = st + delta[:, :, None] * k[t][:, None, :]
        ys.append(np.einsum("hvk,hk->hv", st, q[t]))
        sts.append(st.copy())
    return np.stack(ys), np.stack(sts)


def random_recurrence_inputs(orc, rng, S=5, HK=2, HV=4, DK=128, DV=16):
    q = bf16v(orc, rng.normal(0, 1, (S, HK, DK)) / DK)
    k = bf16v(orc, rng.normal(0, 1, (S, HK, DK)) / np.sqrt(DK))
    v = bf16v(orc, rng.normal(0, 1, (S, HV, DV)))
    decay = bf16v(orc, rng.uniform(0.6, 1.0, (S, HV)))
    beta = bf16v(orc, rng.uniform(0.1, 0.9, (S, HV)))
    s0 = to16(rng.normal(0, 0.1, (HV, DV, DK)), 0)
    return q, k, v, decay, beta, s0


def test_recurrence_matches_numpy_and_catches_a_wrong_head(orc):
    rng = np.random.default_rng(1)
    HK = 2
    q, k, v, decay, beta, s0 = random_recurrence_inputs(orc, rng, HK=HK)
    y, st = orc.gdn_recurrence(HK, q, k, v, decay, beta, s0)
    wy, wst = np_recurrence(HK, q, k, v, decay, beta, bf(s0).reshape(st.shape[1:]))
    assert rel_l2(y, wy) < 1e-2, rel_l2(y, wy)
    assert rel_l2(bf(st), wst) < 1e-2
    orc.gdn_plant_fault(1)
    try:
        y2, _ = orc.gdn_recurrence(HK, q, k, v, decay, beta, s0)
    finally:
        orc.gdn_plant_fault(0)
    assert rel_l2(y2, wy) > 0.2


@pytest.mark.parametrize("geo", [dict(), dict(bits=4, group=32, fmt=1, gate_silu=1), dict(hk=4, hv=4, seed=3)])
def test_verify_matches_numpy(orc, geo):
    L = GdnLayer(**geo)
    rng = np.random.default_rng(5)
    x = orc.bf16(rng.normal(0, 1, (4, L.hidden)).astype(np.float32))
    for origin in (None, L.random_state(rng)):
        out, ck = orc.gdn_verify(L, x, origin)
        wout, wconv, wrec = np_gdn_verify(L, x, origin)
        assert rel_l2(bf(out), wout) < 2e-2, rel_l2(bf(out), wout)
        conv = bf(ck[:, :3 * L.C]).reshape(-1, 3, L.C)
        rec = bf(ck[:, 3 * L.C:]).reshape(wrec.shape)
        assert rel_l2(conv, wconv) < 1e-2
        assert rel_l2(rec, wrec) < 2e-2, rel_l2(rec, wrec)


def test_verify_planted_head_fault_fails(orc):
    L = GdnLayer(hk=2, hv=4)
    rng = np.random.default_rng(6)
    x = orc.bf16(rng.normal(0, 1, (3, L.hidden)).astype(np.float32))
    wout, _, _ = np_gdn_verify(L, x)
    orc.gdn_plant_fault(1)
    try:
        out, _ = orc.gdn_verify(L, x)
    finally:
        orc.gdn_plant_fault(0)
    assert rel_l2(bf(out), wout) > 0.1
    fout, _, _ = np_gdn_verify(L, x, fault_hk_mod=True)
    assert rel_l2(bf(out), fout) < 2e-2  # (the fault is the mapping, nothing else)


def test_rows_chain_through_checkpoints(orc):
    """S rows in one call equal S one-row calls, each from the previous call's checkpoint, bit
    for bit (outputs and every checkpoint)."""
    L = GdnLayer(seed=2)
    rng = np.random.default_rng(7)
    x = orc.bf16(rng.normal(0, 1, (5, L.hidden)).astype(np.float32))
    origin = L.random_state(rng)
    out, ck = orc.gdn_verify(L, x, origin)
    state = origin
    for t in range(5):
        o1, c1 = orc.gdn_verify(L, x[t:t + 1], state)
        assert np.array_equal(o1[0], out[t]) and np.array_equal(c1[0], ck[t])
        state = c1[0]
