"""RMSNorm with unit gamma (the verify chain's pre-norm and the head's input):
x = T(h / sqrt(mean(h^2) + eps)), T = bf16 round-to-nearest-even. The oracle is pinned by a
float64 numpy restatement (bit-exact: every square and partial sum of bf16 inputs is exact
in double) and by closed forms that a dropped mean, a wrong eps placement or a wrong
rounding point would fail."""
import numpy as np
import pytest


def np_rmsnorm(orc, h, eps):
    hf = orc.bf16_to_f32(h).astype(np.float64)
    ss = np.array([np.sum(r * r) for r in hf])
    inv = 1.0 / np.sqrt(ss / h.shape[1] + eps)
    return orc.bf16((hf * inv[:, None]).astype(np.float32))


@pytest.mark.parametrize("H", [512, 2048, 2560])
def test_rmsnorm_vs_numpy(orc, H):
    rng = np.random.default_rng(H)
    h = orc.bf16(rng.normal(0, 1, (8, H)) * np.exp(rng.uniform(-6, 6, (8, 1))))
    assert np.array_equal(orc.rmsnorm(h), np_rmsnorm(orc, h, 1e-6))


def test_rmsnorm_closed_forms(orc):
    H = 2048
    c = np.float32(0.75)
    rows = np.zeros((4, H), np.float32)
    rows[0] = c                                   # constant row: c / sqrt(c^2 + eps)
    rows[1, 0::2], rows[1, 1::2] = c, -c          # alternating signs: same magnitude
    rows[3, 7] = 1.0                              # one-hot: sqrt(H) (bf16 of 45.25...)
    h = orc.bf16(rows)
    got = orc.bf16_to_f32(orc.rmsnorm(h, eps=1e-6)).astype(np.float64)
    v = np.float32(0.75 / np.sqrt(0.5625 + 1e-6))
    assert np.all(got[0] == orc.bf16_to_f32(orc.bf16(np.full(H, v, np.float32))))
    assert np.all(got[1, 0::2] == got[0, 0]) and np.all(got[1, 1::2] == -got[0, 0])
    assert np.all(got[2] == 0.0)                  # zero row stays zero (inv = 1/sqrt(eps))
    one = orc.bf16_to_f32(orc.bf16(np.array([1.0 / np.sqrt(1.0 / H + 1e-6)], np.float32)))[0]
    assert got[3, 7] == one and np.count_nonzero(got[3]) == 1


def test_rmsnorm_invariants(orc):
    rng = np.random.default_rng(3)
    h = orc.bf16(rng.normal(0, 1, (4, 2048)))
    base = orc.rmsnorm(h, eps=0.0)
    hf = orc.bf16_to_f32(h)
    for k in (-3, 2, 5):  # power-of-two scaling is exact at every step when eps = 0
        assert np.array_equal(orc.rmsnorm(orc.bf16(hf * np.float32(2.0 ** k)), eps=0.0), base)
    assert np.array_equal(orc.bf16_to_f32(orc.rmsnorm(orc.bf16(-hf))), -orc.bf16_to_f32(orc.rmsnorm(h)))
