"""LM head logit contract (R12), argmax tie semantics (R13), Philox KATs and
rejection-sampling invariants (R16) of the CPU oracle."""
import numpy as np
import pytest
from scipy import stats


def test_head_contract_vs_float64(orc):
    rng = np.random.default_rng(0)
    V, H = 3000, 2048
    W = rng.integers(-127, 128, (V, H)).astype(np.int8)
    s = rng.uniform(1e-4, 1e-3, V).astype(np.float16)
    h = orc.bf16(rng.normal(0, 1, (4, H)))
    got = orc.head_q8_logits(W, s.view(np.uint16), h)
    hf = orc.bf16_to_f32(h).astype(np.float64)
    want = ((W.astype(np.float64) @ hf.T) * s.astype(np.float64)[:, None]).T.astype(np.float32)
    assert np.mean(got == want) > 0.999
    assert np.max(np.abs(got - want) / np.abs(want)) < 2 ** -22


def test_argmax_ties_lowest_index(orc):
    lg = np.full((2, 4099), -1000.0, np.float32)
    lg[0, 17] = 9.0
    lg[0, 2048] = lg[0, 3072] = 11.0   # tests/mlx_backend_test.cpp:26-36
    lg[1, 4098] = 1.0
    idx, val = orc.argmax(lg)
    assert idx.tolist() == [2048, 4098] and val.tolist() == [11.0, 1.0]


def test_head_duplicate_rows_tie(orc):
    rng = np.random.default_rng(1)
    V, H = 64, 2048
    W = rng.integers(-127, 128, (V, H)).astype(np.int8)
    s = np.full(V, 1e-3, np.float16)
    h = orc.bf16(rng.normal(0, 1, (1, H)))
    lg = orc.head_q8_logits(W, s.view(np.uint16), h)
    best = int(np.argmax(lg[0]))
    W[40] = W[best]
    W[best + 1 if best + 1 != 40 else best + 2] = W[best]
    lg = orc.head_q8_logits(W, s.view(np.uint16), h)
    idx, _ = orc.argmax(lg)
    assert idx[0] == min(best, 40)


PHILOX_KAT = [  # Random123 kat_vectors, philox4x32_10
    ([0, 0, 0, 0], [0, 0], [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
    ([0xffffffff] * 4, [0xffffffff] * 2, [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]),
    ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0],
     [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]),
]


@pytest.mark.parametrize("ctr,key,out", PHILOX_KAT)
def test_philox_kat(orc, q38, ctr, key, out):
    import ctypes as C
    assert orc.philox(ctr, key) == out
    o = (C.c_uint32 * 4)()
    q38.lib.q38_philox4x32_10((C.c_uint32 * 4)(*ctr), (C.c_uint32 * 2)(*key), o)
    assert list(o) == out


def test_sampling_equal_distributions_accept_all(orc):
    rng = np.random.default_rng(2)
    for t in range(50):
        lg = rng.normal(0, 2, (4, 100)).astype(np.float32)
        drafts = rng.integers(0, 100, 3)
        a, nxt = orc.accept_sampled(lg, lg[:3], drafts, 0.7, 11, 0, t)
        assert a == 3


def test_sampling_impossible_draft_rejected(orc):
    rng = np.random.default_rng(3)
    tl = rng.normal(0, 1, (4, 50)).astype(np.float32)
    dl = rng.normal(0, 1, (3, 50)).astype(np.float32)
    tl[0, 7] = -1e4   # p(7) == 0 after exp underflow, q(7) > 0
    for t in range(20):
        a, nxt = orc.accept_sampled(tl, dl, [7, 1, 2], 0.7, 5, 1, t)
        assert a == 0 and nxt != 7


def test_sampling_output_follows_target(orc):
    """The first emitted token is distributed as p_0 whatever q is (speculative sampling)."""
    rng = np.random.default_rng(4)
    V, T = 8, 0.7
    tl = rng.normal(0, 1, (2, V)).astype(np.float32)
    dl = rng.normal(0, 1, (1, V)).astype(np.float32)
    q = np.exp(dl[0] / T)
    q /= q.sum()
    p = np.exp(tl[0] / T)
    p /= p.sum()
    n = 20000
    counts = np.zeros(V)
    for t in range(n):
        d = int(rng.choice(V, p=q))
        a, nxt = orc.accept_sampled(tl, dl, [d], T, 99, 0, t)
        counts[d if a == 1 else nxt] += 1
    chi = stats.chisquare(counts, p * n)
    assert chi.pvalue > 1e-4, (counts, p * n)
