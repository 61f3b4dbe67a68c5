"""LM head logit contract (R12), argmax tie semantics (R13), Philox KATs and
rejection-sampling invariants (R16) of the CPU oracle."""
import numpy as np
import pytest
from scipy import stats

from sampling_cases import k3_case, k3_pvalues, softmax_T


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


def _run_rounds(orc, tl, dl, T, n, seed=21):
    k, V = dl.shape
    rng = np.random.default_rng(seed)
    q = softmax_T(dl, T)
    drafts = np.stack([rng.choice(V, size=n, p=q[i]) for i in range(k)], 1)
    res = np.array([orc.accept_sampled(tl, dl, drafts[t], T, 0xC0FFEE, 3, t) for t in range(n)])
    return drafts, res[:, 0], res[:, 1]


def _k3_pvalues(orc, tl, dl, T, n):
    """n oracle rounds of the k = 3 case, checked by sampling_cases.k3_pvalues."""
    drafts, acc, nxt = _run_rounds(orc, tl, dl, T, n)
    return k3_pvalues(tl, dl, T, drafts, acc, nxt)


def test_sampling_k3_every_emitted_token(orc):
    """k = 3: every position of the emitted sequence follows its target row, the residual
    draw at each first rejection (positions 0, 1 and 2) follows norm(max(0, p_i - q_i)),
    the bonus token after three acceptances follows p_3, and each acceptance happens with
    probability sum_x min(p_i(x), q_i(x)) (Leviathan et al. 2023, Theorem 1)."""
    tl, dl, T = k3_case()
    pv, hist = _k3_pvalues(orc, tl, dl, T, 24000)
    assert hist.min() >= 1500, hist          # every accepted count 0..3 is well represented
    bad = {key: v for key, v in pv.items() if v < 1e-4}
    assert not bad, (bad, hist)


@pytest.mark.parametrize("fault,keys", [(1, ("bonus", "pos3")), (2, ("res1", "res2"))])
def test_sampling_k3_planted_wrong_row_fails(orc, fault, keys):
    """The same checks catch a sampler that draws from the wrong row: the bonus token from
    p_{k-1} (fault 1), or the residual after a rejection at i >= 1 from row i - 1 (fault 2)."""
    tl, dl, T = k3_case()
    orc.lib.orc_plant_fault(fault)
    try:
        pv, _ = _k3_pvalues(orc, tl, dl, T, 24000)
    finally:
        orc.lib.orc_plant_fault(0)
    for key in keys:
        assert pv[key] < 1e-12, (key, pv[key])
    # the rows the fault does not touch still pass
    for key in ("res0", "acc0", "acc1", "acc2"):
        assert pv[key] > 1e-4, (key, pv[key])


def _rne_bf16_by_neighbours(f32):
    """float32 -> bf16 bits by choosing the nearer of the two bf16 neighbours in float64
    (ties to the even mantissa, beyond the largest finite value to infinity): a second,
    independent formulation of round-to-nearest-even."""
    out = np.empty(f32.shape, np.uint16)
    for i, v in enumerate(f32.reshape(-1)):
        v = np.float32(v)
        if np.isnan(v):
            out.flat[i] = 0x7FC0 if not np.signbit(v) else 0xFFC0
            continue
        sign = 0x8000 if np.signbit(v) else 0
        a = abs(float(v))
        lo = int(np.array(abs(v), np.float32).view(np.uint32)) >> 16          # truncation toward 0
        lo_v = float(np.array(lo << 16, np.uint32).view(np.float32))
        if lo_v == a:
            out.flat[i] = sign | lo
            continue
        hi = lo + 1
        hi_v = float(np.array(hi << 16, np.uint32).view(np.float32)) if hi < 0x7F80 else float("inf")
        if hi == 0x7F80:   # above the largest finite bf16: halfway point is max + half an ulp
            hi_v = 2.0 ** 128
        dlo, dhi = a - lo_v, hi_v - a
        pick = lo if (dlo < dhi or (dlo == dhi and lo % 2 == 0)) else hi
        out.flat[i] = sign | (0x7F80 if pick >= 0x7F80 else pick)
    return out


def test_residual_add_float32_restatement(orc):
    """orc_residual_add = bf16(float32(h) + float32(y)) with round-to-nearest-even, against
    numpy's IEEE float32 add and a neighbour-comparison rounding; plus closed forms
    (h + 0 = h, h + (-h) = +0, signed zeros, overflow to infinity, inf - inf = NaN, exact
    halfway cases in both directions, subnormals)."""
    rng = np.random.default_rng(33)
    h = orc.bf16(rng.normal(0, 1, 4000) * 10.0 ** rng.integers(-30, 30, 4000))
    y = orc.bf16(rng.normal(0, 1, 4000) * 10.0 ** rng.integers(-30, 30, 4000))
    one = 0x3F80
    special_h = [0x0000, 0x8000, 0x8000, 0x7F7F, 0xFF7F, 0x7F80, 0x0001, 0x8001, 0x0080, one, one, one, 0x4000]
    special_y = [0x8000, 0x8000, 0x0000, 0x7F7F, 0xFF7F, 0xFF80, 0x0001, 0x0003, 0x8001, 0x3B80, 0x3BC0, 0x3C40,
                 0x3C00]
    # 1 + 2^-8 is halfway between 1 and 1 + 2^-7 (ties to 1, even); 1 + 3*2^-9 rounds up
    # to 1 + 2^-7; 1 + 2^-7 + 2^-8 is the next tie (to the even 1 + 2^-6); 2 + 2^-7 is
    # halfway between 2 and 2 + 2^-6 (to 2)
    h = np.concatenate([h, np.array(special_h, np.uint16), h[:500]])
    y = np.concatenate([y, np.array(special_y, np.uint16), (h[:500] ^ 0x8000).astype(np.uint16)])
    got = orc.residual_add(h, y)
    with np.errstate(over="ignore", invalid="ignore"):
        s32 = orc.bf16_to_f32(h) + orc.bf16_to_f32(y)
    want = _rne_bf16_by_neighbours(s32)
    nan = np.isnan(s32)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.isnan(orc.bf16_to_f32(got[nan])).all()
    n0 = 4000
    g = got[n0:n0 + len(special_h)].tolist()
    assert g[0] == 0x0000 and g[1] == 0x8000 and g[2] == 0x0000      # +0 + -0 = +0; -0 + -0 = -0
    assert g[3] == 0x7F80 and g[4] == 0xFF80                          # overflow to +-inf
    assert np.isnan(orc.bf16_to_f32(np.array([g[5]], np.uint16)))[0]  # inf + -inf
    assert g[6] == 0x0002 and g[7] == 0x0002 and g[8] == 0x007F       # subnormal sums are exact
    assert g[9] == one and g[10] == 0x3F81 and g[11] == 0x3F82 and g[12] == 0x4000
    assert (got[-500:] == 0).all()                                   # h + (-h) = +0
    assert np.array_equal(orc.residual_add(h[:4000], np.zeros(4000, np.uint16)),
                          np.where((h[:4000] & 0x7FFF) == 0, 0, h[:4000]).astype(np.uint16))


# ---------------------------------------------------------------- Q4 draft head (R14)
# Device tensor contract of the Q4/g64 head: [V, H/2] bytes, input 2i in the low nibble and
# 2i + 1 in the high nibble, both signed int4; [V, H/64] fp16 scales. The logit is
# sum_g s[v, g] * sum_{c in g} w[c] h[c]. The checks below are chosen so that a swapped
# nibble order, a missing sign extension or a transposed scale index fails one of them.

def _pack_q4(w):
    """[V, H] ints in [-8, 7] -> [V, H/2] bytes, low nibble first."""
    u = (np.asarray(w, np.int64) & 0xF).astype(np.uint8)
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)


def _np_q4_logits(orc, w, s16, h):
    hf = orc.bf16_to_f32(h).astype(np.float64)
    V, H = w.shape
    s = s16.view(np.float16).astype(np.float64).reshape(V, H // 64)
    g = (w.astype(np.float64).reshape(V, H // 64, 64)[None] * hf.reshape(-1, 1, H // 64, 64)).sum(-1)
    return (g * s[None]).sum(-1)


def _close_f32(got, want64):
    want = want64.astype(np.float32)
    return np.all(np.abs(got.astype(np.float64) - want) <= np.spacing(np.abs(want)).astype(np.float64))


def test_q4_explicit_closed_forms(orc):
    H, V = 2048, 6
    rng = np.random.default_rng(40)
    h = orc.bf16(rng.normal(0, 1, (2, H)))
    hf = orc.bf16_to_f32(h).astype(np.float64)
    w = np.zeros((V, H), np.int64)
    s = np.ones((V, H // 64), np.float32)
    w[0, 0::2], w[0, 1::2] = 1, -1                       # +1 low nibble, -1 high nibble
    w[1, :] = -8                                          # the most negative nibble
    s[1] = 2.0 ** -(np.arange(H // 64) % 4)               # a different scale per group
    w[2, 5 * 64:6 * 64] = 7                               # one group only
    s[2] = 0.5
    w[4, 1001] = 3                                        # one weight, odd input (high nibble)
    s[4] = 0.25
    w[5] = rng.integers(-8, 8, H)
    s[5] = rng.uniform(1.6e-3, 1.6e-2, H // 64)
    s16 = s.astype(np.float16).view(np.uint16)
    got = orc.head_q4_logits(_pack_q4(w), s16, h)
    sf = s16.view(np.float16).astype(np.float64)
    closed = np.stack([
        hf[:, 0::2].sum(1) - hf[:, 1::2].sum(1),
        -8 * (hf.reshape(2, H // 64, 64).sum(2) * sf[1]).sum(1),
        3.5 * hf[:, 5 * 64:6 * 64].sum(1),
        np.zeros(2),
        0.75 * hf[:, 1001],
    ], 1)
    assert _close_f32(got[:, :5], closed)
    assert _close_f32(got, _np_q4_logits(orc, w, s16, h))


def _mix64(z):
    z = np.asarray(z, np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def _np_stream_key(seed, layer, tensor):
    g = np.uint64(0x9E3779B97F4A7C15)
    with np.errstate(over="ignore"):
        k = _mix64(_mix64(np.uint64(seed)) + g * np.uint64(layer + 1))
        return _mix64(k + g * np.uint64(tensor + 1))


def test_q4_synthetic_vs_numpy(orc):
    """The synthetic draft head (generator streams T_DRAFT_W / T_DRAFT_S of layer 0xFFFD)
    regenerated in numpy (an independent splitmix64: w = (bits >> 60) - 8, scale = f16 of
    1.6e-3 + u * (1.6e-2 - 1.6e-3)), logits recomputed in float64; and the same weights
    packed as nibbles give the same logits through the explicit-weight path."""
    seed, H, v0, nv = 0x51A5EED, 2048, 151936 - 300, 300
    h = orc.rmsnorm(orc.embed(seed, [5, 6, 7], H))
    got = orc.head_q4_synth_logits(seed, H, h, v0=v0, nv=nv)
    gk = np.uint64(0x9E3779B97F4A7C15)
    wk, sk = _np_stream_key(seed, 0xFFFD, 32), _np_stream_key(seed, 0xFFFD, 33)
    with np.errstate(over="ignore"):
        idx = np.arange(v0 * H, (v0 + nv) * H, dtype=np.uint64)
        w = ((_mix64(wk + gk * (idx + np.uint64(1))) >> np.uint64(60)).astype(np.int64) - 8).reshape(nv, H)
        gi = np.arange(v0 * (H // 64), (v0 + nv) * (H // 64), dtype=np.uint64)
        u = (_mix64(sk + gk * (gi + np.uint64(1))) >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    s16 = (1.6e-3 + u * (1.6e-2 - 1.6e-3)).astype(np.float32).astype(np.float16).view(np.uint16)
    ref = np.empty(nv * H, np.int8)
    orc.lib.orc_gen_int4(orc.key(seed, 0xFFFD, 32), v0 * H, nv * H, ref.ctypes.data)
    assert np.array_equal(ref.reshape(nv, H), w)
    assert np.array_equal(s16, orc.uniform_f16(orc.key(seed, 0xFFFD, 33), v0 * (H // 64), nv * (H // 64),
                                                1.6e-3, 1.6e-2))
    assert _close_f32(got, _np_q4_logits(orc, w, s16, h))
    assert np.array_equal(orc.head_q4_logits(_pack_q4(w), s16, h), got)
