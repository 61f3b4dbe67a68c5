"""Verify tail on the GPU: exact greedy argmax + logit of the Q8 head, fast logits, and
the Q4/g64 draft head, against the CPU oracle."""
import ctypes as C

import numpy as np
import pytest

import gpu_util as G
from moe_cases import SEED, f16, pack_q4

pytestmark = pytest.mark.gpu


def greedy(q38, hd, h_np):
    M = h_np.shape[0]
    h = G.to_dev(h_np)
    am = G.empty(M, np.int32)
    lg = G.empty(M, np.float32)
    ws = G.workspace(hd.workspace_size(M))
    q38.check(q38.lib.q38_head_greedy(hd.h, h.data_ptr(), M, am.data_ptr(), lg.data_ptr(), ws.data_ptr(),
                                      ws.numel(), G.stream()))
    return G.to_host(am).astype(np.uint32), G.to_host(lg)


def logits(q38, hd, h_np):
    M = h_np.shape[0]
    h = G.to_dev(h_np)
    out = G.empty((M, hd.vocab), np.float32)
    ws = G.workspace(hd.workspace_size(M))
    q38.check(q38.lib.q38_head_logits(hd.h, h.data_ptr(), M, out.data_ptr(), ws.data_ptr(), ws.numel(),
                                      G.stream()))
    return G.to_host(out)


def explicit_head(q38, gpu, W, s):
    Wd, sd = G.to_dev(W), G.to_dev(s)
    hd = q38.Head(gpu, q38.Q38_HEAD_Q8, W.shape[0], W.shape[1], weights=Wd, scales=sd)
    hd._keep = (Wd, sd)
    return hd


@pytest.mark.parametrize("M,H", [(1, 2048), (2, 2048), (3, 2048), (4, 2048), (5, 2048), (8, 2048),
                                 (16, 2048), (3, 1024), (16, 1024), (4, 2560), (11, 2560)])
def test_explicit_head_exact(gpu, q38, orc, M, H):
    """Greedy argmax + logit bit-exact against the contract; fast logits within float
    tolerance. Rows 1-4 take the 4-row kernel, 5-16 the 16-row kernel (two tiles per block);
    V = 5000 leaves a ragged last tile."""
    rng = np.random.default_rng(M * 7 + H)
    V = 5000
    W = rng.integers(-127, 128, (V, H)).astype(np.int8)
    s = f16(rng.uniform(1e-4, 1e-3, V))
    h = orc.bf16(rng.normal(0, 1, (M, H)))
    hd = explicit_head(q38, gpu, W, s)
    try:
        am, lg = greedy(q38, hd, h)
        want = orc.head_q8_logits(W, s, h)
        wi, wv = orc.argmax(want)
        assert np.array_equal(am, wi) and np.array_equal(lg, wv)
        fast = logits(q38, hd, h)
        assert np.allclose(fast, want, rtol=1e-4, atol=1e-5)
    finally:
        hd.close()


def test_head_near_ties(gpu, q38, orc):
    rng = np.random.default_rng(11)
    V, H = 4096, 2048
    W = rng.integers(-127, 128, (V, H)).astype(np.int8)
    s = f16(np.full(V, 5e-4))
    h = orc.bf16(rng.normal(0, 1, (4, H)))
    base = orc.head_q8_logits(W, s, h)
    for r in range(4):
        b = int(np.argmax(base[r]))
        dup = (b + 1000 * (r + 1)) % V
        W[dup] = W[b]                         # exact tie: the lower index must win
    W[3000, :] = W[int(np.argmax(base[0]))]
    W[3000, 0] = W[3000, 0] + (1 if W[3000, 0] < 127 else -1)   # a one-step neighbour
    hd = explicit_head(q38, gpu, W, s)
    try:
        am, lg = greedy(q38, hd, h)
        want = orc.head_q8_logits(W, s, h)
        wi, wv = orc.argmax(want)
        assert np.array_equal(am, wi) and np.array_equal(lg, wv)
    finally:
        hd.close()


def test_all_equal_logits_full_fallback(gpu, q38, orc):
    """h = 0 makes every logit 0: all rows are candidates (overflow path), argmax 0."""
    rng = np.random.default_rng(12)
    V, H = 3000, 2048
    W = rng.integers(-127, 128, (V, H)).astype(np.int8)
    s = f16(rng.uniform(1e-4, 1e-3, V))
    hd = explicit_head(q38, gpu, W, s)
    try:
        am, lg = greedy(q38, hd, np.zeros((2, H), np.uint16))
        assert am.tolist() == [0, 0] and lg.tolist() == [0.0, 0.0]
    finally:
        hd.close()


def test_synthetic_full_vocab_exact(gpu, q38, orc):
    hd = q38.Head(gpu, q38.Q38_HEAD_Q8, 151936, 2048, seed=SEED)
    try:
        h = orc.rmsnorm(orc.embed(SEED, [1, 2, 3, 4], 2048))
        am, lg = greedy(q38, hd, h)
        want = orc.head_q8_synth_logits(SEED, 2048, h)
        wi, wv = orc.argmax(want)
        assert np.array_equal(am, wi) and np.array_equal(lg, wv)
    finally:
        hd.close()


def test_q4_draft_head(gpu, q38, orc):
    hd = q38.Head(gpu, q38.Q38_HEAD_Q4G64, 151936, 2048, seed=SEED)
    try:
        h = orc.rmsnorm(orc.embed(SEED, [5, 6, 7], 2048))
        got = logits(q38, hd, h)
        want = orc.head_q4_synth_logits(SEED, 2048, h)
        err = np.abs(got - want)
        assert err.max() <= 1e-4 * np.abs(want).max() + 1e-5
    finally:
        hd.close()


def test_q4_explicit_head_closed_forms(gpu, q38, orc):
    """An explicit Q4/g64 head (caller-owned nibbles and scales) against the oracle's
    explicit-weight path and closed forms: +1/-1 in the low/high nibbles, all -8, one group
    of 7s, one weight at an odd input, random rows (V = 70 leaves a ragged last pass)."""
    H, V = 2048, 70
    rng = np.random.default_rng(41)
    w = rng.integers(-8, 8, (V, H))
    s = rng.uniform(1.6e-3, 1.6e-2, (V, H // 64)).astype(np.float32)
    w[0] = 0
    w[0, 0::2], w[0, 1::2], s[0] = 1, -1, 1.0
    w[1], s[1] = -8, 2.0 ** -(np.arange(H // 64) % 4)
    w[2] = 0
    w[2, 320:384], s[2] = 7, 0.5
    w[3] = 0
    w[3, 1001], s[3] = 3, 0.25
    s16 = f16(s)
    Wp = pack_q4(w)
    h = orc.bf16(rng.normal(0, 1, (4, H)))
    hf = orc.bf16_to_f32(h).astype(np.float64)
    Wd, sd = G.to_dev(Wp), G.to_dev(s16)
    hd = q38.Head(gpu, q38.Q38_HEAD_Q4G64, V, H, weights=Wd, scales=sd)
    try:
        got = logits(q38, hd, h)
        want = orc.head_q4_logits(Wp, s16, h)
        closed = np.stack([hf[:, 0::2].sum(1) - hf[:, 1::2].sum(1),
                           -8 * (hf.reshape(4, 32, 64).sum(2) * s16.view(np.float16).astype(np.float64)[1]).sum(1),
                           3.5 * hf[:, 320:384].sum(1), 0.75 * hf[:, 1001]], 1)
        assert np.allclose(want[:, :4], closed, rtol=1e-6, atol=1e-6)
        err = np.abs(got - want)
        assert err.max() <= 1e-4 * np.abs(want).max() + 1e-5, err.max()
    finally:
        hd.close()


def test_q4_synthetic_tensors_match_generator(gpu, q38, orc):
    """The device-generated draft head: nibbles (low first) equal orc_gen_int4 and the g64
    scales equal the T_DRAFT_S stream, bit for bit, on rows across the vocab."""
    H, V = 2048, 151936
    hd = q38.Head(gpu, q38.Q38_HEAD_Q4G64, V, H, seed=SEED)
    try:
        wp, sp = hd.device_weights()
        for v in (0, 1, 77777, V - 1):
            got = G.d2h(wp + v * (H // 2), H // 2, np.uint8)
            w = np.empty(H, np.int8)
            orc.lib.orc_gen_int4(orc.key(SEED, 0xFFFD, 32), v * H, H, w.ctypes.data)
            assert np.array_equal(got, pack_q4(w[None])[0]), v
        s = G.d2h(sp, V * (H // 64), np.uint16)
        assert np.array_equal(s, orc.uniform_f16(orc.key(SEED, 0xFFFD, 33), 0, V * (H // 64), 1.6e-3, 1.6e-2))
    finally:
        hd.close()


@pytest.mark.parametrize("M,H", [(1, 2048), (4, 2048), (16, 2048), (3, 2560)])
def test_rmsnorm_vs_oracle(gpu, q38, orc, M, H):
    """q38_rmsnorm (the head's input norm) against the oracle's float64 RMSNorm: within one
    bf16 ulp per element (the device sums the squares in float), and exact almost always."""
    from moe_cases import bf16_ulps
    rng = np.random.default_rng(M + H)
    h_np = orc.bf16(rng.normal(0, 1, (M, H)) * np.exp(rng.uniform(-4, 4, (M, 1))))
    h = G.to_dev(h_np)
    y = G.empty((M, H), np.uint16)
    q38.check(q38.lib.q38_rmsnorm(h.data_ptr(), M, H, C.c_float(1e-6), y.data_ptr(), G.stream()))
    got = G.to_host(y, np.uint16)
    ulps = bf16_ulps(orc, got, orc.rmsnorm(h_np))
    assert ulps.max() <= 1 and np.mean(ulps == 0) >= 0.99, (ulps.max(), np.mean(ulps == 0))


def test_head_rows_beyond_limit_rejected(gpu, q38):
    hd = q38.Head(gpu, q38.Q38_HEAD_Q8, 64, 2048, seed=SEED)
    try:
        assert hd.workspace_size(17) == 0
        h = G.empty((17, 2048), np.uint16)
        out = G.empty((17, 64), np.float32)
        ws = G.workspace(hd.workspace_size(16))
        rc = q38.lib.q38_head_logits(hd.h, h.data_ptr(), 17, out.data_ptr(), ws.data_ptr(), ws.numel(), G.stream())
        assert rc == q38.Q38_EINVAL
        rc = q38.lib.q38_head_logits(hd.h, h.data_ptr(), 4, out.data_ptr(), ws.data_ptr(), 16, G.stream())
        assert rc == q38.Q38_ESPACE
    finally:
        hd.close()


def test_head_planes_wide_dynamic_range(gpu, q38, orc):
    """Rows mixing large and tiny magnitudes (the planes cannot hold the tiny ones
    exactly): the measured residual widens the window and the argmax stays exact."""
    rng = np.random.default_rng(21)
    V, H = 4096, 2048
    W = rng.integers(-128, 128, (V, H)).astype(np.int8)
    s = f16(rng.uniform(1e-4, 1e-3, V))
    x = rng.normal(0, 1, (4, H)) * np.exp(rng.uniform(-18, 0, (4, H)))
    x[:, :4] = 40.0
    h = orc.bf16(x)
    hd = explicit_head(q38, gpu, W, s)
    try:
        am, lg = greedy(q38, hd, h)
        want = orc.head_q8_logits(W, s, h)
        wi, wv = orc.argmax(want)
        assert np.array_equal(am, wi) and np.array_equal(lg, wv)
    finally:
        hd.close()


def head_probs(q38, hd, h_np, T, with_probs=True):
    M = h_np.shape[0]
    h = G.to_dev(h_np)
    probs = G.empty((M, hd.vocab), np.float32) if with_probs else None
    stats = G.empty((M, 2), np.float32)
    ws = G.workspace(q38.lib.q38_head_probs_workspace_size(hd.h, M))
    q38.check(q38.lib.q38_head_probs(hd.h, h.data_ptr(), M, T, probs.data_ptr() if with_probs else None,
                                     stats.data_ptr(), ws.data_ptr(), ws.numel(), G.stream()))
    return (G.to_host(probs) if with_probs else None), G.to_host(stats)


def softmax64(L, T):
    z = (L.astype(np.float64) - L.max(axis=1, keepdims=True)) / T
    e = np.exp(z)
    return e / e.sum(axis=1, keepdims=True), e.sum(axis=1)


@pytest.mark.parametrize("kind,rows", [("q8", 4), ("q4", 3)])
@pytest.mark.parametrize("T", [1.0, 0.7])
def test_head_probs_full_vocab(gpu, q38, orc, kind, rows, T):
    """q38_head_probs: the softmax of the head's own logits (q38_head_logits), against a float64
    softmax of those logits; the per-row max is the logits' max bit for bit, the probabilities
    sum to 1, and the stats-only call gives the same stats."""
    k = q38.Q38_HEAD_Q8 if kind == "q8" else q38.Q38_HEAD_Q4G64
    hd = q38.Head(gpu, k, 151936, 2048, seed=SEED)
    try:
        h = orc.rmsnorm(orc.embed(SEED, list(range(30, 30 + rows)), 2048))
        L = logits(q38, hd, h)
        p, st = head_probs(q38, hd, h, T)
        want, wsum = softmax64(L, T)
        assert np.array_equal(st[:, 0], L.max(axis=1))
        assert np.allclose(st[:, 1], wsum, rtol=1e-5, atol=0)
        assert np.abs(p - want).max() <= 1e-5 * want.max()
        assert np.allclose(p.sum(axis=1, dtype=np.float64), 1.0, atol=1e-4)
        _, st2 = head_probs(q38, hd, h, T, with_probs=False)
        assert np.array_equal(st2.view(np.uint32), st.view(np.uint32))
    finally:
        hd.close()


def test_head_probs_closed_forms_and_rejects(gpu, q38):
    """h = 0 gives equal logits: every probability 1 / V, stats (0, V). Temperatures that are
    not positive and finite, and row counts past the head's limit, are rejected."""
    rng = np.random.default_rng(13)
    V, H = 3000, 2048
    W = rng.integers(-127, 128, (V, H)).astype(np.int8)
    s = f16(rng.uniform(1e-4, 1e-3, V))
    hd = explicit_head(q38, gpu, W, s)
    try:
        p, st = head_probs(q38, hd, np.zeros((2, H), np.uint16), 0.5)
        assert np.allclose(p, 1.0 / V, rtol=1e-6) and st[:, 0].tolist() == [0.0, 0.0]
        assert np.allclose(st[:, 1], V, rtol=1e-6)
        h = G.to_dev(np.zeros((2, H), np.uint16))
        stats = G.empty((17, 2), np.float32)
        ws = G.workspace(q38.lib.q38_head_probs_workspace_size(hd.h, 16))
        for T in (0.0, -1.0, float("nan"), float("inf")):
            assert q38.lib.q38_head_probs(hd.h, h.data_ptr(), 2, T, None, stats.data_ptr(), ws.data_ptr(),
                                          ws.numel(), G.stream()) == q38.Q38_EINVAL
        assert q38.lib.q38_head_probs(hd.h, h.data_ptr(), 17, 1.0, None, stats.data_ptr(), ws.data_ptr(),
                                      ws.numel(), G.stream()) == q38.Q38_EINVAL
        assert q38.lib.q38_head_probs(hd.h, h.data_ptr(), 2, 1.0, None, stats.data_ptr(), ws.data_ptr(), 64,
                                      G.stream()) == q38.Q38_ESPACE
        assert q38.lib.q38_head_probs_workspace_size(hd.h, 17) == 0
    finally:
        hd.close()
