"""Router (R1, R2) and gather-by-expert plan (R3) of the CPU oracle, pinned by closed
forms, an independent numpy restatement and ordering cases that separate the logit
contract from a naive sequential sum."""
import math

import numpy as np
import pytest


def bf16_values(orc, x):
    return orc.bf16_to_f32(orc.bf16(np.asarray(x, np.float32)))


def test_all_equal_logits(orc):
    ex, wt = orc.route(np.zeros((3, 512), np.float32), 10)
    assert (ex == np.arange(10)).all()
    assert np.allclose(wt, 0.1, rtol=0, atol=1e-7)
    ex, wt = orc.route(np.zeros((1, 512), np.float32), 10, normalize=0)
    assert np.allclose(wt, 1 / 512, rtol=1e-6)


def test_planted_topk_and_ties(orc):
    rng = np.random.default_rng(0)
    lg = bf16_values(orc, rng.normal(0, 0.5, (4, 512)))
    planted = [[7, 400, 3, 99, 511, 0, 256, 128, 64, 32], [1, 2, 3, 4, 5, 6, 7, 8, 9, 10],
               [500, 400, 300, 200, 100, 50, 40, 30, 20, 10], [63, 64, 65, 127, 128, 129, 191, 192, 193, 255]]
    for r, ids in enumerate(planted):
        for rank, e in enumerate(ids):
            lg[r, e] = 8.0 - 0.25 * rank
    ex, wt = orc.route(lg, 10)
    assert ex.tolist() == planted
    assert np.allclose(wt.sum(1), 1.0, atol=1e-6)
    # exact tie between two top experts: the lower index ranks first
    lg2 = np.zeros((1, 512), np.float32)
    lg2[0, 300] = lg2[0, 17] = 5.0
    ex, wt = orc.route(lg2, 10)
    assert ex[0, :2].tolist() == [17, 300] and wt[0, 0] == wt[0, 1]


def numpy_route(lg, k):
    out = []
    for row in lg.astype(np.float64):
        p = np.exp(row - row.max())
        p /= p.sum()
        order = sorted(range(len(row)), key=lambda i: (-p[i], i))[:k]
        w = p[order] / p[order].sum()
        out.append((order, w))
    return out


def test_against_numpy_restatement(orc):
    rng = np.random.default_rng(1)
    for _ in range(20):
        lg = bf16_values(orc, rng.normal(0, 1.0, (4, 512)))
        ex, wt = orc.route(lg, 10)
        for r, (order, w) in enumerate(numpy_route(lg, 10)):
            top = np.sort(lg[r])[::-1]
            if top[9] == top[10]:
                continue  # boundary tie: semantics covered by test_planted_topk_and_ties
            assert set(ex[r].tolist()) == set(order)
            assert np.allclose(wt[r], w[[order.index(e) for e in ex[r]]], rtol=2e-6)


def test_exp_contract_accuracy(orc):
    xs = np.concatenate([np.linspace(-86.9, 0, 20001), -np.logspace(-8, 1.9, 2000)]).astype(np.float32)
    worst = 0.0
    for x in xs:
        got = orc.lib.orc_exp_contract(float(x))
        want = math.exp(float(x))
        worst = max(worst, abs(got - want) / want)
    assert worst < 4 * 2.0 ** -23, worst
    assert orc.lib.orc_exp_contract(-87.5) == 0.0
    assert orc.lib.orc_exp_contract(0.0) == 1.0


def test_logit_contract_vs_float64(orc):
    rng = np.random.default_rng(2)
    x = orc.bf16(rng.normal(0, 1, (4, 2048)))
    W = orc.bf16(rng.normal(0, 0.02, (512, 2048)))
    lg = orc.router_logits(x, W)
    ref = orc.bf16_to_f32(x).astype(np.float64) @ orc.bf16_to_f32(W).astype(np.float64).T
    exact_round = bf16_values(orc, ref.astype(np.float32))
    assert np.mean(lg == exact_round) > 0.99
    assert np.max(np.abs(lg - ref) / np.maximum(np.abs(ref), 1e-3)) < 2 ** -7


def test_logit_contract_order(orc):
    # lane 0 holds 1 (c=0), lane 1 holds 2^24 (c=8), lane 33 holds -2^24 (c=264): the
    # contract's butterfly pairs lanes 1 and 33 first and returns 1; a sequential sum in
    # index order returns 0.
    x = np.zeros(2048, np.float32)
    w = np.zeros(2048, np.float32)
    x[[0, 8, 264]] = 1.0
    w[0], w[8], w[264] = 1.0, 2.0 ** 24, -(2.0 ** 24)
    xb, wb = orc.bf16(x), orc.bf16(w)
    assert orc.lib.orc_dot_contract(xb.ctypes.data, wb.ctypes.data, 2048) == 1.0


def test_plan_closed_form(orc):
    rng = np.random.default_rng(4)
    for M in (1, 2, 4, 16):
        ex = np.stack([rng.choice(64, 10, replace=False) for _ in range(M)]).astype(np.int32)
        n, uexp, uoff, rl, rp = orc.plan(ex, 64)
        flat = ex.reshape(-1)
        assert uexp.tolist() == sorted(set(flat.tolist()))
        assert n == len(uexp) and uoff[-1] == M * 10
        for u, e in enumerate(uexp):
            members = rl[uoff[u]:uoff[u + 1]]
            assert (flat[members] == e).all()
            assert list(members) == sorted(members)          # ascending (row, slot)
            assert (rp[members] == np.arange(uoff[u], uoff[u + 1])).all()
        # stable sort by expert id == the plan's route list
        assert rl.tolist() == sorted(range(M * 10), key=lambda i: (flat[i], i))


def test_router_bias(orc):
    """The additive router bias of the prefill workload: zero bias changes nothing, +100 on
    ten experts selects exactly those, -inf masks an expert; logits = T(x.w) + bias."""
    import oracle_lib
    d = oracle_lib.make_desc(hidden=512, inter=128, experts=64, top_k=4)
    x = orc.rmsnorm(orc.embed(5, list(range(6)), 512))
    y0, ex0, wt0, lg0 = orc.moe_layer_synth(d, 9, 0, x)
    y1, ex1, wt1, lg1 = orc.moe_layer_synth(d, 9, 0, x, bias=np.zeros(64, np.float32))
    assert np.array_equal(lg0.view(np.uint32), lg1.view(np.uint32)) and np.array_equal(y0, y1)
    b = np.zeros(64, np.float32)
    hot = [3, 17, 40, 63]
    b[hot] = 100.0
    _, ex2, _, lg2 = orc.moe_layer_synth(d, 9, 0, x, bias=b)
    assert all(sorted(r) == hot for r in ex2.tolist())
    assert np.array_equal(lg2, lg0 + b)
    m = np.zeros(64, np.float32)
    m[ex0[:, 0]] = -np.inf
    _, ex3, _, _ = orc.moe_layer_synth(d, 9, 0, x, bias=m)
    assert not np.isin(ex3, ex0[:, 0]).any()


def test_zipf_workload_shape():
    """Zipf(1.1) bias: a permutation of -s tau ln(rank) over all experts."""
    from workloads import zipf_router_bias
    b = zipf_router_bias(512, 7)
    assert b.dtype == np.float32 and b.shape == (512,)
    assert np.allclose(np.sort(b)[::-1], -1.1 * 0.28 * np.log(np.arange(1, 513)), atol=1e-6)
    assert np.array_equal(b, zipf_router_bias(512, 7)) and not np.array_equal(b, zipf_router_bias(512, 8))
