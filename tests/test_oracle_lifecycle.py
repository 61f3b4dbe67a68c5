"""Greedy decision (R15) and commit planning (R17): KATs of tests/mtp_lifecycle_test.cpp:39-71
and tests/mlx_backend_test.cpp:711-769, the compiled reference, and the product's host ABI."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib


def product_decide(q38, drafts, target, stop=()):
    d = (C.c_uint32 * max(len(drafts), 1))(*drafts)
    t = (C.c_uint32 * max(len(target), 1))(*target)
    s = (C.c_uint32 * max(len(stop), 1))(*stop)
    out = q38.GreedyDecision()
    rc = q38.lib.q38_mtp_decide_greedy(d, len(drafts), t, len(target), s, len(stop), C.byref(out))
    return rc, out.accepted, out.correction_row, out.next_token


CASES = [
    ([10, 20, 30], [11, 20, 30, 40], (), (0, 0, 11)),
    ([10, 20, 30], [10, 20, 31, 40], (), (2, 2, 31)),
    ([10, 20, 30], [10, 20, 30, 40], (), (3, 3, 40)),
    ([10, 20, 30], [10, 20, 30, 40], (20, 99), (1, 1, 20)),
]


@pytest.mark.parametrize("drafts,target,stop,expect", CASES)
def test_decide_kat(orc, q38, drafts, target, stop, expect):
    assert orc.decide_greedy(drafts, target, stop) == (0, *expect)
    assert product_decide(q38, drafts, target, stop) == (0, *expect)
    ref = oracle_lib.load_ref()
    if ref is not None:
        assert ref.decide_greedy(drafts, target, stop) == (0, *expect)


def test_decide_rejects(orc, q38):
    assert orc.decide_greedy([], [1])[0] != 0
    assert orc.decide_greedy([1, 2], [1, 2])[0] != 0          # missing bonus row
    assert product_decide(q38, [], [1])[0] == q38.Q38_EINVAL
    assert product_decide(q38, [1, 2], [1, 2])[0] == q38.Q38_EINVAL


def test_decide_random_vs_reference(orc, q38):
    ref = oracle_lib.load_ref()
    rng = np.random.default_rng(3)
    for _ in range(500):
        k = int(rng.integers(1, 6))
        target = rng.integers(0, 4, k + 1).tolist()
        drafts = [t if rng.random() < 0.7 else int(rng.integers(0, 4)) for t in target[:k]]
        stop = rng.integers(0, 4, int(rng.integers(0, 3))).tolist()
        o = orc.decide_greedy(drafts, target, stop)
        assert product_decide(q38, drafts, target, stop) == o
        if ref is not None:
            assert ref.decide_greedy(drafts, target, stop) == o


def test_plan_commit_kat(orc, q38):
    assert orc.plan_commit(12, 3, 1) == (0, [12, 2, 2, 14])
    assert orc.plan_commit(0, 1, 2)[0] != 0
    out = (C.c_uint64 * 4)()
    assert q38.lib.q38_plan_mtp_commit(12, 3, 1, out) == 0 and list(out) == [12, 2, 2, 14]
    assert q38.lib.q38_plan_mtp_commit(0, 1, 2, out) == q38.Q38_ESTATE
    ref = oracle_lib.load_ref()
    if ref is not None:
        for off, dr, ac in [(12, 3, 1), (0, 4, 4), (100, 3, 0), (0, 1, 2)]:
            assert ref.plan_commit(off, dr, ac) == orc.plan_commit(off, dr, ac)
