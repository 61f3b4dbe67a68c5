"""Rejection-sampling acceptance on the GPU vs the oracle on identical logits and Philox
uniforms (>= 99.9% identical decisions), and per-slot commit/rollback KATs."""
import ctypes as C

import numpy as np
import pytest

import gpu_util as G
from sampling_cases import k3_case, k3_pvalues, softmax_T

pytestmark = pytest.mark.gpu


def gpu_accept(q38, tl, dl, drafts, T, seed, slot, rnd):
    t, d, dr = G.to_dev(tl), G.to_dev(dl), G.to_dev(np.asarray(drafts, np.uint32))
    out = G.empty(2, np.int64)
    ws = G.workspace(q38.lib.q38_mtp_accept_workspace_size(len(drafts), tl.shape[1]))
    q38.check(q38.lib.q38_mtp_accept_sampled(t.data_ptr(), d.data_ptr(), dr.data_ptr(), len(drafts), tl.shape[1],
                                             T, seed, slot, rnd, out.data_ptr(), ws.data_ptr(), ws.numel(),
                                             G.stream()))
    o = G.to_host(out)
    return int(o[0]), int(o[1])


def test_sampled_decisions_match(gpu, q38, orc):
    rng = np.random.default_rng(0)
    V, k, T = 1000, 3, 0.7
    same = 0
    n = 2000  # the bar: >= 99.9% identical decisions, i.e. at most n // 1000 differences
    for rnd in range(n):
        tl = rng.normal(0, 2, (k + 1, V)).astype(np.float32)
        dl = (tl[:k] + rng.normal(0, 1, (k, V))).astype(np.float32)
        q = np.exp(dl / T)
        q /= q.sum(1, keepdims=True)
        drafts = [int(rng.choice(V, p=q[i])) for i in range(k)]
        same += gpu_accept(q38, tl, dl, drafts, T, 77, 1, rnd) == orc.accept_sampled(tl, dl, drafts, T, 77, 1, rnd)
    print(f"sampled acceptance: {same}/{n} rounds identical to the oracle")
    assert same >= n - n // 1000, same


def test_sampled_k3_distributions_on_device(gpu, q38):
    """The device sampler's own output at k = 3, without the oracle: every emitted position
    follows its target row, each first-rejection draw follows norm(max(0, p_i - q_i)), the
    bonus token follows p_3, and the acceptance rates are sum_x min(p_i, q_i)."""
    tl, dl, T = k3_case()
    k, V = dl.shape
    n = 12000
    rng = np.random.default_rng(22)
    q = softmax_T(dl, T)
    drafts = np.stack([rng.choice(V, size=n, p=q[i]) for i in range(k)], 1)
    t, d = G.to_dev(tl), G.to_dev(dl)
    ws = G.workspace(q38.lib.q38_mtp_accept_workspace_size(k, V))
    dr = G.to_dev(drafts.astype(np.uint32))
    out = G.empty((n, 2), np.int64)
    for r in range(n):
        q38.check(q38.lib.q38_mtp_accept_sampled(t.data_ptr(), d.data_ptr(), dr.data_ptr() + 4 * k * r, k, V, T,
                                                 0xBEEF, 2, r, out.data_ptr() + 16 * r, ws.data_ptr(), ws.numel(),
                                                 G.stream()))
    o = G.to_host(out)
    pv, hist = k3_pvalues(tl, dl, T, drafts, o[:, 0], o[:, 1])
    print("device k=3 sampling p-values:", {key: f"{v:.3g}" for key, v in pv.items()}, "accepted:", hist)
    assert hist.min() >= 700, hist
    bad = {key: v for key, v in pv.items() if v < 1e-4}
    assert not bad, (bad, hist)


def test_sampled_full_vocab(gpu, q38, orc):
    rng = np.random.default_rng(1)
    V, k, T = 151936, 3, 0.7
    for rnd in range(4):
        tl = rng.normal(0, 2, (k + 1, V)).astype(np.float32)
        dl = (tl[:k] + rng.normal(0, 0.5, (k, V))).astype(np.float32)
        drafts = [int(np.argmax(dl[i])) for i in range(k)]
        assert gpu_accept(q38, tl, dl, drafts, T, 5, 0, rnd) == orc.accept_sampled(tl, dl, drafts, T, 5, 0, rnd)


def test_slot_commit_rollback(gpu, q38):
    H = 8
    s = C.c_void_p()
    q38.check(q38.lib.q38_slot_create(gpu.h, H, 5, 99, C.byref(s)))
    try:
        tc, sr, dc = C.c_uint64(), C.c_int32(), C.c_int32()
        assert q38.lib.q38_slot_commit(s, 0, G.stream()) == q38.Q38_ESTATE      # nothing staged
        for accepted in range(5):
            rows = np.repeat(np.arange(5, dtype=np.uint16)[:, None] + 100 * accepted, H, 1)
            rows_dev = G.to_dev(rows)  # alive until the staging copy ran
            q38.check(q38.lib.q38_slot_stage(s, 4, rows_dev.data_ptr(), G.stream()))
            q38.check(q38.lib.q38_slot_info(s, C.byref(tc), C.byref(sr), C.byref(dc)))
            before = tc.value
            assert (sr.value, dc.value) == (5, 4)
            assert q38.lib.q38_slot_commit(s, 5, G.stream()) == q38.Q38_ESTATE   # rejected, state intact
            q38.check(q38.lib.q38_slot_info(s, C.byref(tc), C.byref(sr), C.byref(dc)))
            assert (tc.value, sr.value) == (before, 5)
            q38.check(q38.lib.q38_slot_commit(s, accepted, G.stream()))
            q38.check(q38.lib.q38_slot_info(s, C.byref(tc), C.byref(sr), C.byref(dc)))
            assert tc.value == before + accepted + 1 and sr.value == 0
            hid = G.d2h(q38.lib.q38_slot_hidden(s), H, np.uint16)
            assert (hid == accepted + 100 * accepted).all()
        q38.check(q38.lib.q38_slot_stage(s, 2, G.to_dev(np.zeros((3, H), np.uint16)).data_ptr(), G.stream()))
        q38.check(q38.lib.q38_slot_rollback(s))
        q38.check(q38.lib.q38_slot_info(s, C.byref(tc), C.byref(sr), C.byref(dc)))
        assert sr.value == 0 and q38.lib.q38_slot_commit(s, 0, G.stream()) == q38.Q38_ESTATE
    finally:
        q38.lib.q38_slot_destroy(s)
