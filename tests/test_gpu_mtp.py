"""MTP draft head (q38_mtp_*, include/q38.h) against the CPU oracle composed from its pinned
functions — embedding, RMSNorm, Q8 head logits, the synthetic MoE layer, residual add, Q4 head
logits — in the order of the reference's draft step: combine_inputs on the non-fused path
(src/mtp_head.cpp:223-267: T(W_e . rms(embed(t)) ) + T(W_h . rms(stream))), the head's decoder
block (its SparseMoe is layer 48, src/sparse_moe.cpp:376-381), the final norm and the draft LM
head (forward_decode, src/mtp_head.cpp:454-470); the greedy chain (draft_lazy_chain,
src/mtp_runner.cpp:152-211) against a host replay of single steps; the row argmax
(greedy_from_logits, src/mtp_verifier.cpp:20-55) against numpy's first-maximum rule."""
import ctypes as C

import numpy as np
import pytest

import gpu_util as G
import oracle_lib
from moe_cases import SEED, bf16_ulps, tol_check

pytestmark = pytest.mark.gpu

H, V = 2048, 151936


@pytest.fixture(scope="module")
def head(gpu, q38):
    m = q38.MtpHead(gpu, q38.desc(), V, SEED)
    yield m
    m.close()


def stream_rows(orc, M, salt=0):
    """Pre-norm residual rows of the magnitude the target's stream has (sums of embeddings)."""
    a = orc.bf16_to_f32(orc.embed(SEED, [900 + 7 * i + salt for i in range(M)], H))
    b = orc.bf16_to_f32(orc.embed(SEED, [3000 + 11 * i + salt for i in range(M)], H))
    return orc.bf16((3.0 * a + 2.0 * b).astype(np.float32))


def step(q38, head, stream, tokens, trace=True):
    M = len(tokens)
    s_in = G.to_dev(stream)
    t_in = G.to_dev(np.asarray(tokens, np.uint32))
    logits = G.empty((M, V), np.float32)
    s_out = G.empty((M, H), np.uint16)
    comb, fin = G.empty((M, H), np.uint16), G.empty((M, H), np.uint16)
    tr = q38.MtpTrace(comb.data_ptr(), fin.data_ptr()) if trace else None
    ws = G.workspace(head.workspace_size(M))
    q38.check(q38.lib.q38_mtp_forward_decode(head.h, s_in.data_ptr(), t_in.data_ptr(), M, logits.data_ptr(),
                                             s_out.data_ptr(), C.byref(tr) if tr else None, ws.data_ptr(),
                                             ws.numel(), G.stream()))
    return (G.to_host(logits), G.to_host(s_out, np.uint16), G.to_host(comb, np.uint16),
            G.to_host(fin, np.uint16))


def oracle_combined(q38, orc, stream, tokens):
    ne = orc.rmsnorm(orc.embed(SEED, tokens, H))
    nh = orc.rmsnorm(stream)
    pe = orc.head_q8_synth_logits(SEED ^ q38.Q38_MTP_FC_EMBED_SALT, H, ne, 0, H)
    ph = orc.head_q8_synth_logits(SEED ^ q38.Q38_MTP_FC_HIDDEN_SALT, H, nh, 0, H)
    t = lambda v: orc.bf16_to_f32(orc.bf16(v)).astype(np.float64)
    return orc.bf16((t(pe) + t(ph)).astype(np.float32)), pe, ph


@pytest.mark.parametrize("M", [1, 2, 4])
def test_draft_step_vs_oracle(q38, orc, head, M):
    stream = stream_rows(orc, M)
    tokens = [17 + 1000 * i for i in range(M)]
    logits, s_out, comb, fin = step(q38, head, stream, tokens)
    # combine_inputs: the Q8 projections' fast pass is within ~1e-6 relative of the exact
    # contract, so the bf16 join differs by at most one ulp, and rarely
    want_x, pe, ph = oracle_combined(q38, orc, stream, tokens)
    ulps = bf16_ulps(orc, comb, want_x)
    assert ulps.max() <= 1 and (ulps > 0).mean() < 0.01, (ulps.max(), (ulps > 0).mean())
    assert np.abs(pe).max() > 0.1 and np.abs(ph).max() > 0.1  # both inputs reach the join
    # the decoder block on the GPU's combined rows: x + MoE(rms(x)) (layer 48 of the seed)
    d = oracle_lib.make_desc()
    y = orc.moe_layer_synth(d, SEED, 48, orc.rmsnorm(comb))[0]
    tol_check(orc, s_out, orc.residual_add(comb, y))
    # final norm of the output stream, then the draft LM head on the GPU's final rows
    assert bf16_ulps(orc, fin, orc.rmsnorm(s_out)).max() <= 1
    want = orc.head_q4_synth_logits(SEED, H, fin)
    assert np.abs(logits - want).max() <= 1e-4 * np.abs(want).max() + 1e-5


def test_stream_and_token_both_matter(q38, orc, head):
    """Changing only the stream or only the token changes the combined row (both FC inputs
    are wired), and identical inputs give identical rows."""
    s = stream_rows(orc, 1)
    _, _, c0, _ = step(q38, head, s, [5])
    _, _, c1, _ = step(q38, head, stream_rows(orc, 1, salt=1), [5])
    _, _, c2, _ = step(q38, head, s, [6])
    _, _, c3, _ = step(q38, head, s, [5])
    assert not np.array_equal(c0, c1) and not np.array_equal(c0, c2) and np.array_equal(c0, c3)


@pytest.mark.parametrize("M", [1, 3, 4])
def test_greedy_chain_equals_step_replay(q38, orc, head, M):
    depth = 3
    stream = stream_rows(orc, M, salt=2)
    tokens = [40 + 313 * i for i in range(M)]
    drafts = G.empty((M, depth), np.uint32)
    s_last = G.empty((M, H), np.uint16)
    ws = G.workspace(head.workspace_size(M))
    s_dev, t_dev = G.to_dev(stream), G.to_dev(np.asarray(tokens, np.uint32))  # alive until the chain ran
    q38.check(q38.lib.q38_mtp_draft_greedy(head.h, s_dev.data_ptr(), t_dev.data_ptr(), M, depth, drafts.data_ptr(),
                                           s_last.data_ptr(), ws.data_ptr(), ws.numel(), G.stream()))
    got = G.to_host(drafts).view(np.uint32)
    # replay: single steps, argmax on the host (first maximum), output stream fed back
    s, t = stream, list(tokens)
    for k in range(depth):
        logits, s_out, _, fin = step(q38, head, s, t, trace=True)
        nxt = np.argmax(logits, axis=1)
        assert np.array_equal(got[:, k], nxt), (k, got[:, k], nxt)
        # the oracle's logits on the same final rows pick the same token unless near-tied
        want = orc.head_q4_synth_logits(SEED, H, fin)
        top2 = np.sort(want, axis=1)[:, -2:]
        for r in range(M):
            if top2[r, 1] - top2[r, 0] > 2.5e-4 * np.abs(want[r]).max() + 3e-5:  # beyond twice the error bound
                assert np.argmax(want[r]) == nxt[r]
        s, t = s_out, [int(v) for v in nxt]
    assert np.array_equal(G.to_host(s_last, np.uint16), s)


@pytest.mark.parametrize("V_", [1, 255, 256, 257, 4099, 151936])
def test_argmax_rows_ties_lowest(q38, V_):
    rng = np.random.default_rng(V_)
    M = 5 if V_ > 1 else 64
    lg = rng.normal(0, 1, (M, V_)).astype(np.float32)
    for r in range(M):
        if V_ >= 4:
            a, b = sorted(rng.choice(V_, 2, replace=False))
            lg[r, a] = lg[r, b] = lg[r].max() + 1.0  # a planted tie: the lower index wins
    lg[0, :] = -np.inf if V_ > 1 else lg[0, :]
    if V_ > 1:
        lg[0, V_ // 2] = -1e30
    idx, val = G.empty(M, np.uint32), G.empty(M, np.float32)
    ws = G.workspace(8 * M)
    lg_dev = G.to_dev(lg)
    q38.check(q38.lib.q38_argmax_rows(lg_dev.data_ptr(), M, V_, idx.data_ptr(), val.data_ptr(), ws.data_ptr(),
                                      ws.numel(), G.stream()))
    got = G.to_host(idx).view(np.uint32)
    assert np.array_equal(got, np.argmax(lg, axis=1))
    assert np.array_equal(G.to_host(val), lg[np.arange(M), np.argmax(lg, axis=1)])


def test_validation(q38, orc, gpu, head):
    lib = q38.lib
    ws = G.workspace(head.workspace_size(4))
    s = G.to_dev(stream_rows(orc, 4))
    t = G.to_dev(np.arange(4, dtype=np.uint32))
    d = G.empty((4, 3), np.uint32)
    assert head.workspace_size(5) == 0 and head.workspace_size(0) == 0
    assert lib.q38_mtp_forward_decode(head.h, s.data_ptr(), t.data_ptr(), 5, None, None, None, ws.data_ptr(),
                                      ws.numel(), G.stream()) == q38.Q38_EINVAL
    assert lib.q38_mtp_draft_greedy(head.h, s.data_ptr(), t.data_ptr(), 4, 0, d.data_ptr(), None, ws.data_ptr(),
                                    ws.numel(), G.stream()) == q38.Q38_EINVAL
    assert lib.q38_mtp_draft_greedy(head.h, s.data_ptr(), t.data_ptr(), 4, 3, d.data_ptr(), None, ws.data_ptr(),
                                    head.workspace_size(3), G.stream()) == q38.Q38_ESPACE
    layer, fe, fh, dh = head.parts()
    out = C.c_void_p()
    # components in the wrong roles are rejected
    assert lib.q38_mtp_head_create(gpu.h, layer, dh, fh, dh, SEED, 1e-6, C.byref(out)) == q38.Q38_EINVAL
    assert lib.q38_mtp_head_create(gpu.h, layer, fe, fh, fe, SEED, 1e-6, C.byref(out)) == q38.Q38_EINVAL
    # the same components borrowed into a second head give the same step
    assert lib.q38_mtp_head_create(gpu.h, layer, fe, fh, dh, SEED, 1e-6, C.byref(out)) == q38.Q38_OK
    try:
        a = step(q38, head, stream_rows(orc, 2), [3, 4])

        class Borrowed:
            h = out
            workspace_size = head.workspace_size

        b = step(q38, Borrowed, stream_rows(orc, 2), [3, 4])
        assert all(np.array_equal(x, y) for x, y in zip(a, b))
    finally:
        lib.q38_mtp_head_destroy(out)
