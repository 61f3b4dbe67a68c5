"""The MTP draft head on HC streams (q38_mtp_head_set_streams) against the CPU oracle composed
from its pinned pieces in the reference's order:
- combine_inputs (src/mtp_head.cpp:223-267): the offset norms 1 + w of
  pre_fc_norm_embedding (over H) and pre_fc_norm_hidden (over the row's HC * H values,
  offset_norm at :44-48), the embedding projection, the hidden projection of every stream,
  and the embedding projection added to each stream;
- the head's block as the mixer read -> the layer-48 MoE -> the mixer write;
- the final mixer's read, built without injection as the reference builds it (:153-160), and
  the Q4 draft head (forward_decode, :454-470).

Every stage is checked on the GPU's own input to it. The greedy chain equals a host replay of
single steps bit for bit. The geometry is the reference family's: H 2048 with 5 streams (the
10240-wide stream of :316-318)."""
import ctypes as C

import numpy as np
import pytest

import gpu_util as G
import oracle_lib
from moe_cases import SEED, bf16_ulps, tol_check
from test_oracle_hc import bf, random_case, to_bf16_bits, ulp_diff

pytestmark = pytest.mark.gpu

H, V, HC, R = 2048, 151936, 5, 256


def offset(w_bits):
    """T(1 + w): offset_norm's bf16 sum (src/mtp_head.cpp:44-48)."""
    return to_bf16_bits((1.0 + bf(w_bits)).astype(np.float32))


def weighted_norm(orc, x_bits, w_bits):
    """T(T(rms(x)) * T(1 + w)): the pinned unit-gain RMSNorm, then the weight."""
    n = bf(orc.rmsnorm(x_bits)).astype(np.float32)
    return to_bf16_bits(n * bf(offset(w_bits))[None, :])


@pytest.fixture(scope="module")
def stream_head(gpu, q38):
    rng = np.random.default_rng(77)
    db, wb, _ = random_case(rng, H=H, HC=HC, R=R, bits=4, G=64, inj=True, M=1)
    df, wf, _ = random_case(rng, H=H, HC=HC, R=R, bits=4, G=64, inj=False, M=1)
    block = q38.Hc(gpu, q38.HcDesc(H, HC, R, 4, 64, 1, db.eps), {k: G.to_dev(v) for k, v in wb.items()})
    final = q38.Hc(gpu, q38.HcDesc(H, HC, R, 4, 64, 0, df.eps), {k: G.to_dev(v) for k, v in wf.items()})
    we = to_bf16_bits(rng.normal(0, 0.1, H).astype(np.float32))
    wh = to_bf16_bits(rng.normal(0, 0.1, HC * H).astype(np.float32))
    m = q38.MtpHead(gpu, q38.desc(), V, SEED)
    we_d, wh_d = G.to_dev(we), G.to_dev(wh)
    m.set_streams(block, final, we_d, wh_d)
    yield dict(head=m, block=(db, wb), final=(df, wf), we=we, wh=wh)
    m.close()
    block.close()
    final.close()


def streams_in(orc, M, salt=0):
    """Pre-mixer streams of the target: HC differently scaled copies of embedding sums."""
    rows = []
    for s in range(HC):
        a = orc.bf16_to_f32(orc.embed(SEED, [900 + 7 * i + 31 * s + salt for i in range(M)], H))
        rows.append((1.0 + 0.5 * s) * a)
    return orc.bf16(np.concatenate(rows, axis=1).astype(np.float32))


def step(q38, head, stream, tokens):
    M = len(tokens)
    s_in = G.to_dev(stream)
    t_in = G.to_dev(np.asarray(tokens, np.uint32))
    logits = G.empty((M, V), np.float32)
    s_out = G.empty((M, HC * H), np.uint16)
    comb, fin = G.empty((M, HC * H), np.uint16), G.empty((M, H), np.uint16)
    tr = q38.MtpTrace(comb.data_ptr(), fin.data_ptr())
    ws = G.workspace(head.workspace_size(M))
    q38.check(q38.lib.q38_mtp_forward_decode(head.h, s_in.data_ptr(), t_in.data_ptr(), M, logits.data_ptr(),
                                             s_out.data_ptr(), C.byref(tr), ws.data_ptr(), ws.numel(), G.stream()))
    return (G.to_host(logits), G.to_host(s_out, np.uint16), G.to_host(comb, np.uint16),
            G.to_host(fin, np.uint16))


@pytest.mark.parametrize("M", [1, 2, 4])
def test_stream_step_vs_oracle(q38, orc, stream_head, M):
    sh, head = stream_head, stream_head["head"]
    assert q38.lib.q38_mtp_head_streams(head.h) == HC
    stream = streams_in(orc, M)
    tokens = [17 + 1000 * i for i in range(M)]
    logits, s_out, comb, fin = step(q38, head, stream, tokens)
    # combine_inputs
    ne = weighted_norm(orc, orc.embed(SEED, tokens, H), sh["we"])
    nh = weighted_norm(orc, stream, sh["wh"]).reshape(M * HC, H)
    pe = orc.head_q8_synth_logits(SEED ^ q38.Q38_MTP_FC_EMBED_SALT, H, ne, 0, H)
    ph = orc.head_q8_synth_logits(SEED ^ q38.Q38_MTP_FC_HIDDEN_SALT, H, nh, 0, H)
    t = lambda v: orc.bf16_to_f32(orc.bf16(v)).astype(np.float64)
    want_x = orc.bf16((t(ph).reshape(M, HC, H) + t(pe)[:, None, :]).astype(np.float32)).reshape(M, HC * H)
    ulps = bf16_ulps(orc, comb, want_x)
    assert ulps.max() <= 1 and (ulps > 0).mean() < 0.01, (ulps.max(), (ulps > 0).mean())
    # every stream carries its own hidden projection (the streams differ) and the shared
    # embedding projection
    cs = comb.reshape(M, HC, H)
    assert not np.array_equal(cs[:, 0], cs[:, 1])
    # the block on the GPU's combined rows: read -> MoE (layer 48) -> write
    db, wb = sh["block"]
    mixed, inj, _, _ = orc.hc_read(db, wb, comb)
    y = orc.moe_layer_synth(oracle_lib.make_desc(), SEED, 48, mixed)[0]
    tol_check(orc, s_out, orc.hc_write(H, HC, comb, y, inj))
    # the final mixer's read of the output streams, then the Q4 head on the GPU's final rows
    df, wf = sh["final"]
    fm = orc.hc_read(df, wf, s_out)[0]
    a, b = bf(fin).astype(np.float64), bf(fm).astype(np.float64)
    assert np.linalg.norm(a - b) <= 1e-2 * np.linalg.norm(b) and np.abs(a - b).max() <= 2e-2
    assert (ulp_diff(fin, fm) > 0).mean() <= 5e-2
    want = orc.head_q4_synth_logits(SEED, H, fin)
    assert np.abs(logits - want).max() <= 1e-4 * np.abs(want).max() + 1e-5


@pytest.mark.parametrize("M", [1, 4])
def test_stream_chain_equals_step_replay(q38, orc, stream_head, M):
    head = stream_head["head"]
    depth = 3
    stream = streams_in(orc, M, salt=2)
    tokens = [40 + 313 * i for i in range(M)]
    drafts = G.empty((M, depth), np.uint32)
    s_last = G.empty((M, HC * H), np.uint16)
    ws = G.workspace(head.workspace_size(M))
    s_dev, t_dev = G.to_dev(stream), G.to_dev(np.asarray(tokens, np.uint32))
    q38.check(q38.lib.q38_mtp_draft_greedy(head.h, s_dev.data_ptr(), t_dev.data_ptr(), M, depth, drafts.data_ptr(),
                                           s_last.data_ptr(), ws.data_ptr(), ws.numel(), G.stream()))
    got = G.to_host(drafts).view(np.uint32)
    s, t = stream, list(tokens)
    for k in range(depth):
        logits, s_out, _, _ = step(q38, head, s, t)
        nxt = np.argmax(logits, axis=1)
        assert np.array_equal(got[:, k], nxt), (k, got[:, k], nxt)
        s, t = s_out, [int(v) for v in nxt]
    assert np.array_equal(G.to_host(s_last, np.uint16), s)


def test_stream_validation_and_reset(q38, orc, gpu, stream_head):
    lib = q38.lib
    head = stream_head["head"]
    db, wb = stream_head["block"]
    df, wf = stream_head["final"]
    blk, fnl = head._streams[0], head._streams[1]
    # the mixers' roles: the block mixer carries injection weights, the final one does not
    bad = q38.MtpStreams(fnl.h, fnl.h, None, None)
    assert lib.q38_mtp_head_set_streams(head.h, C.byref(bad)) == q38.Q38_EINVAL
    bad = q38.MtpStreams(blk.h, blk.h, None, None)
    assert lib.q38_mtp_head_set_streams(head.h, C.byref(bad)) == q38.Q38_EINVAL
    # a mixer of another stream count
    rng = np.random.default_rng(5)
    d4, w4, _ = random_case(rng, H=H, HC=4, R=R, bits=4, G=64, inj=False, M=1)
    other = q38.Hc(gpu, q38.HcDesc(H, 4, R, 4, 64, 0, d4.eps), {k: G.to_dev(v) for k, v in w4.items()})
    try:
        bad = q38.MtpStreams(blk.h, other.h, None, None)
        assert lib.q38_mtp_head_set_streams(head.h, C.byref(bad)) == q38.Q38_EINVAL
    finally:
        other.close()
    # failed calls left the stream head as it was
    assert lib.q38_mtp_head_streams(head.h) == HC
    a = step(q38, head, streams_in(orc, 2), [3, 4])
    # zero norm weights (null) equal explicit zeros
    zeros_e, zeros_h = G.to_dev(np.zeros(H, np.uint16)), G.to_dev(np.zeros(HC * H, np.uint16))
    we_d, wh_d = head._streams[2], head._streams[3]
    head.set_streams(blk, fnl, zeros_e, zeros_h)
    b = step(q38, head, streams_in(orc, 2), [3, 4])
    head.set_streams(blk, fnl)
    c = step(q38, head, streams_in(orc, 2), [3, 4])
    assert all(np.array_equal(x, y) for x, y in zip(b, c))
    assert not np.array_equal(a[2], b[2])  # the norm weights reach the join
    # back to the single-stream head and to the stream head again
    head.clear_streams()
    assert lib.q38_mtp_head_streams(head.h) == 1
    head.set_streams(blk, fnl, we_d, wh_d)
    d = step(q38, head, streams_in(orc, 2), [3, 4])
    assert all(np.array_equal(x, y) for x, y in zip(a, d))
