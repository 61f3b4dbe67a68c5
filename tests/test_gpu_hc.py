"""HyperConnection mixer on the GPU through the C ABI, against the CPU oracle.

read (q38_hc_read): the normalised streams and the rank activations within one bf16 step of
the oracle (their float accumulation order differs from the oracle's double dots), the block
input `mixed` within the MoE bar (relative L2 <= 1e-2, max |diff| <= 2e-2) and the injection
gates within one bf16 step. write and initialize_stream are elementwise float steps and are
compared bit for bit. Reference: src/hyper_connection.cpp:298-307, 309-493, 692-709.
"""
from __future__ import annotations

import numpy as np
import pytest

import gpu_util as G
from test_oracle_hc import bf, random_case, to_bf16_bits, ulp_diff

pytestmark = pytest.mark.gpu


def build(q38, gpu, rng, H=2048, HC=4, R=256, bits=4, Gs=64, inj=True):
    d, w, _ = random_case(rng, H=H, HC=HC, R=R, bits=bits, G=Gs, inj=inj, M=1)
    dev = {k: G.to_dev(v) for k, v in w.items()}
    hc = q38.Hc(gpu, q38.HcDesc(H, HC, R, bits, Gs, 1 if inj else 0, d.eps), dev)
    return d, w, hc


def gpu_read(q38, hc, d, stream_np):
    M = stream_np.shape[0]
    K = d.streams * d.hidden
    st = G.to_dev(stream_np)
    mixed = G.empty((M, d.hidden), np.uint16)
    inj = G.empty((M, d.streams), np.uint16) if d.with_injection else None
    ws = G.workspace(hc.workspace_size(M))
    hc.read(st, M, mixed, inj, ws, G.stream())
    raw = G.to_host(ws)
    xn = raw[: M * K * 2].view(np.uint16).reshape(M, K)
    off = (M * K * 2 + 255) // 256 * 256
    act = raw[off: off + M * d.rank * 4].view(np.float32).reshape(M, d.rank)
    return (G.to_host(mixed, np.uint16), G.to_host(inj, np.uint16) if inj is not None else None, xn, act)


def check_read(orc, d, w, stream_np, got):
    mixed, inj, xn, act = got
    m_ref, i_ref, xn_ref, act_ref = orc.hc_read(d, w, stream_np)
    u = ulp_diff(xn, xn_ref)
    assert u.max() <= 1 and (u > 0).mean() <= 1e-3, (u.max(), (u > 0).mean())
    ua = ulp_diff(to_bf16_bits(act), to_bf16_bits(act_ref))
    assert ua.max() <= 2 and (ua > 0).mean() <= 2e-2, (ua.max(), (ua > 0).mean())
    a, b = bf(mixed).astype(np.float64), bf(m_ref).astype(np.float64)
    rel = np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)
    assert rel <= 1e-2 and np.abs(a - b).max() <= 2e-2, (rel, np.abs(a - b).max())
    assert (ulp_diff(mixed, m_ref) > 0).mean() <= 5e-2
    if d.with_injection:
        assert ulp_diff(inj, i_ref).max() <= 1


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 16])
def test_hc_read_rows(gpu, q38, orc, M):
    """H 2048, 4 streams, rank 256, 4-bit groups of 64 (the decoder mixers' geometry)."""
    rng = np.random.default_rng(500 + M)
    d, w, hc = build(q38, gpu, rng)
    try:
        stream = to_bf16_bits(rng.normal(0, 1.0, (M, d.streams * d.hidden)).astype(np.float32))
        check_read(orc, d, w, stream, gpu_read(q38, hc, d, stream))
    finally:
        hc.close()


@pytest.mark.parametrize("H,HC,R,bits,Gs,inj,M", [
    (2048, 4, 256, 8, 64, True, 4),     # 8-bit projections
    (2048, 4, 256, 4, 32, True, 3),     # 32-input groups
    (2560, 4, 128, 4, 64, True, 4),     # the reference family's hidden size
    (2048, 5, 256, 4, 64, True, 4),     # 5 streams: the 10240-wide stream of the MTP head
    (2048, 4, 512, 4, 128, False, 2),   # widest rank, no injection (the final mixer)
    (1024, 1, 64, 8, 32, True, 16),     # one stream
    (4096, 8, 256, 4, 64, True, 5),     # widest stream (32768 values)
])
def test_hc_read_geometries(gpu, q38, orc, H, HC, R, bits, Gs, inj, M):
    rng = np.random.default_rng(H + 7 * HC + R + bits + Gs + M)
    d, w, hc = build(q38, gpu, rng, H=H, HC=HC, R=R, bits=bits, Gs=Gs, inj=inj)
    try:
        stream = to_bf16_bits(rng.normal(0, 1.0, (M, HC * H)).astype(np.float32))
        check_read(orc, d, w, stream, gpu_read(q38, hc, d, stream))
    finally:
        hc.close()


def test_hc_read_scaled_streams(gpu, q38, orc):
    """Streams of very different scales (1e-3 .. 1e3) normalise to the same range."""
    rng = np.random.default_rng(11)
    d, w, hc = build(q38, gpu, rng)
    try:
        K = d.streams * d.hidden
        x = rng.normal(0, 1.0, (4, K)).astype(np.float32)
        x *= np.repeat(np.array([1e-3, 1.0, 30.0, 1e3], np.float32), d.hidden)[None, :]
        stream = to_bf16_bits(x)
        check_read(orc, d, w, stream, gpu_read(q38, hc, d, stream))
    finally:
        hc.close()


@pytest.mark.parametrize("M", [1, 4, 16, 33])
def test_hc_write_bit_exact(gpu, q38, orc, M):
    rng = np.random.default_rng(900 + M)
    d, w, hc = build(q38, gpu, rng)
    try:
        H, HC = d.hidden, d.streams
        stream = to_bf16_bits(rng.normal(0, 1.0, (M, HC * H)).astype(np.float32))
        block = to_bf16_bits(rng.normal(0, 0.5, (M, H)).astype(np.float32))
        gates = to_bf16_bits(rng.uniform(0, 2, (M, HC)).astype(np.float32))
        s_d, b_d, g_d = G.to_dev(stream), G.to_dev(block), G.to_dev(gates)
        out = G.empty((M, HC * H), np.uint16)
        hc.write(s_d, b_d, g_d, M, out, G.stream())
        assert np.array_equal(G.to_host(out, np.uint16), orc.hc_write(H, HC, stream, block, gates))
        hc.write(s_d, b_d, g_d, M, s_d, G.stream())  # in place
        assert np.array_equal(G.to_host(s_d, np.uint16), orc.hc_write(H, HC, stream, block, gates))
    finally:
        hc.close()


def test_hc_initialize_stream(gpu, q38):
    rng = np.random.default_rng(3)
    for M, H, HC in ((1, 2048, 4), (5, 2560, 4), (3, 64, 2)):
        emb = to_bf16_bits(rng.normal(0, 1.0, (M, H)).astype(np.float32))
        out = G.empty((M, HC * H), np.uint16)
        q38.check(q38.lib.q38_hc_initialize_stream(G.to_dev(emb).data_ptr(), M, H, HC, out.data_ptr(), G.stream()))
        assert np.array_equal(G.to_host(out, np.uint16), np.tile(emb, (1, HC)))


def test_hc_read_then_write_round(gpu, q38, orc):
    """One mixer round as the decoder runs it (read -> block -> write) with an identity block
    (block output = mixed): the GPU stream after the write stays within one bf16 step of the
    oracle's."""
    rng = np.random.default_rng(21)
    d, w, hc = build(q38, gpu, rng)
    try:
        M, H, HC = 4, d.hidden, d.streams
        stream = to_bf16_bits(rng.normal(0, 1.0, (M, HC * H)).astype(np.float32))
        mixed, inj, _, _ = gpu_read(q38, hc, d, stream)
        out = G.empty((M, HC * H), np.uint16)
        hc.write(G.to_dev(stream), G.to_dev(mixed), G.to_dev(inj), M, out, G.stream())
        m_ref, i_ref, _, _ = orc.hc_read(d, w, stream)
        ref = orc.hc_write(H, HC, stream, m_ref, i_ref)
        u = ulp_diff(G.to_host(out, np.uint16), ref)
        assert u.max() <= 2 and (u > 0).mean() <= 2e-2
    finally:
        hc.close()


def test_hc_rejects(gpu, q38):
    rng = np.random.default_rng(1)
    d, w, hc = build(q38, gpu, rng)
    try:
        bad = [q38.HcDesc(2000, 4, 256, 4, 64, 1, 1e-6), q38.HcDesc(2048, 17, 256, 4, 64, 1, 1e-6),
               q38.HcDesc(2048, 4, 256, 3, 64, 1, 1e-6), q38.HcDesc(2048, 4, 200, 4, 64, 1, 1e-6),
               q38.HcDesc(2048, 4, 1024, 4, 64, 1, 1e-6), q38.HcDesc(2048, 4, 256, 4, 48, 1, 1e-6),
               q38.HcDesc(2048, 4, 256, 4, 64, 1, 0.0)]
        for bd in bad:
            with pytest.raises(q38.Q38Error) as e:
                q38.Hc(gpu, bd, hc._keep)
            assert e.value.code == q38.Q38_EINVAL
        K = d.streams * d.hidden
        st = G.to_dev(np.zeros((17, K), np.uint16))
        mixed = G.empty((17, d.hidden), np.uint16)
        inj = G.empty((17, d.streams), np.uint16)
        ws = G.workspace(hc.workspace_size(16))
        with pytest.raises(q38.Q38Error) as e:
            hc.read(st, 17, mixed, inj, ws, G.stream())
        assert e.value.code == q38.Q38_EINVAL
        small = G.workspace(hc.workspace_size(4) - 256)
        with pytest.raises(q38.Q38Error) as e:
            hc.read(st, 4, mixed, inj, small, G.stream())
        assert e.value.code == q38.Q38_ESPACE
        with pytest.raises(q38.Q38Error) as e:
            hc.read(st, 4, mixed, None, ws, G.stream())  # this mixer returns an injection
        assert e.value.code == q38.Q38_EINVAL
    finally:
        hc.close()


def chain_hc(q38, layers, mixers, stream_np):
    import ctypes as C
    M = stream_np.shape[0]
    st = G.to_dev(stream_np)
    d, hd = layers[0].desc, mixers[0].desc
    ws = G.workspace(q38.lib.q38_verify_chain_hc_workspace_size(C.byref(d), C.byref(hd), M))
    la = (C.c_void_p * len(layers))(*[L.h.value for L in layers])
    ma = (C.c_void_p * len(mixers))(*[h.h.value for h in mixers])
    q38.check(q38.lib.q38_verify_chain_hc(la, ma, len(layers), st.data_ptr(), M, ws.data_ptr(), ws.numel(),
                                          G.stream()))
    return G.to_host(st, np.uint16)


@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_chain_hc_fused_tail_equals_split_path(gpu, q38, M):
    """At 1-4 rows the HC chain's MoE is the fused gate/up + down kernel whose combine tail
    writes the streams; with the fused kernel switched off the same chain takes the split
    kernels and k_combine_hc. Both give the same streams bit for bit over 2 layers."""
    from moe_cases import SEED
    rng = np.random.default_rng(90 + M)
    layers = [q38.MoeLayer(gpu, q38.desc(), seed=SEED, layer=l) for l in range(2)]
    built = [build(q38, gpu, rng) for _ in range(2)]
    mixers = [b[2] for b in built]
    try:
        stream = to_bf16_bits(rng.normal(0, 1.0, (M, 4 * 2048)).astype(np.float32))
        fused = chain_hc(q38, layers, mixers, stream)
        q38.lib.q38_set_fused_layers(0)
        try:
            split = chain_hc(q38, layers, mixers, stream)
        finally:
            q38.lib.q38_set_fused_layers(1)
        assert np.array_equal(fused, split)
        assert not np.array_equal(fused, stream)
    finally:
        for L in layers:
            L.close()
        for h in mixers:
            h.close()


def test_chain_hc_layers(gpu, q38, orc):
    """The decoder's MLP half over 3 layers (mixer read -> MoE -> mixer write) at 4 rows:
    the fused chain equals the layer-by-layer composition of q38_hc_read, q38_moe_forward and
    q38_hc_write bit for bit, and each layer, fed the GPU's own stream (teacher forcing),
    matches the oracle's read -> MoE -> write: routing of the GPU's block input bit-exact,
    the block input within one bf16 step, the new stream within the MoE bar."""
    import ctypes as C
    import oracle_lib
    from moe_cases import SEED, tol_check
    rng = np.random.default_rng(77)
    M, NL = 4, 3
    layers = [q38.MoeLayer(gpu, q38.desc(), seed=SEED, layer=l) for l in range(NL)]
    built = [build(q38, gpu, rng) for _ in range(NL)]
    mixers = [b[2] for b in built]
    try:
        d0, H, HC = built[0][0], 2048, 4
        stream = to_bf16_bits(rng.normal(0, 1.0, (M, HC * H)).astype(np.float32))
        fused = chain_hc(q38, layers, mixers, stream)
        s = stream
        od = oracle_lib.make_desc()
        for l in range(NL):
            d, w, hc = built[l]
            mixed, inj, _, _ = gpu_read(q38, hc, d, s)
            x_d = G.to_dev(mixed)
            y = G.empty((M, H), np.uint16)
            ex = G.empty(M * 10, np.int32)
            wt = G.empty(M * 10, np.float32)
            ws = G.workspace(q38.lib.q38_moe_workspace_size(C.byref(layers[l].desc), M))
            r = q38.routes(experts=ex, weights=wt)
            q38.check(q38.lib.q38_moe_forward(layers[l].h, x_d.data_ptr(), M, y.data_ptr(), C.byref(r),
                                              ws.data_ptr(), ws.numel(), G.stream()))
            out = G.empty((M, HC * H), np.uint16)
            hc.write(G.to_dev(s), y, G.to_dev(inj), M, out, G.stream())
            s_next = G.to_host(out, np.uint16)
            # oracle, teacher-forced on the GPU's stream s
            m_ref, i_ref, _, _ = orc.hc_read(d, w, s)
            assert ulp_diff(mixed, m_ref).max() <= 1
            assert ulp_diff(inj, i_ref).max() <= 1
            y_ref, ex_ref, wt_ref, _ = orc.moe_layer_synth(od, SEED, l, mixed)
            assert np.array_equal(G.to_host(ex).reshape(M, 10), ex_ref)
            assert np.array_equal(G.to_host(wt).reshape(M, 10), wt_ref)
            tol_check(orc, G.to_host(y, np.uint16), y_ref)
            tol_check(orc, s_next, orc.hc_write(H, HC, s, y_ref, inj))
            s = s_next
        assert np.array_equal(fused, s)
    finally:
        for L in layers:
            L.close()
        for h in mixers:
            h.close()
