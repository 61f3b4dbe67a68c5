"""The decoder's MLP output map on the GPU (q38_mlp_output_map; DecoderLayer::
apply_mlp_output_map, src/decoder_layer.cpp:198-210) and the decoder's MLP half with it
(q38_verify_chain_hc_mapped, :494-497):
- full and low-rank maps equal the oracle bit for bit at 1, 4 and 16 rows;
- the mapped chain equals the composition of its own calls bit for bit: per layer
  q38_hc_read -> q38_moe_forward -> q38_mlp_output_map -> q38_hc_write (and the fused step for
  a layer without a map);
- with no maps it equals q38_verify_chain_hc bit for bit;
- bad map geometry is refused with the reference's messages."""
import ctypes as C

import numpy as np
import pytest

import gpu_util as G
from affine_cases import to16
from moe_cases import SEED
from test_gpu_hc import build, chain_hc, gpu_read
from test_oracle_hc import to_bf16_bits

pytestmark = pytest.mark.gpu

H = 2048


class DevMap:
    def __init__(self, q38, full=None, left=None, right=None):
        self.keep = [None if a is None else G.to_dev(a) for a in (full, left, right)]
        ptr = lambda t: None if t is None else t.data_ptr()
        rank = 0 if full is not None else left.shape[1]
        self.m = q38.MlpMap(H, rank, *[ptr(t) for t in self.keep])


def maps_for(rng, kind):
    if kind == "full":
        return dict(full=to16(rng.normal(0, 1 / np.sqrt(H), (H, H)), 0))
    R = 128
    return dict(left=to16(rng.normal(0, 1 / np.sqrt(H), (H, R)), 0),
                right=to16(rng.normal(0, 0.1 / np.sqrt(R), (R, H)), 0))


def run_map(q38, dm, y):
    M = y.shape[0]
    yd, out = G.to_dev(y), G.empty((M, H), np.uint16)
    ws = G.workspace(q38.lib.q38_mlp_map_workspace_size(C.byref(dm.m), M))
    q38.check(q38.lib.q38_mlp_output_map(C.byref(dm.m), yd.data_ptr(), M, out.data_ptr(), ws.data_ptr(), ws.numel(),
                                         G.stream()))
    return G.to_host(out, np.uint16)


@pytest.mark.parametrize("kind", ["full", "low_rank"])
@pytest.mark.parametrize("M", [1, 4, 16])
def test_map_equals_oracle(gpu, q38, orc, kind, M):
    rng = np.random.default_rng(M + (7 if kind == "full" else 0))
    mp = maps_for(rng, kind)
    y = to16(rng.normal(0, 1, (M, H)), 0)
    got = run_map(q38, DevMap(q38, **mp), y)
    assert np.array_equal(got, orc.mlp_map(y, **mp))


def chain_mapped(q38, layers, mixers, maps, stream_np):
    M = stream_np.shape[0]
    st = G.to_dev(stream_np)
    ws = G.workspace(q38.lib.q38_verify_chain_hc_mapped_workspace_size(C.byref(layers[0].desc),
                                                                       C.byref(mixers[0].desc), M))
    la = (C.c_void_p * len(layers))(*[L.h.value for L in layers])
    ma = (C.c_void_p * len(mixers))(*[h.h.value for h in mixers])
    pa = None if maps is None else (C.POINTER(q38.MlpMap) * len(maps))(
        *[C.POINTER(q38.MlpMap)() if m is None else C.pointer(m.m) for m in maps])
    q38.check(q38.lib.q38_verify_chain_hc_mapped(la, ma, pa, len(layers), st.data_ptr(), M, ws.data_ptr(), ws.numel(),
                                                 G.stream()))
    return G.to_host(st, np.uint16)


def test_mapped_chain_equals_its_calls(gpu, q38):
    rng = np.random.default_rng(91)
    M, NL = 4, 3
    layers = [q38.MoeLayer(gpu, q38.desc(), seed=SEED, layer=l) for l in range(NL)]
    built = [build(q38, gpu, rng) for _ in range(NL)]
    mixers = [b[2] for b in built]
    maps = [DevMap(q38, **maps_for(rng, "full")), None, DevMap(q38, **maps_for(rng, "low_rank"))]
    try:
        HC = built[0][0].streams
        stream = to_bf16_bits(rng.normal(0, 1.0, (M, HC * H)).astype(np.float32))
        # no maps: the plain chain, bit for bit
        assert np.array_equal(chain_mapped(q38, layers, mixers, None, stream), chain_hc(q38, layers, mixers, stream))
        got = chain_mapped(q38, layers, mixers, maps, stream)
        s = stream
        for l in range(NL):
            if maps[l] is None:
                s = chain_hc(q38, layers[l:l + 1], mixers[l:l + 1], s)
                continue
            d, w, hc = built[l]
            mixed, inj, _, _ = gpu_read(q38, hc, d, s)
            x_d = G.to_dev(mixed)
            y = G.empty((M, H), np.uint16)
            ws = G.workspace(q38.lib.q38_moe_workspace_size(C.byref(layers[l].desc), M))
            q38.check(q38.lib.q38_moe_forward(layers[l].h, x_d.data_ptr(), M, y.data_ptr(), None, ws.data_ptr(),
                                              ws.numel(), G.stream()))
            ym = run_map(q38, maps[l], G.to_host(y, np.uint16))
            out = G.empty((M, HC * H), np.uint16)
            hc.write(G.to_dev(s), G.to_dev(ym), G.to_dev(inj), M, out, G.stream())
            s = G.to_host(out, np.uint16)
        assert np.array_equal(got, s)
        assert not np.array_equal(got, chain_hc(q38, layers, mixers, stream))  # the maps reach the stream
    finally:
        for L in layers:
            L.close()
        for h in mixers:
            h.close()


def test_bad_maps_refused(gpu, q38):
    lib = q38.lib
    y = G.empty((4, H), np.uint16)
    out = G.empty((4, H), np.uint16)
    ws = G.workspace(1 << 20)
    for m, msg in ((q38.MlpMap(H, 16, None, None, None), b"incomplete Niwaki low-rank map pair"),
                   (q38.MlpMap(H, 0, None, None, None), b"incomplete Niwaki low-rank map pair"),
                   (q38.MlpMap(H, H + 1, None, y.data_ptr(), y.data_ptr()), b"invalid Niwaki low-rank map geometry")):
        assert lib.q38_mlp_output_map(C.byref(m), y.data_ptr(), 4, out.data_ptr(), ws.data_ptr(), ws.numel(),
                                      G.stream()) == q38.Q38_EINVAL
        assert msg in lib.q38_last_error()
