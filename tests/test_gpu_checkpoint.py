"""MoE layers read from on-disk VQ checkpoints (q38_moe_layer_load) on the GPU: the loaded
layer equals a layer created directly from the same arrays (q38_moe_layer_create) bit for bit,
routing equals the oracle's bit for bit and outputs are within tolerance of it, for the
reference family's geometries: d8/14-bit packed codes with 64-input scale groups, d2/K256 byte
codes (pack_bits null, the first layers of the reference checkpoint, docs/vq-backend-bringup.md:7-9),
d4/8-bit with per-row scales, and a layer mixing byte-coded gate/up with a packed down; the
shared expert in the reference's MLX affine form (4- and 8-bit, 32- and 64-input groups, BF16
and F16 scales, an intermediate size of its own), and a store with flat names loaded under the
"language_model." wrapper."""
import ctypes as C

import numpy as np
import pytest

import gpu_util as G
import oracle_lib
from checkpoint_cases import PREFIX, Checkpoint
from moe_cases import run_forward, tol_check

pytestmark = pytest.mark.gpu

CASES = {
    "d8_g64_shared": dict(gu=(8, 14), down=(8, 14), gu_group=64, down_group=64, shared=True),
    "d2_bytes_g64": dict(gu=(2, 0), down=(2, 0), gu_group=64, down_group=64, shared=False),
    "d4_rows_shared8": dict(gu=(4, 8), down=(4, 8), gu_group=512, down_group=128, shared=True, sa_bits=8,
                            sa_group=32, sa_fmt=1, shared_inter=256),
    "d2_gu_d8_down": dict(gu=(2, 0), down=(8, 14), gu_group=64, down_group=128, shared=True),
    "d8_g64_flat": dict(gu=(8, 14), down=(8, 14), gu_group=64, down_group=64, shared=True, flat=True),
}


class Handle:
    def __init__(self, h, q38):
        self.h, self.q38 = h, q38

    def close(self):
        self.q38.lib.q38_moe_layer_destroy(self.h)


def direct_layer(q38, gpu, ck, desc):
    keep = [G.to_dev(ck.router), G.to_dev(ck.wsg.reshape(-1))]
    w = q38.MoeWeights()
    w.router, w.shared_gate = keep[0].data_ptr(), keep[1].data_ptr()
    for p in range(3):
        c, s, b = G.to_dev(ck.words(p).reshape(-1)), G.to_dev(ck.scales[p].view(np.uint16).reshape(-1)), None
        dim, bits = ck.kernel_geometry(p)
        book = np.zeros(((1 << bits), dim), np.float16)
        book[:ck.books[p].shape[0]] = ck.books[p]
        b = G.to_dev(book.view(np.uint16).reshape(-1))
        keep += [c, s, b]
        w.codes[p], w.scales[p], w.books[p] = c.data_ptr(), s.data_ptr(), b.data_ptr()
    if not ck.shared:
        return q38.MoeLayer(gpu, desc, weights=w), keep
    a = q38.AffineShared()
    for p in range(3):
        t = [G.to_dev(ck.sa["w"][p]), G.to_dev(ck.sa["s"][p]), G.to_dev(ck.sa["b"][p])]
        keep += t
        a.weight[p], a.scales[p], a.biases[p] = t[0].data_ptr(), t[1].data_ptr(), t[2].data_ptr()
    a.bits, a.group, a.inter, a.scale_dtype = ck.sa["bits"], ck.sa["group"], ck.sa["inter"], ck.sa["fmt"]
    h = C.c_void_p()
    q38.check(q38.lib.q38_moe_layer_create_affine_shared(gpu.h, C.byref(desc), C.byref(w), C.byref(a), C.byref(h)))
    return Handle(h, q38), keep


@pytest.mark.parametrize("case", list(CASES))
def test_loaded_layer(gpu, q38, orc, tmp_path, case):
    ck = Checkpoint(seed=3, **CASES[case])
    path = ck.write(str(tmp_path / case))
    desc = q38.MoeDesc()
    q38.check(q38.lib.q38_checkpoint_inspect(path.encode(), ck.prefix.encode(), C.byref(desc)))
    h = C.c_void_p()
    q38.check(q38.lib.q38_moe_layer_load(gpu.h, path.encode(), ck.prefix.encode(), 0, C.byref(h)))

    class Loaded:
        pass

    loaded = Loaded()
    loaded.h = h
    direct, keep = direct_layer(q38, gpu, ck, desc)
    try:
        od = oracle_lib.make_desc(hidden=ck.H, inter=ck.I, experts=ck.E, top_k=ck.k, gu=ck.kernel_geometry(0),
                                  down=ck.kernel_geometry(2), gu_group=ck.groups[0], down_group=ck.groups[2],
                                  shared=int(ck.shared))
        books = []
        for p in range(3):
            dim, bits = ck.kernel_geometry(p)
            b = np.zeros(((1 << bits), dim), np.float16)
            b[:ck.books[p].shape[0]] = ck.books[p]
            books.append(b.view(np.uint16).reshape(-1))
        rng = np.random.default_rng(11)
        for M in (1, 4, 16):
            x = orc.bf16(rng.normal(0, 1, (M, ck.H)))
            y1, ex1, wt1, _, _ = run_forward(q38, loaded, desc, x)
            y2, ex2, wt2, _, _ = run_forward(q38, direct, desc, x)
            assert np.array_equal(y1, y2) and np.array_equal(ex1, ex2) and np.array_equal(wt1, wt2), (case, M)
            codes = [ck.words(p).reshape(-1) for p in range(3)]
            scales = [ck.scales[p].view(np.uint16).reshape(-1) for p in range(3)]
            if ck.shared:
                yo, exo, wto, _ = orc.moe_layer_dense_affine_shared(od, ck.router, ck.wsg.reshape(-1), codes, scales,
                                                                    books, ck.sa, x)
            else:
                yo, exo, wto, _ = orc.moe_layer_dense(od, ck.router, ck.wsg.reshape(-1), codes, scales, books, x)
            assert np.array_equal(ex1, exo), (case, M)
            assert np.array_equal(wt1, wto), (case, M)
            tol_check(orc, y1, yo)
    finally:
        q38.lib.q38_moe_layer_destroy(h)
        direct.close()


def test_unsupported_affine_bits_refused(gpu, q38, tmp_path):
    """A 3-bit affine shared expert is a valid reference checkpoint (Q3), but the device kernels
    take 2-, 4- and 8-bit values (whole in a word): loading reports it."""
    ck = Checkpoint(shared=True)
    t = ck.tensors()
    cfg = ck.config()
    cfg["quantization"]["bits"] = 3
    for p, name in enumerate(("gate_proj", "up_proj", "down_proj")):
        w = t[f"{PREFIX}.shared_expert.{name}.weight"]
        t[f"{PREFIX}.shared_expert.{name}.weight"] = np.zeros((w.shape[0], w.shape[1] * 3 // 4), np.uint32)
    path = ck.write(str(tmp_path / "q3"), tensors=t, config=cfg)
    h = C.c_void_p()
    assert q38.lib.q38_moe_layer_load(gpu.h, path.encode(), PREFIX.encode(), 0, C.byref(h)) == q38.Q38_EINVAL
    assert b"bits must be 2, 4 or 8" in q38.lib.q38_last_error()
