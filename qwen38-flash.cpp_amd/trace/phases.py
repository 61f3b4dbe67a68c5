"""Phase stamps of the verify layer's two kernels (k_route_norm, k_gd4) from the inside.

Build the stamped library first (make -C qwen38-flash.cpp_amd trace), then run on a GPU:

    python3 qwen38-flash.cpp_amd/trace/phases.py M

It runs a chain of 8 synthetic config-1 layers at M rows (1..4) five times and prints, for
the last layer of the last pass, the min / median / max over workgroups of each stamp,
in microseconds from the first workgroup's start (the 100 MHz real-time counter, 10 ns
steps). Stamp numbers (Q38_STAMP in the kernels):
  k_gd4 gate/up half (gu):  0 start, 1-2 logits requested, 11 softmax keys, 12 threshold,
    13 candidates ranked, 3 routing done, 15 codebook chunk in LDS (wave M), 14 plan built,
    4 plan published, 5 first items' loads issued, 6 item 0's MFMA sums, 7 its cross-wave
    sums, 8 item 0 done, 9 all gate/up items done (their values stored);
  k_gd4 down half (dn):  0 start, 1 plan read, 6-8 loads of items 0-2 issued, 2 codebook
    chunk stored to LDS, 5 item 0's gate/up values present, 12 its SwiGLU rows in LDS,
    13 its MFMA sums, 14 its cross-wave sums, 3 item 0 done, 4 all down items done;
  k_gd4 combine tail (last 32 workgroups): 0 start, 1 first read of the down sums,
    2 all present, 3 output stored;
  k_route_norm (route):  0 start, 1 layer input loaded, 6 norm partial sums, 7 normalised
    input stored, 2 staged in LDS, 4 partial-sum planes reset, 5 router dot products,
    3 logits stored.
"""
import ctypes as C
import os
import sys

_HERE = os.path.dirname(os.path.abspath(__file__))
os.environ.setdefault("Q38_LIB", os.path.join(_HERE, "libq38.so"))
sys.path.insert(0, os.path.dirname(_HERE))

import numpy as np  # noqa: E402
import torch  # noqa: E402  (before q38: the HIP runtime of the torch build)
import q38  # noqa: E402

NL, G, NR = 8, 256, 65  # layers, k_gd4 workgroups, k_route_norm workgroups (H = 2048)


def main():
    M = int(sys.argv[1]) if len(sys.argv) > 1 else 4
    assert 1 <= M <= 4
    dev = torch.device("cuda:0")
    sp = torch.cuda.current_stream().cuda_stream
    ctx = q38.Ctx(0)
    d = q38.desc()
    layers = [q38.MoeLayer(ctx, d, seed=0x51A5EED, layer=i) for i in range(NL)]
    larr = (C.c_void_p * NL)(*[L.h.value for L in layers])
    ws = torch.empty(q38.lib.q38_moe_workspace_size(C.byref(d), 4), dtype=torch.uint8, device=dev)
    h = torch.empty((M, 2048), dtype=torch.int16, device=dev)
    toks = (C.c_uint32 * M)(*[11 + 7 * r for r in range(M)])
    for _ in range(5):
        q38.check(q38.lib.q38_embed_synthetic(0x51A5EED, toks, M, 2048, h.data_ptr(), sp))
        q38.check(q38.lib.q38_verify_chain(larr, NL, h.data_ptr(), M, 1e-6, None, ws.data_ptr(), ws.numel(), sp))
        torch.cuda.synchronize()
    q38.check(q38.lib.q38_ctx_synchronize(ctx.h, sp))
    for fn in ("q38_trace_read", "q38_trace_read_route"):
        getattr(q38.lib, fn).argtypes = [C.c_void_p]
    buf = np.zeros(32768, np.uint64)
    rbuf = np.zeros(32768, np.uint64)
    assert q38.lib.q38_trace_read(buf.ctypes.data) == 0, "not the stamped build (make trace)"
    assert q38.lib.q38_trace_read_route(rbuf.ctypes.data) == 0
    gu = buf[8192:8192 + 16 * G].reshape(G, 16).astype(np.int64)
    dn = buf[16384:16384 + 16 * G].reshape(G, 16).astype(np.int64)
    cb = buf[24576:24576 + 16 * G].reshape(G, 16).astype(np.int64)
    rt = rbuf[:16 * NR].reshape(NR, 16).astype(np.int64)
    t0, r0 = gu[:, 0].min(), rt[:, 0].min()

    def show(name, a, idx, ref, rows=None):
        a = a if rows is None else a[rows]
        for i in idx:
            v = (a[:, i] - ref) * 10 / 1000.0
            print(f"{name}[{i:2d}]  min {v.min():6.2f}  p50 {np.median(v):6.2f}  max {v.max():6.2f} us")

    print(f"M = {M}: k_route_norm (from its first workgroup's start)")
    show("route", rt, [0, 1, 6, 7, 2, 4, 5, 3], r0)
    print(f"k_route_norm start -> k_gd4 start: {(t0 - r0) / 100:.2f} us")
    print("k_gd4 (from its first workgroup's start)")
    show("gu", gu, [0, 1, 11, 12, 13, 3, 15, 14, 4, 5, 6, 7, 8, 9], t0)
    n_items = dn[:, 10].astype(int)
    show("dn", dn, [0, 1, 6, 2, 5, 12, 13, 14, 3], t0, n_items > 0)
    show("dn", dn, [4], t0)
    print("down items per workgroup:", dict(enumerate(np.bincount(n_items).tolist())))
    show("combine", cb, [0, 1, 2, 3], t0, np.arange(G) >= G - 32)
    v = (cb[:, 4] - t0) / 100
    print(f"workgroup end  min {v.min():6.2f}  p50 {np.median(v):6.2f}  max {v.max():6.2f} us")
    for L in layers:
        L.close()
    ctx.close()


if __name__ == "__main__":
    main()
