"""q38_verify_chain_profiled: every phase kernel is timed (start at the phase's first kernel,
stop at its last), on uniform (one fused gate/up + down + combine kernel at up to 4 rows, as
for the scale-group stacks),
mixed (two bank kernels per phase) and per-64-input scale group stacks; the profiled pass
computes the same values as the plain one."""
import ctypes as C

import numpy as np
import pytest

import gpu_util as G
from moe_cases import SEED

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kind,M", [("uniform", 4), ("uniform", 1), ("mixed", 16), ("group64", 4), ("group64", 8)])
def test_profiled_chain(gpu, q38, orc, kind, M):
    import torch
    d = {"uniform": q38.desc(), "mixed": q38.desc(mixed=1), "group64": q38.desc(gu_group=64, down_group=64)}[kind]
    layers = [q38.MoeLayer(gpu, d, seed=SEED, layer=l) for l in range(3)]
    try:
        arr = (C.c_void_p * 3)(*[L.h.value for L in layers])
        ws = G.workspace(q38.lib.q38_moe_workspace_size(C.byref(d), M))
        h0 = orc.embed(SEED, list(range(40, 40 + M)), 2048)
        h = G.to_dev(h0)
        q38.check(q38.lib.q38_verify_chain(arr, 3, h.data_ptr(), M, C.c_float(1e-6), None, ws.data_ptr(), ws.numel(),
                                           G.stream()))
        plain = G.to_host(h, np.uint16)
        hp = G.to_dev(h0)
        tm = q38.MoeTimings()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        rc = q38.lib.q38_verify_chain_profiled(arr, 3, hp.data_ptr(), M, C.c_float(1e-6), None, ws.data_ptr(),
                                               ws.numel(), C.byref(tm), G.stream())
        e1.record()
        torch.cuda.synchronize()
        assert rc == q38.Q38_OK, q38.last_error()
        assert np.array_equal(G.to_host(hp, np.uint16), plain)
        phases = [tm.routing_ms, tm.gate_up_ms, tm.down_ms, tm.merge_ms]
        # config-1 layers (per-row or 64-input scales) at up to 4 rows run gate/up, down and
        # the combine in one kernel: its time is gate_up_ms, and the down and merge phases are 0
        fused = kind in ("uniform", "group64") and M <= 4
        timed = phases[:2] if fused else phases
        assert tm.layers == 3 and all(np.isfinite(p) and p > 0 for p in timed), phases
        if fused:
            assert tm.down_ms == 0.0 and tm.merge_ms == 0.0, phases
        assert sum(phases) <= 1.05 * e0.elapsed_time(e1) + 0.01, (phases, e0.elapsed_time(e1))
    finally:
        for L in layers:
            L.close()
