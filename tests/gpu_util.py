"""Device-buffer plumbing for the GPU tests: torch allocates, libamdhip64 copies."""
from __future__ import annotations

import ctypes as C

import numpy as np

_hip = None


def hip():
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        _hip.hipMemcpy.restype = C.c_int
        _hip.hipDeviceSynchronize.restype = C.c_int
    return _hip


def d2h(ptr: int, shape, dtype) -> np.ndarray:
    out = np.empty(shape, dtype)
    hip().hipDeviceSynchronize()
    rc = hip().hipMemcpy(out.ctypes.data, ptr, out.nbytes, 2)
    assert rc == 0, rc
    return out


def to_dev(arr: np.ndarray):
    import torch
    a = np.ascontiguousarray(arr)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    elif a.dtype == np.uint32:
        a = a.view(np.int32)
    elif a.dtype == np.uint64:
        a = a.view(np.int64)
    return torch.from_numpy(a.copy()).cuda()


def empty(shape, dtype):
    import torch
    m = {np.uint16: torch.int16, np.int32: torch.int32, np.uint32: torch.int32, np.float32: torch.float32,
         np.int64: torch.int64, np.int8: torch.int8, np.uint8: torch.uint8}
    return torch.zeros(shape, dtype=m[dtype], device="cuda")


def to_host(t, dtype=None) -> np.ndarray:
    import torch
    torch.cuda.synchronize()
    a = t.cpu().numpy()
    return a.view(dtype) if dtype is not None else a


def stream() -> int:
    import torch
    return torch.cuda.current_stream().cuda_stream


def workspace(nbytes: int):
    import torch
    return torch.empty(int(nbytes), dtype=torch.uint8, device="cuda")
