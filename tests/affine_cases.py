"""Builders for the affine (MLX quantized) shared expert: packing, random tensors, and an
independent float64 numpy restatement of SparseMoe::forward_shared over dequantized weights."""
from __future__ import annotations

import numpy as np


def pack_affine(q, bits):
    """[O, IN] values in [0, 2^bits) -> [O, IN * bits / 32] uint32, value j of a word at bits
    j * bits (LSB first): MLX's packing for 2-, 4- and 8-bit affine weights."""
    q = np.asarray(q, np.uint64)
    O, IN = q.shape
    vpw = 32 // bits
    shifts = np.arange(vpw, dtype=np.uint64) * np.uint64(bits)
    return (q.reshape(O, IN // vpw, vpw) << shifts).sum(-1).astype(np.uint32)


def to16(v, fmt):
    """float -> bf16 (fmt 0, round to nearest even) or fp16 (fmt 1) bits."""
    f = np.asarray(v, np.float32)
    if fmt == 1:
        return f.astype(np.float16).view(np.uint16)
    u = f.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def from16(u, fmt):
    u = np.asarray(u, np.uint16)
    return u.view(np.float16).astype(np.float64) if fmt == 1 else (u.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def random_affine(rng, H, Is, bits, group, fmt, scale=0.02):
    """Random affine gate / up [Is, H] and down [H, Is] with MLX-like scales and biases
    (weights of spread ~scale, centred)."""
    out = {"w": [], "s": [], "b": [], "q": [], "bits": bits, "group": group, "inter": Is, "fmt": fmt}
    for O, IN in ((Is, H), (Is, H), (H, Is)):
        q = rng.integers(0, 1 << bits, (O, IN))
        s = rng.uniform(0.5, 1.5, (O, IN // group)) * scale * 4 / (1 << bits)
        b = -s * ((1 << bits) - 1) / 2 + rng.normal(0, scale * 0.05, (O, IN // group))
        out["q"].append(q)
        out["w"].append(pack_affine(q, bits))
        out["s"].append(to16(s, fmt))
        out["b"].append(to16(b, fmt))
    return out


def dequant(sa, p):
    q = sa["q"][p].astype(np.float64)
    g = sa["group"]
    s = np.repeat(from16(sa["s"][p], sa["fmt"]), g, axis=1)
    b = np.repeat(from16(sa["b"][p], sa["fmt"]), g, axis=1)
    return s * q + b


def np_affine_expert(orc, sa, x):
    """forward_shared without the gate: T(down(T(T(silu(T(g))) * T(u)))) per row, float64 dots
    over the dequantized weights (src/sparse_moe.cpp:1306-1313)."""
    xf = orc.bf16_to_f32(np.asarray(x, np.uint16)).astype(np.float64)
    T = lambda v: orc.bf16_to_f32(orc.bf16(np.asarray(v, np.float64).astype(np.float32))).astype(np.float64)
    g = T(xf @ dequant(sa, 0).T)
    u = T(xf @ dequant(sa, 1).T)
    s = T(g / (1.0 + np.exp(-g)))
    h = T(s * u)
    return T(h @ dequant(sa, 2).T).astype(np.float32)
