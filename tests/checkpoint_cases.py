"""Synthetic on-disk VQ checkpoints in the reference's format (config.json vq_modules +
safetensors, src/model_manifest.cpp:210-230, src/sparse_moe.cpp:618-661) for the loader tests."""
from __future__ import annotations

import json
import os

import numpy as np

PREFIX = "model.layers.0.mlp"
PREFIX_WRAPPED = "language_model." + PREFIX  # (the reference's name; a flat store drops the wrapper)


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16)


def bf16_bits(a):
    u = np.asarray(a, np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def packed(codes, bits):
    """Codes [rows, n] -> packed u32 words [rows, ceil(n/32)*bits] (32-code blocks, LSB first)."""
    rows, n = codes.shape
    nw = (n + 31) // 32 * bits
    out = np.zeros((rows, nw), np.uint64)
    for i in range(n):
        bit = (i % 32) * bits
        w = (i // 32) * bits + bit // 32
        sh = bit % 32
        v = codes[:, i].astype(np.uint64) << np.uint64(sh)
        out[:, w] |= v & np.uint64(0xFFFFFFFF)
        if sh + bits > 32:
            out[:, w + 1] |= v >> np.uint64(32)
    return out.astype(np.uint32)


class Checkpoint:
    """One MoE layer in the reference's on-disk layout: E routed VQ experts (gate/up (dim, bits)
    and down (dim, bits) geometry, scale groups gu_group / down_group; bits 0 = byte codes,
    pack_bits null in the manifest) and, with shared, an MLX affine shared expert
    (shared_expert.{gate,up,down}_proj .weight / .scales / .biases, sa_bits values, sa_group
    inputs per scale, sa_fmt 0 BF16 or 1 F16 scales, intermediate size shared_inter) with the
    model-wide "quantization" metadata. flat: tensors and modules stored without the
    "language_model." wrapper that the layer prefix PREFIX_WRAPPED carries."""

    def __init__(self, H=512, I=128, E=64, k=4, gu=(8, 14), down=(8, 14), gu_group=64, down_group=64,
                 shared=True, seed=0, normalize=True, sa_bits=4, sa_group=64, sa_fmt=0, shared_inter=None,
                 flat=False):
        from affine_cases import random_affine
        rng = np.random.default_rng(seed)
        self.H, self.I, self.E, self.k, self.gu, self.down = H, I, E, k, gu, down
        self.groups = (gu_group, gu_group, down_group)
        self.shared, self.normalize, self.flat = shared, normalize, flat
        geo = (gu, gu, down)
        ins, outs = (H, H, I), (I, I, H)
        self.router = bf16_bits(rng.normal(0, 0.02, (E, H)))
        self.wsg = bf16_bits(rng.normal(0, 0.02, (1, H)))
        self.books, self.codes, self.scales = [], [], []
        for p in range(3):
            dim, bits = geo[p]
            K = 256 if bits == 0 else 1 << bits
            self.books.append(f16(rng.normal(0, 1, (K, dim))))
            n = ins[p] // dim
            rows = E * outs[p]
            self.codes.append(rng.integers(0, K, (rows, n)).astype(np.uint32))
            self.scales.append(f16(rng.uniform(0.005, 0.02, (rows, ins[p] // self.groups[p]))))
        self.sa = random_affine(rng, H, shared_inter or I, sa_bits, sa_group, sa_fmt) if shared else None

    def kernel_geometry(self, p):
        dim, bits = (self.gu, self.gu, self.down)[p]
        return dim, (8 if bits == 0 else bits)

    def words(self, p):
        """Codes in the q38 packed layout [E*OUT, words] (byte codes = 8-bit words)."""
        dim, bits = self.kernel_geometry(p)
        return packed(self.codes[p], bits)

    @property
    def prefix(self):
        """The layer prefix a caller passes (the wrapped name when the store is flat)."""
        return PREFIX_WRAPPED if self.flat else PREFIX

    def config(self, experts_field=None):
        mods = {}
        names = ("gate_proj", "up_proj", "down_proj")
        geo = (self.gu, self.gu, self.down)
        ins, outs = (self.H, self.H, self.I), (self.I, self.I, self.H)
        for p in range(3):
            dim, bits = geo[p]
            spec = {"experts": experts_field or self.E, "out": outs[p], "in": ins[p],
                    "k": int(self.books[p].shape[0]), "dim": dim, "group": self.groups[p],
                    "pack_bits": None if bits == 0 else bits}
            mods[f"{PREFIX}.switch_mlp.{names[p]}"] = spec
        text = {"num_experts": self.E, "num_experts_per_tok": self.k, "norm_topk_prob": self.normalize,
                "hidden_size": self.H}
        cfg = {"text_config": text, "vq_modules": mods}
        if self.shared:
            text["shared_expert_intermediate_size"] = self.sa["inter"]
            cfg["quantization"] = {"group_size": self.sa["group"], "bits": self.sa["bits"]}
        return cfg

    def tensors(self):
        t = {f"{PREFIX}.gate.weight": self.router}  # uint16 = BF16 bits
        names = ("gate_proj", "up_proj", "down_proj")
        outs = (self.I, self.I, self.H)
        for p in range(3):
            dim, bits = (self.gu, self.gu, self.down)[p]
            E, O = self.E, outs[p]
            c = self.codes[p].reshape(E, O, -1)
            enc = (lambda a: a.astype(np.uint8)) if bits == 0 else (lambda a: packed(a.reshape(-1, a.shape[-1]), bits)
                                                                      .reshape(a.shape[0], a.shape[1], -1))
            t[f"{PREFIX}.switch_mlp.{names[p]}.codes"] = enc(c)
            t[f"{PREFIX}.switch_mlp.{names[p]}.codebook"] = self.books[p]
            t[f"{PREFIX}.switch_mlp.{names[p]}.vq_scales"] = self.scales[p].reshape(E, O, -1)
            if self.shared:
                sdt = np.float16 if self.sa["fmt"] == 1 else np.uint16  # (uint16 = BF16 bits)
                t[f"{PREFIX}.shared_expert.{names[p]}.weight"] = self.sa["w"][p]
                t[f"{PREFIX}.shared_expert.{names[p]}.scales"] = self.sa["s"][p].view(sdt)
                t[f"{PREFIX}.shared_expert.{names[p]}.biases"] = self.sa["b"][p].view(sdt)
        if self.shared:
            t[f"{PREFIX}.shared_expert_gate.weight"] = self.wsg
        return t

    def write(self, directory, tensors=None, config=None):
        os.makedirs(directory, exist_ok=True)
        with open(os.path.join(directory, "config.json"), "w") as f:
            json.dump(config or self.config(), f)
        write_safetensors(os.path.join(directory, "model.safetensors"), tensors or self.tensors())
        return directory


_DTYPES = {np.dtype(np.uint8): "U8", np.dtype(np.uint32): "U32", np.dtype(np.int32): "I32",
           np.dtype(np.float16): "F16", np.dtype(np.float32): "F32", np.dtype(np.uint16): "BF16"}


def write_safetensors(path, tensors):
    """safetensors file: 8-byte header length, JSON header (name -> dtype, shape, data_offsets),
    then the data. uint16 arrays are written as BF16 (bf16 bit patterns)."""
    header, blobs, off = {}, [], 0
    for name in sorted(tensors):
        a = np.ascontiguousarray(tensors[name])
        b = a.tobytes()
        header[name] = {"dtype": _DTYPES[a.dtype], "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    header["__metadata__"] = {"format": "np"}
    raw = json.dumps(header, separators=(",", ":")).encode()
    raw += b" " * (-len(raw) % 8)
    with open(path, "wb") as f:
        f.write(len(raw).to_bytes(8, "little") + raw + b"".join(blobs))
