"""The on-disk VQ checkpoint reader (qwen38-flash.cpp_amd/host/qwen38_checkpoint.cpp) on the
CPU through q38_checkpoint_inspect: the layer description derived from config.json's vq_modules
and the safetensors tensors, and the reference's checks with its messages —
src/model_manifest.cpp:210-230 ("unsupported vector quantization geometry for <module>") and
src/sparse_moe.cpp:618-661 ("invalid vector quantization tensors for <base>")."""
import ctypes as C
import json
import os

import numpy as np
import pytest

from checkpoint_cases import PREFIX, Checkpoint, write_safetensors


@pytest.fixture()
def q38():
    import q38 as mod
    return mod


def inspect(q38, path):
    d = q38.MoeDesc()
    rc = q38.lib.q38_checkpoint_inspect(path.encode(), PREFIX.encode(), C.byref(d))
    return rc, d, q38.lib.q38_last_error().decode()


@pytest.mark.parametrize("gu,down,gg,dg,shared", [((8, 14), (8, 14), 64, 64, True), ((2, 0), (2, 0), 64, 64, False),
                                                  ((4, 8), (8, 14), 512, 128, True), ((2, 0), (8, 14), 64, 128, True)])
def test_desc_from_checkpoint(q38, tmp_path, gu, down, gg, dg, shared):
    ck = Checkpoint(gu=gu, down=down, gu_group=gg, down_group=dg, shared=shared)
    rc, d, err = inspect(q38, ck.write(str(tmp_path)))
    assert rc == 0, err
    want = (512, 128, 64, 4, gu[0], gu[1] or 8, down[0], down[1] or 8, gg, dg, 1, int(shared), 0, 0)
    got = tuple(getattr(d, f) for f, _ in d._fields_)
    assert got == want


def test_byte_codes_are_one_per_byte(q38, tmp_path):
    """pack_bits null: U8 codes [E, out, in/dim] (not packed words)."""
    ck = Checkpoint(gu=(2, 0), down=(2, 0), shared=False)
    t = ck.tensors()
    assert t[f"{PREFIX}.switch_mlp.gate_proj.codes"].dtype == np.uint8
    assert t[f"{PREFIX}.switch_mlp.gate_proj.codes"].shape == (64, 128, 256)
    rc, _, err = inspect(q38, ck.write(str(tmp_path)))
    assert rc == 0, err


def expect_error(q38, path, needle):
    rc, _, err = inspect(q38, path)
    assert rc == q38.Q38_EINVAL and needle in err, (rc, err)


def test_geometry_errors(q38, tmp_path):
    ck = Checkpoint(shared=False)
    base = ck.config()
    mod = f"{PREFIX}.switch_mlp.gate_proj"
    cases = [("experts", 63), ("dim", 7), ("group", 100), ("k", 1), ("out", 0), ("pack_bits", 32)]
    for i, (key, val) in enumerate(cases):
        cfg = json.loads(json.dumps(base))
        cfg["vq_modules"][mod][key] = val
        expect_error(q38, ck.write(str(tmp_path / f"g{i}"), config=cfg),
                     f"unsupported vector quantization geometry for {mod}")


def test_tensor_contract_errors(q38, tmp_path):
    ck = Checkpoint(shared=False)
    base = f"{PREFIX}.switch_mlp.up_proj"
    bad = {
        "codes shape": (f"{base}.codes", lambda a: a[:, :-1]),
        "codes dtype": (f"{base}.codes", lambda a: a.astype(np.int32)),
        "scales dtype": (f"{base}.vq_scales", lambda a: a.astype(np.float32)),
        "codebook shape": (f"{base}.codebook", lambda a: a[:-1]),
        "codebook dtype": (f"{base}.codebook", lambda a: a.astype(np.float32)),
        "scales shape": (f"{base}.vq_scales", lambda a: a[:, :, :-1]),
    }
    for i, (name, (key, f)) in enumerate(bad.items()):
        t = ck.tensors()
        t[key] = np.ascontiguousarray(f(t[key]))
        expect_error(q38, ck.write(str(tmp_path / f"t{i}"), tensors=t), f"invalid vector quantization tensors for {base}")


def test_layer_level_errors(q38, tmp_path):
    ck = Checkpoint(shared=False)
    t = ck.tensors()
    del t[f"{PREFIX}.gate.weight"]
    expect_error(q38, ck.write(str(tmp_path / "a"), tensors=t), f"missing tensor {PREFIX}.gate.weight")
    t = ck.tensors()
    t[f"{PREFIX}.shared_expert_gate.weight"] = np.zeros((1, 512), np.uint16)
    expect_error(q38, ck.write(str(tmp_path / "b"), tensors=t),
                 f"missing tensor {PREFIX}.shared_expert.gate_proj.weight")
    cfg = ck.config()
    del cfg["vq_modules"][f"{PREFIX}.switch_mlp.down_proj"]
    expect_error(q38, ck.write(str(tmp_path / "c"), config=cfg), "no vq_modules entry")


def test_affine_shared_expert_checks(q38, tmp_path):
    """The affine shared expert's checks: the reference's messages for a missing quantization
    section, bits that disagree with it, non-integral bits and bad tensors
    (src/sparse_moe.cpp:662-700, src/quantization_geometry.cpp:9-35, src/model_manifest.cpp:188-192);
    a VQ module for a shared expert is refused (experts must be num_experts), and one covering
    all experts is not a shared expert the reference can apply."""
    ck = Checkpoint(shared=True, sa_bits=4, sa_group=64)
    base = f"{PREFIX}.shared_expert.up_proj"
    cfg = ck.config()
    del cfg["quantization"]
    expect_error(q38, ck.write(str(tmp_path / "q0"), config=cfg), "model is missing quantization metadata")
    cfg = ck.config()
    cfg["quantization"]["bits"] = 8
    expect_error(q38, ck.write(str(tmp_path / "q1"), config=cfg),
                 f"MoE tensor disagrees with quantization metadata for {PREFIX}.shared_expert.gate_proj")
    cfg = ck.config()
    cfg["quantization"][base] = {"bits": 4, "group_size": 48}
    expect_error(q38, ck.write(str(tmp_path / "q2"), config=cfg), "non-integral MoE quantization bits")
    cfg = ck.config()
    cfg["quantization"][base] = {"bits": 9, "group_size": 64}
    expect_error(q38, ck.write(str(tmp_path / "q3"), config=cfg), f"invalid quantization override for {base}")
    for i, (key, f) in enumerate([(f"{base}.scales", lambda a: a.astype(np.float32)),
                                  (f"{base}.biases", lambda a: a[:, :-1]),
                                  (f"{base}.weight", lambda a: a.astype(np.int32))]):
        t = ck.tensors()
        t[key] = np.ascontiguousarray(f(t[key]))
        rc, _, err = inspect(q38, ck.write(str(tmp_path / f"t{i}"), tensors=t))
        assert rc == q38.Q38_EINVAL and ("invalid affine quantization tensors" in err or "quantization" in err), err
    # a per-module override of the quantization is honoured (here: the same values)
    cfg = ck.config()
    cfg["quantization"][f"language_model.{base}"] = {"bits": 4, "group_size": 64}
    rc, _, err = inspect(q38, ck.write(str(tmp_path / "ov"), config=cfg))
    assert rc == 0, err
    cfg = ck.config()
    cfg["text_config"]["shared_expert_intermediate_size"] = 256
    expect_error(q38, ck.write(str(tmp_path / "si"), config=cfg), "disagrees with shared_expert_intermediate_size")
    # VQ shared modules: experts 1 (the old exemption) and experts E
    cfg = ck.config()
    cfg["vq_modules"][f"{PREFIX}.shared_expert.gate_proj"] = dict(cfg["vq_modules"][f"{PREFIX}.switch_mlp.gate_proj"],
                                                                   experts=1)
    expect_error(q38, ck.write(str(tmp_path / "v1"), config=cfg),
                 f"unsupported vector quantization geometry for {PREFIX}.shared_expert.gate_proj")
    cfg["vq_modules"][f"{PREFIX}.shared_expert.gate_proj"]["experts"] = ck.E
    expect_error(q38, ck.write(str(tmp_path / "v2"), config=cfg), "shared experts load in affine form")


@pytest.mark.parametrize("shared_inter,sa_bits,sa_group,sa_fmt", [(128, 4, 64, 0), (256, 8, 32, 1), (64, 2, 64, 0)])
def test_affine_shared_geometry(q38, tmp_path, shared_inter, sa_bits, sa_group, sa_fmt):
    ck = Checkpoint(shared=True, shared_inter=shared_inter, sa_bits=sa_bits, sa_group=sa_group, sa_fmt=sa_fmt)
    rc, d, err = inspect(q38, ck.write(str(tmp_path)))
    assert rc == 0 and d.has_shared == 1, err


def test_flat_names_resolve_under_the_wrapper(q38, tmp_path):
    """Tensors and modules stored without "language_model." resolve when the layer is named
    with it (ModelManifest::resolve_tensor_name / vector_quantization_for /
    quantization_for, src/model_manifest.cpp:470-500)."""
    ck = Checkpoint(shared=True, flat=True)
    path = ck.write(str(tmp_path))
    d = q38.MoeDesc()
    rc = q38.lib.q38_checkpoint_inspect(path.encode(), ck.prefix.encode(), C.byref(d))
    assert rc == 0, q38.lib.q38_last_error()
    rc2, d2, err = inspect(q38, path)
    assert rc2 == 0, err
    assert bytes(d) == bytes(d2)
    rc = q38.lib.q38_checkpoint_inspect(path.encode(), b"other_model." + PREFIX.encode(), C.byref(d))
    assert rc == q38.Q38_EINVAL


def test_safetensors_header_checks(q38, tmp_path):
    ck = Checkpoint(shared=False)
    d = ck.write(str(tmp_path / "ok"))
    st = os.path.join(d, "model.safetensors")
    raw = open(st, "rb").read()
    n = int.from_bytes(raw[:8], "little")
    # header length past the file
    d1 = ck.write(str(tmp_path / "h1"))
    with open(os.path.join(d1, "model.safetensors"), "wb") as f:
        f.write((len(raw) + 10).to_bytes(8, "little") + raw[8:])
    expect_error(q38, d1, "header exceeds the file")
    # a tensor's data offsets past the data
    header = json.loads(raw[8:8 + n])
    key = f"{PREFIX}.switch_mlp.gate_proj.vq_scales"
    b, e = header[key]["data_offsets"]
    header[key]["data_offsets"] = [b, e + 10 ** 9]
    hb = json.dumps(header, separators=(",", ":")).encode()
    d2 = str(tmp_path / "h2")
    ck.write(d2)
    with open(os.path.join(d2, "model.safetensors"), "wb") as f:
        f.write(len(hb).to_bytes(8, "little") + hb + raw[8 + n:])
    expect_error(q38, d2, "outside the file")
    # malformed JSON
    d3 = str(tmp_path / "h3")
    ck.write(d3)
    with open(os.path.join(d3, "config.json"), "w") as f:
        f.write('{"text_config": {"num_experts": 64,')
    expect_error(q38, d3, "invalid JSON")


def test_index_weight_map(q38, tmp_path):
    """Sharded checkpoints: model.safetensors.index.json names the files; a path outside the
    directory is refused."""
    ck = Checkpoint(shared=False)
    d = str(tmp_path / "s")
    ck.write(d)
    t = ck.tensors()
    names = sorted(t)
    os.remove(os.path.join(d, "model.safetensors"))
    half = len(names) // 2
    wm = {}
    for i, part in enumerate((names[:half], names[half:])):
        fn = f"model-{i + 1:05d}-of-00002.safetensors"
        write_safetensors(os.path.join(d, fn), {k: t[k] for k in part})
        wm.update({k: fn for k in part})
    with open(os.path.join(d, "model.safetensors.index.json"), "w") as f:
        json.dump({"weight_map": wm}, f)
    rc, _, err = inspect(q38, d)
    assert rc == 0, err
    wm[names[0]] = "../evil.safetensors"
    with open(os.path.join(d, "model.safetensors.index.json"), "w") as f:
        json.dump({"weight_map": wm}, f)
    expect_error(q38, d, "outside the checkpoint")


def test_writer_matches_safetensors_library(tmp_path):
    """The fixtures' safetensors writer against the safetensors package's own reader (U8, U32,
    F16 tensors read back identically; BF16 entries carry the dtype name the reference uses)."""
    from safetensors import safe_open
    ck = Checkpoint(gu=(2, 0), down=(8, 14), shared=True)
    d = ck.write(str(tmp_path))
    t = ck.tensors()
    with safe_open(f"{d}/model.safetensors", framework="np") as f:
        for k, v in t.items():
            if v.dtype == np.uint16:
                continue  # BF16: numpy has no bfloat16 type to read into
            assert np.array_equal(f.get_tensor(k), v), k
    raw = open(f"{d}/model.safetensors", "rb").read()
    n = int.from_bytes(raw[:8], "little")
    header = json.loads(raw[8:8 + n])
    assert header[f"{PREFIX}.gate.weight"]["dtype"] == "BF16"
