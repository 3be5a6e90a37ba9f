"""Checkpoint ingest on the host (no GPU): the safetensors container
(safetensors.zig:126-237 semantics), the reference's suffix lookup
(weights.zig:204-207) and the block-FP8 tensor checks of loadExpert
(moe.zig:251-292)."""
from __future__ import annotations

import os

import numpy as np
import pytest

from colizig_amd import ingest, moe, synth


def _tiny(tmp_path, prefix="model", router_dt="BF16", split=False):
    host = synth.make_layer(256, 4, 2, 128, 0, True, seed=3)
    rng = np.random.default_rng(3)
    r_bits = rng.integers(0, 1 << 16, size=(4, 256), dtype=np.uint16)
    r_bits[(r_bits & 0x7F80) == 0x7F80] = 0  # no inf/NaN
    t = {}
    pre = f"{prefix}." if prefix else ""
    t[f"{pre}layers.0.mlp.gate.weight"] = ("BF16", r_bits) if router_dt == "BF16" else ("F32", host["router"])
    for e, ex in enumerate(host["experts"]):
        for proj, key in (("gate_proj", "gate"), ("up_proj", "up"), ("down_proj", "down")):
            t[f"{pre}layers.0.mlp.experts.{e}.{proj}.weight"] = ("F8_E4M3", ex[f"{key}_w"])
            t[f"{pre}layers.0.mlp.experts.{e}.{proj}.weight_scale_inv"] = ("F32", ex[f"{key}_s"])
    if split:
        names = sorted(t)
        ingest.write_safetensors(str(tmp_path / "a.safetensors"), {n: t[n] for n in names[::2]})
        ingest.write_safetensors(str(tmp_path / "b.safetensors"), {n: t[n] for n in names[1::2]})
        path = str(tmp_path)
    else:
        path = str(tmp_path / "m.safetensors")
        ingest.write_safetensors(path, t)
    return host, r_bits, path


def test_views_are_the_stored_bytes(tmp_path):
    host, r_bits, path = _tiny(tmp_path)
    ck = ingest.Checkpoint(path)
    w, s = ck.fp8_matrix("layers.0.mlp.experts.2.down_proj", 256, 128)
    assert np.array_equal(w, host["experts"][2]["down_w"]) and np.array_equal(s, host["experts"][2]["down_s"])
    r = ck.f32("layers.0.mlp.gate.weight")
    assert r.dtype == np.float32 and np.array_equal(r.view(np.uint32), r_bits.astype(np.uint32) << 16)


def test_suffix_lookup_prefix_then_bare(tmp_path):
    paths = []
    for sub, prefix in (("x", "model"), ("y", "")):
        os.makedirs(tmp_path / sub)
        paths.append(_tiny(tmp_path / sub, prefix=prefix)[2])
    for p in paths:
        ck = ingest.Checkpoint(p)
        assert ck.find("layers.0.mlp.gate.weight") is not None
        assert ck.find("layers.0.mlp.gate.bias") is None


def test_sharded_directory(tmp_path):
    host, _, d = _tiny(tmp_path, router_dt="F32", split=True)
    ck = ingest.Checkpoint(d)
    assert len(ck.files) == 2
    assert np.array_equal(ck.f32("layers.0.mlp.gate.weight"), host["router"])
    for e in range(4):
        ck.fp8_matrix(f"layers.0.mlp.experts.{e}.gate_proj", 128, 256)


def test_shape_dtype_and_missing_errors(tmp_path):
    _, _, path = _tiny(tmp_path)
    ck = ingest.Checkpoint(path)
    with pytest.raises(ingest.CheckpointError, match="shape"):
        ck.fp8_matrix("layers.0.mlp.experts.0.gate_proj", 256, 128)
    with pytest.raises(ingest.CheckpointError, match="missing"):
        ck.fp8_matrix("layers.0.mlp.experts.9.gate_proj", 128, 256)
    with pytest.raises(ingest.CheckpointError, match="expected F8_E4M3"):
        ck.fp8_matrix("layers.0.mlp.gate", 4, 256)


def test_corrupt_files_rejected(tmp_path):
    _, _, path = _tiny(tmp_path)
    data = bytearray(open(path, "rb").read())
    bad = tmp_path / "bad.safetensors"
    bad.write_bytes((10 ** 12).to_bytes(8, "little") + bytes(data[8:]))
    with pytest.raises(ingest.CheckpointError, match="header"):
        ingest.SafetensorsFile(str(bad))
    bad.write_bytes(bytes(data[:-100]))  # data segment cut short: offsets out of range
    with pytest.raises(ingest.CheckpointError, match="out of range"):
        ingest.SafetensorsFile(str(bad))
    bad.write_bytes(b"\x03\x00\x00\x00\x00\x00\x00\x00{x}")
    with pytest.raises(ingest.CheckpointError, match="JSON"):
        ingest.SafetensorsFile(str(bad))


def test_duplicate_tensor_across_files(tmp_path):
    a = np.zeros((2, 2), np.float32)
    ingest.write_safetensors(str(tmp_path / "a.safetensors"), {"t": ("F32", a)})
    ingest.write_safetensors(str(tmp_path / "b.safetensors"), {"t": ("F32", a)})
    with pytest.raises(ingest.CheckpointError, match="two files"):
        ingest.Checkpoint(str(tmp_path))
