"""Checkpoint ingest: MoE layers from safetensors files into the HBM expert
cache (Layer.load, moe.zig:306-328; loadExpert, moe.zig:251-292).

Tensor names follow the reference's lookup (weights.zig:204-207): a suffix
such as ``layers.{l}.mlp.experts.{e}.gate_proj.weight`` is looked up as
``<prefix>.<suffix>`` first, then bare.  Per layer:

- router ``layers.{l}.mlp.gate.weight`` [E, H], F32 or BF16, kept in its
  own dtype in HBM (NativeMatrix.load, tensors.zig:74-94: other dtypes are
  refused);
- experts ``layers.{l}.mlp.experts.{e}.{gate,up,down}_proj.weight`` (F8_E4M3
  bytes, [I, H] / [I, H] / [H, I]) with ``.weight_scale_inv`` (F32, one per
  128 x 128 block), the multiplier the reference applies to the E4M3 value
  (fp8.zig:105);
- a shared expert, when the layer has one: ``shared_expert.{gate,up,down}_proj``
  as F32 or BF16 NativeMatrix rows (the reference's form, moe.zig:316-325), or
  in the routed experts' block-FP8 form, and ``shared_expert_gate.weight`` [H]
  (F32 or BF16).

The safetensors container (safetensors.zig:126-237): an 8-byte little-endian
header length, a JSON header {name: {dtype, shape, data_offsets}}, then the
data segment.  Files are memory-mapped read-only; nothing in a file is
executed.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass

import numpy as np

from . import moe

_MAX_HEADER = 100 << 20

# safetensors dtype -> (numpy dtype of the stored bytes, bytes per element)
_DTYPES = {
    "F64": (np.float64, 8), "F32": (np.float32, 4), "F16": (np.float16, 2), "BF16": (np.uint16, 2),
    "F8_E4M3": (np.uint8, 1), "F8_E5M2": (np.uint8, 1), "I64": (np.int64, 8), "I32": (np.int32, 4),
    "I16": (np.int16, 2), "I8": (np.int8, 1), "U8": (np.uint8, 1), "BOOL": (np.uint8, 1),
}


class CheckpointError(ValueError):
    pass


@dataclass
class TensorInfo:
    dtype: str
    shape: tuple
    begin: int  # byte offsets in the data segment
    end: int


class SafetensorsFile:
    """One .safetensors file: its header and read-only views of its tensors."""

    def __init__(self, path: str):
        self.path = path
        size = os.path.getsize(path)
        if size < 8:
            raise CheckpointError(f"{path}: not a safetensors file")
        with open(path, "rb") as f:
            n = int.from_bytes(f.read(8), "little")
            if n == 0 or n > _MAX_HEADER:
                raise CheckpointError(f"{path}: header length {n}")
            if 8 + n > size:
                raise CheckpointError(f"{path}: header past the end of the file")
            try:
                header = json.loads(f.read(n).decode("utf-8"))
            except (UnicodeDecodeError, json.JSONDecodeError) as e:
                raise CheckpointError(f"{path}: bad header JSON ({e})") from None
        self.data_offset = 8 + n
        data_len = size - self.data_offset
        self.tensors: dict[str, TensorInfo] = {}
        for name, v in header.items():
            if name == "__metadata__":
                continue
            try:
                dt, shape, (b, e) = v["dtype"], tuple(int(s) for s in v["shape"]), v["data_offsets"]
            except (KeyError, TypeError, ValueError):
                raise CheckpointError(f"{path}: bad entry for {name}") from None
            if dt not in _DTYPES:
                raise CheckpointError(f"{path}: {name}: unsupported dtype {dt}")
            numel = int(np.prod(shape, dtype=np.int64)) if shape else 1
            if not (0 <= b <= e <= data_len) or e - b != numel * _DTYPES[dt][1]:
                raise CheckpointError(f"{path}: {name}: data offsets out of range or size mismatch")
            self.tensors[name] = TensorInfo(dt, shape, int(b), int(e))
        self._map = np.memmap(path, dtype=np.uint8, mode="r") if data_len > 0 else None

    def raw(self, name: str) -> tuple[TensorInfo, np.ndarray]:
        """The tensor's stored elements (BF16 as uint16, F8 as uint8), no copy."""
        t = self.tensors[name]
        npdt, _ = _DTYPES[t.dtype]
        buf = self._map[self.data_offset + t.begin:self.data_offset + t.end]
        return t, buf.view(npdt).reshape(t.shape)


def _bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    return (np.asarray(u16, dtype=np.uint32) << 16).view(np.float32)


class Checkpoint:
    """A set of safetensors files (a directory or a list of paths) with the
    reference's suffix lookup."""

    def __init__(self, paths, prefix: str = "model"):
        if isinstance(paths, (str, os.PathLike)) and os.path.isdir(paths):
            paths = sorted(os.path.join(paths, f) for f in os.listdir(paths) if f.endswith(".safetensors"))
        elif isinstance(paths, (str, os.PathLike)):
            paths = [paths]
        self.files = [SafetensorsFile(str(p)) for p in paths]
        if not self.files:
            raise CheckpointError("no .safetensors files")
        self.prefix = prefix
        self.where: dict[str, SafetensorsFile] = {}
        for f in self.files:
            for name in f.tensors:
                if name in self.where:
                    raise CheckpointError(f"tensor {name} in two files")
                self.where[name] = f

    def find(self, suffix: str) -> str | None:
        """weights.zig:204-207: `<prefix>.<suffix>`, then `<suffix>`."""
        for name in (f"{self.prefix}.{suffix}" if self.prefix else None, suffix):
            if name and name in self.where:
                return name
        return None

    def raw(self, suffix: str) -> tuple[TensorInfo, np.ndarray]:
        name = self.find(suffix)
        if name is None:
            raise CheckpointError(f"tensor {suffix} missing")
        return self.where[name].raw(name)

    def f32(self, suffix: str) -> np.ndarray:
        """An F32 / BF16 / F16 tensor as float32 (exact widening)."""
        t, a = self.raw(suffix)
        if t.dtype == "F32":
            return np.ascontiguousarray(a, dtype=np.float32)
        if t.dtype == "BF16":
            return _bf16_to_f32(a)
        if t.dtype == "F16":
            return a.astype(np.float32)
        raise CheckpointError(f"{suffix}: dtype {t.dtype}, expected F32, BF16 or F16")

    def native(self, suffix: str, shape: tuple) -> np.ndarray:
        """NativeMatrix.load (tensors.zig:74-94): an F32 matrix as float32 or a
        BF16 one as its uint16 bits; any other dtype is refused."""
        t, a = self.raw(suffix)
        if t.dtype not in ("F32", "BF16"):
            raise CheckpointError(f"{suffix}: dtype {t.dtype}, expected F32 or BF16")
        if t.shape != shape:
            raise CheckpointError(f"{suffix}: shape {t.shape}, expected {shape}")
        return np.ascontiguousarray(a)

    def dtype(self, suffix: str) -> str:
        return self.raw(suffix)[0].dtype

    def fp8_matrix(self, stem: str, rows: int, cols: int) -> tuple[np.ndarray, np.ndarray]:
        """`stem.weight` (F8_E4M3 [rows, cols]) and `stem.weight_scale_inv`
        (F32 [ceil(rows/128), ceil(cols/128)]), as Fp8Matrix.load takes them."""
        t, w = self.raw(f"{stem}.weight")
        if t.dtype != "F8_E4M3":
            raise CheckpointError(f"{stem}.weight: dtype {t.dtype}, expected F8_E4M3")
        if t.shape != (rows, cols):
            raise CheckpointError(f"{stem}.weight: shape {t.shape}, expected {(rows, cols)}")
        s = self.f32(f"{stem}.weight_scale_inv")
        if s.shape != (moe.nblk(rows), moe.nblk(cols)):
            raise CheckpointError(f"{stem}.weight_scale_inv: shape {s.shape}, "
                                  f"expected {(moe.nblk(rows), moe.nblk(cols))}")
        return w, s


def load_layer(ckpt: Checkpoint, layer: int, d: moe.Dims, layer_id: int | None = None) -> moe.Layer:
    """Layer.load + loadExpert for every expert (moe.zig:251-328): the
    checkpoint's layer `layer` registered as library layer `layer_id`
    (default: the same number), experts uploaded to their HBM slots."""
    H, E, I, SI = d.hidden, d.experts, d.inter, d.shared_inter
    p = f"layers.{layer}.mlp"
    router = ckpt.native(f"{p}.gate.weight", (E, H))
    lid = layer if layer_id is None else layer_id
    if router.dtype == np.uint16:  # BF16 rows stay BF16 (dotBf16 logits)
        L = moe.Layer.load(lid, d, np.zeros((E, H), np.float32))
        L.set_router_bf16(router)
    else:
        L = moe.Layer.load(lid, d, router)
    for e in range(E):
        gw, gs = ckpt.fp8_matrix(f"{p}.experts.{e}.gate_proj", I, H)
        uw, us = ckpt.fp8_matrix(f"{p}.experts.{e}.up_proj", I, H)
        dw, ds = ckpt.fp8_matrix(f"{p}.experts.{e}.down_proj", H, I)
        L.load_expert(e, gw, gs, uw, us, dw, ds)
    if SI:
        g = ckpt.f32(f"{p}.shared_expert_gate.weight").reshape(-1)
        if g.shape != (H,):
            raise CheckpointError(f"{p}.shared_expert_gate.weight: {g.size} values, expected {H}")
        if ckpt.dtype(f"{p}.shared_expert.gate_proj.weight") == "F8_E4M3":
            gw, gs = ckpt.fp8_matrix(f"{p}.shared_expert.gate_proj", SI, H)
            uw, us = ckpt.fp8_matrix(f"{p}.shared_expert.up_proj", SI, H)
            dw, ds = ckpt.fp8_matrix(f"{p}.shared_expert.down_proj", H, SI)
            L.set_shared(gw, gs, uw, us, dw, ds, g)
        else:  # NativeMatrix rows (moe.zig:316-325), one dtype for the three
            gm = ckpt.native(f"{p}.shared_expert.gate_proj.weight", (SI, H))
            um = ckpt.native(f"{p}.shared_expert.up_proj.weight", (SI, H))
            dm = ckpt.native(f"{p}.shared_expert.down_proj.weight", (H, SI))
            if not (gm.dtype == um.dtype == dm.dtype):
                raise CheckpointError(f"{p}.shared_expert: gate/up/down of different dtypes")
            L.set_shared_native(gm, um, dm, g)
    return L


def write_safetensors(path: str, tensors: dict) -> None:
    """Writes {name: (dtype, array)} as a safetensors file (tests and tools
    that build small checkpoints; BF16 given as uint16 bits, F8 as uint8)."""
    header, blobs, off = {}, [], 0
    for name, (dt, a) in tensors.items():
        a = np.ascontiguousarray(a)
        if a.dtype != np.dtype(_DTYPES[dt][0]):
            raise CheckpointError(f"{name}: array dtype {a.dtype} does not store {dt}")
        b = a.tobytes()
        header[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(header).encode("utf-8")
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little"))
        f.write(h)
        for b in blobs:
            f.write(b)
