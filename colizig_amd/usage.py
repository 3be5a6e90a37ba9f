"""Learned routed-expert priors for the streaming tier (ExpertUsage,
src/runtime/expert_usage.zig): per (layer, expert) routing counts persisted as
`.colizig_usage` next to the checkpoint and used to pre-warm the HBM expert
pool on the next run.

File format (expert_usage.zig:76-128): the magic ``CZU1``, u32 layers, u32
experts, then layers * experts u64 counts, all little-endian.  A file whose
size or header does not match the model reads as no priors; saving merges
into the existing totals (saturating add)."""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import _lib
from .moe import GpuBackendError

MAGIC = b"CZU1"
FILENAME = ".colizig_usage"


class ExpertUsage:
    def __init__(self, layers: int, experts: int, counts: np.ndarray | None = None):
        self.layers, self.experts = layers, experts
        self.counts = np.zeros((layers, experts), np.uint64) if counts is None else \
            np.ascontiguousarray(counts, dtype=np.uint64).reshape(layers, experts)

    @staticmethod
    def load(path: str, layers: int, experts: int) -> "ExpertUsage | None":
        """expert_usage.zig:76-97: None when absent, unreadable or mismatched."""
        try:
            with open(path, "rb") as f:
                buf = f.read()
        except OSError:
            return None
        if len(buf) != 12 + layers * experts * 8 or buf[:4] != MAGIC:
            return None
        if int.from_bytes(buf[4:8], "little") != layers or int.from_bytes(buf[8:12], "little") != experts:
            return None
        return ExpertUsage(layers, experts, np.frombuffer(buf, dtype="<u8", offset=12).copy())

    def save(self, path: str) -> None:
        """expert_usage.zig:99-128: merge into the existing totals and rewrite
        (best effort: an I/O error leaves the file as it was)."""
        prior = ExpertUsage.load(path, self.layers, self.experts)
        total = self.counts.astype(np.uint64)
        if prior is not None:
            s = prior.counts + total
            total = np.where(s < prior.counts, np.uint64(np.iinfo(np.uint64).max), s)  # saturate
        data = MAGIC + self.layers.to_bytes(4, "little") + self.experts.to_bytes(4, "little") + \
            total.astype("<u8").tobytes()
        tmp = f"{path}.tmp"
        try:
            with open(tmp, "wb") as f:
                f.write(data)
            os.replace(tmp, path)
        except OSError:
            pass

    def top_ascending(self, layer: int, n: int) -> list[int]:
        """expert_usage.zig:53-75: the layer's n hottest experts with a
        non-zero count (ties: lower id first), returned in ascending heat."""
        row = self.counts[layer]
        order = sorted((e for e in range(self.experts) if row[e] > 0), key=lambda e: (-int(row[e]), e))[:n]
        return order[::-1]

    @staticmethod
    def from_device(layer0: int, layers: int, experts: int) -> "ExpertUsage":
        """The routed-selection counts the device kept for the layers
        layer0 .. layer0 + layers - 1 (one per pick of each routed token,
        bumpUsage, moe.zig:428-432)."""
        u = ExpertUsage(layers, experts)
        rc = _lib.hip().colizig_hip_usage_read(layer0, layers, experts, u.counts.ctypes.data_as(ctypes.c_void_p))
        if rc != 0:
            raise GpuBackendError("colizig_hip_usage_read", rc)
        return u

    @staticmethod
    def from_pool(layer0: int, layers: int, experts: int) -> "ExpertUsage":
        """The streamed layers' counts (the same device counters)."""
        return ExpertUsage.from_device(layer0, layers, experts)

    def warm_pool(self, layer0: int) -> int:
        """warmCaches (expert_usage.zig:137-160) on the HBM pool; returns the
        number of experts filled."""
        rc = _lib.hip().colizig_hip_stream_warm(layer0, self.layers, self.experts,
                                                self.counts.ctypes.data_as(ctypes.c_void_p))
        if rc < 0:
            raise GpuBackendError("colizig_hip_stream_warm", rc)
        return rc
