"""colizig_amd - colizig's block-FP8 MoE expert path on MI355X (gfx950).

libcolizig_hip.so (csrc/) is the product: hand-written HIP kernels behind
colizig's src/backend C-ABI (include/colizig_hip.h).  This package holds the
build step, ctypes bindings, a host mirror of the reference's MoE interface
(moe.py) and a seeded synthetic-layer generator (synth.py).
"""
from . import _lib  # noqa: F401

__all__ = ["_lib", "moe", "synth", "build"]
