"""Child process of tests/test_gpu_loader.py: the engine-side loader
(cz_gpu_loader.cpp, the dlopen counterpart of src/backend/gpu.zig:72-190)
driven through its success path on the GPU.  Prints one JSON line."""
from __future__ import annotations

import ctypes
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

from colizig_amd import _lib, synth  # noqa: E402
from oracle import oracle as orc  # noqa: E402


def main() -> None:
    ld = _lib.loader()
    err = ctypes.create_string_buffer(256)
    out = {"init": ld.czgpu_init(_lib.HIP_LIB.encode(), err, 256), "line": err.value.decode(),
           "available": ld.czgpu_available(), "has_moe": ld.czgpu_has_moe(),
           "device": ld.czgpu_device_name().decode()}
    ld.czgpu_set_vram_budget(1 << 30)
    rng = np.random.default_rng(5)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    worst = 0.0
    calls = []
    mats = {}
    for (S, I, O, key) in [(1, 2048, 768, 0), (1, 2048, 768, 77), (1, 2048, 768, 77), (3, 768, 2048, 78),
                           (2, 200, 5, 79)]:
        # a key names one matrix (Fp8Matrix.key, moe.zig:97-99): a repeated key passes the same bytes
        if key not in mats or key == 0:
            mats[key] = synth.block_quantize(rng.normal(0.0, 0.02, size=(O, I)).astype(np.float32))
        w, s = mats[key]
        x = rng.normal(size=(S, I)).astype(np.float32)
        y = np.zeros((S, O), np.float32)
        ok = ld.czgpu_matmul_fp8(p(y), p(x), p(w), p(s), S, I, O, key)
        ref = orc.matmul_fp8(x, w, s, S, I, O)
        err_l2 = float(np.linalg.norm(y - ref) / np.linalg.norm(ref))
        worst = max(worst, err_l2)
        calls.append(ok)
    out["matmul_ok"] = calls
    out["max_rel_l2"] = worst
    line = ctypes.create_string_buffer(256)
    n = ld.czgpu_stats_line(line, 256)
    out["stats_line"] = line.value.decode()[:n]
    ld.czgpu_deinit()
    out["available_after_deinit"] = ld.czgpu_available()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
