"""The engine-side loader's success path on the GPU (cz_gpu_loader.cpp, the
dlopen counterpart of src/backend/gpu.zig:72-190): init reports the backend
up (1, gpu.zig:98-104), matmuls run on the GPU (true, gpu.zig:175-190) and
match the oracle's matmulFp8 (fp8.zig:215-257) within 1e-5 relative L2,
keyed calls count in the stats line (gpu.zig:160-170), deinit leaves the
backend unavailable.  Run in a child process: the loader's deinit shuts the
library's one context, which this process's other tests share."""
from __future__ import annotations

import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def test_loader_success_path(gpu):
    print("loader success path (child process)", flush=True)
    r = subprocess.run([sys.executable, "-u", os.path.join(HERE, "loader_child.py")], capture_output=True,
                       text=True, timeout=180)
    assert r.returncode == 0, r.stderr[-2000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["init"] == 1 and out["available"] == 1, out
    assert "GPU backend up" in out["line"] and "gfx950" in out["device"]
    assert out["has_moe"] == 1
    assert out["matmul_ok"] == [1, 1, 1, 1, 1]
    assert out["max_rel_l2"] < 1e-5, out
    # keyed calls: 77 (miss, then hit), 78 (miss), 79 (miss); key 0 uploads without counting
    assert "4 matmuls" in out["stats_line"] and "25.0% hit" in out["stats_line"], out["stats_line"]
    assert out["available_after_deinit"] == 0
