"""The HBM plan's scratch figure (colizig_hip_plan_hbm, budget.zig:184-264
restated) against what the forward really allocates: in a fresh process per
case, one forward of a layer with a shared expert (hidden 512, 16 experts,
top-4, inter 256, shared 256) at S tokens in each prefill mode; the plan for
max_tokens = S must count exactly the bytes the forward's scratch holds."""
from __future__ import annotations

import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.parametrize("mode,S", [(0, 64), (1, 64), (1, 1), (0, 300)])
def test_plan_scratch_equals_allocation(gpu, mode, S):
    r = subprocess.run([sys.executable, "-u", os.path.join(HERE, "work_child.py"), str(mode), str(S)],
                       capture_output=True, text=True, timeout=180)
    assert r.returncode == 0, r.stderr[-2000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    print(out, flush=True)
    assert out["allocated"] > 0
    assert out["planned"] == out["allocated"]
