"""Child process of tests/test_gpu_plan_scratch.py: in a fresh library state,
one grouped forward of a layer with a shared expert in the given prefill
mode, then the forward's scratch as allocated (colizig_hip_work_bytes) and as
the HBM plan counts it for that many tokens.  Prints one JSON line."""
from __future__ import annotations

import ctypes
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

from colizig_amd import _lib, moe, synth  # noqa: E402


def main() -> None:
    mode, S = int(sys.argv[1]), int(sys.argv[2])
    moe.init()
    hip = _lib.hip()
    hip.colizig_hip_set_prefill_fp8(mode)
    host = synth.make_layer(512, 16, 4, 256, 256, True, seed=3)
    L = moe.register_layer(0, host)
    L.forward(synth.hidden_states(S, 512, seed=3))
    got = ctypes.c_uint64(0)
    assert hip.colizig_hip_work_bytes(ctypes.byref(got)) == 0
    plan = moe.plan_hbm(moe.dims(512, 16, 4, 256, 256), 1, 1 << 40, max_tokens=S)
    print(json.dumps({"mode": mode, "S": S, "allocated": got.value, "planned": plan["scratch"]}), flush=True)


if __name__ == "__main__":
    main()
