"""The one-launch decode's failure path (cz_fused.h): every exchange between
the workgroups of an XCD is a bounded poll; one that runs out sets a word in
host memory, its kernel finishes with what it read, and colizig_hip_sync
reports -5 (a negative rc means the caller runs its CPU path, the contract
of fp8.zig:182-187 and gpu.zig:72-109).  A host hook makes one chain
position poll for a tag no layer writes, so every poll of that layer gives
up; the chain must still end in bounded time, the error must be reported
once, and the next clean step must match the oracle's chain."""
from __future__ import annotations

import time

import numpy as np
import pytest

from colizig_amd import _lib, moe, synth
from tests.test_gpu_chain import chain_vs_oracle, say

pytestmark = pytest.mark.gpu


def test_placement_census(gpu):
    """The init census found the workgroup placement the one-launch decode
    needs on this device (8 XCDs, one workgroup of each rank per XCD), so the
    one-launch decode serves a Qwen3-30B-A3B-shape chain."""
    hip = _lib.hip()
    assert hip.colizig_hip_fused_placement() == 1
    H, E, K, I = 2048, 128, 8, 768
    L = moe.Layer.load(2600, moe.dims(H, E, K, I), np.zeros((E, H), np.float32))
    L.synth(seed=26)
    assert hip.colizig_hip_fused_decode_active(2600, 1, 1) == 1


@pytest.mark.parametrize("pos", [0, 2])
def test_poll_give_up_reported_then_clean(gpu, oracle_lib, pos):
    """Config-1 shapes, 3 chained layers at batch 1 (the one-launch decode):
    with the hook on position pos, the chain ends within seconds and
    colizig_hip_sync returns -5 with the exchange message, once; with the hook
    off, the next chain from a fresh x0 returns 0 and matches the oracle's
    chain (routing bit-exact, residual within 1e-3)."""
    say(f"one-launch decode: polls of chain position {pos} give up")
    hip = _lib.hip()
    hosts = [synth.make_layer(512, 16, 4, 256, 0, True, seed=910 + l) for l in range(3)]
    base = 2700 + 10 * pos
    for l, h in enumerate(hosts):
        h["registered"] = moe.register_layer(base + l, h)
    assert hip.colizig_hip_fused_decode_active(base, 3, 1) == 1
    x0 = synth.hidden_states(1, 512, seed=pos)
    xb = moe.DeviceBuffer(x0.nbytes)
    xb.upload(x0)
    prev = hip.colizig_hip_set_fused_fault(pos)
    try:
        t0 = time.perf_counter()
        assert hip.colizig_hip_chain_decode(base, 3, xb.ptr, 1, 1e-6, None, None, None, None) == 0
        rc = hip.colizig_hip_sync()
        dt = time.perf_counter() - t0
    finally:
        hip.colizig_hip_set_fused_fault(prev)
    msg = _lib.last_error()
    say(f"  faulted chain: rc {rc} after {dt * 1e3:.1f} ms: {msg}")
    assert rc == -5
    assert "timed out" in msg
    assert dt < 5.0  # every wave left its bounded waits (20 ms each)
    assert hip.colizig_hip_sync() == 0  # reported once, then cleared
    # the next clean steps: the oracle's chain from a fresh x0
    chain_vs_oracle(oracle_lib, hosts, base, 1, tokens=2, seed=100 + pos, label=f"after fault at {pos}")
    xb.free()
