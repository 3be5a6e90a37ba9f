"""The no-alloc forward (colizig_hip_moe_forward_dev_noalloc) against the
allocating one (colizig_hip_moe_forward_dev): same kernels on the same
bytes, so outputs, expert ids and gates are bit-identical.  Two calls in a
row, the second on fewer tokens, so the second runs over scratch that still
holds the first call's contents.  Sizes the static scratch cannot hold, and
the grouped regime, are refused on the host before anything is launched."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from colizig_amd import _lib, moe, synth
from tests.helpers import f32_bits

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _forward(fn, layer, x, K, H):
    S = x.shape[0]
    xb, ob = moe.DeviceBuffer(x.nbytes), moe.DeviceBuffer(S * H * 4)
    ib, gb = moe.DeviceBuffer(S * K * 4), moe.DeviceBuffer(S * K * 4)
    xb.upload(x)
    rc = fn(layer, xb.ptr, S, ob.ptr, ib.ptr, gb.ptr, None)
    assert rc == 0, (rc, _lib.last_error())
    assert _lib.hip().colizig_hip_sync() == 0
    out = ob.download(np.empty((S, H), np.float32))
    idx = ib.download(np.empty((S, K), np.uint32))
    gates = gb.download(np.empty((S, K), np.float32))
    return out, idx, gates


def _compare(layer, H, K, sizes, seed):
    hip = _lib.hip()
    for n, S in enumerate(sizes):
        say(f"  layer {layer}: call {n + 1}, S={S}")
        x = synth.hidden_states(S, H, seed=seed + S)
        ra = _forward(hip.colizig_hip_moe_forward_dev, layer, x, K, H)
        rb = _forward(hip.colizig_hip_moe_forward_dev_noalloc, layer, x, K, H)
        assert np.array_equal(ra[1], rb[1]), f"expert ids differ at S={S}"
        assert np.array_equal(f32_bits(ra[2]), f32_bits(rb[2])), f"gates differ at S={S}"
        assert np.array_equal(f32_bits(ra[0]), f32_bits(rb[0])), f"outputs differ at S={S}"
        assert np.isfinite(rb[0]).all()


def test_noalloc_matches_forward_tiny_shared(gpu):
    say("no-alloc forward vs forward_dev: H512 E16 K4 I256 SI128, S=9 then S=2")
    H, E, K, I, SI = 512, 16, 4, 256, 128
    moe.register_layer(9100, synth.make_layer(H, E, K, I, SI, True, seed=9100))
    _compare(9100, H, K, [9, 2], seed=9100)


def test_noalloc_matches_forward_qwen3_30b(gpu):
    say("no-alloc forward vs forward_dev: H2048 E128 K8 I768, S=4 then S=1")
    H, E, K, I = 2048, 128, 8, 768
    moe.Layer.load(9200, moe.dims(H, E, K, I), np.zeros((E, H), np.float32)).synth(seed=9200)
    _compare(9200, H, K, [4, 1], seed=9200)


def test_noalloc_refuses_what_it_does_not_serve(gpu):
    say("no-alloc forward: refusals on the host")
    hip = _lib.hip()
    # H = 320 keeps every S in the decode regime; 4000 tokens need 5.1 MB of scratch
    H, E, K, I = 320, 4, 2, 64
    moe.register_layer(9300, synth.make_layer(H, E, K, I, 0, True, seed=9300))
    S = 4000
    xb, ob = moe.DeviceBuffer(S * H * 4), moe.DeviceBuffer(S * H * 4)
    assert hip.colizig_hip_moe_forward_dev_noalloc(9300, xb.ptr, S, ob.ptr, None, None, None) == -1
    assert "scratch" in _lib.last_error()
    # 16 tokens of a 128-tiled layer take the grouped regime
    H2, E2, K2, I2 = 512, 16, 4, 256
    moe.register_layer(9301, synth.make_layer(H2, E2, K2, I2, 0, True, seed=9301))
    x2, o2 = moe.DeviceBuffer(16 * H2 * 4), moe.DeviceBuffer(16 * H2 * 4)
    assert hip.colizig_hip_moe_forward_dev_noalloc(9301, x2.ptr, 16, o2.ptr, None, None, None) == -1
    assert "grouped" in _lib.last_error()
    # an unregistered layer
    assert hip.colizig_hip_moe_forward_dev_noalloc(9399, x2.ptr, 1, o2.ptr, None, None, None) == -6
