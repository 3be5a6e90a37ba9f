"""Streaming tier where the streamed layer's routing is a launch of its own:
more than 128 experts, or a BF16 router (with at most 128 experts and an
f32 router, the router kernel's last block routes the token instead).  A
streamed layer runs the same three-kernel decode on the same bytes as a
resident one, so outputs are bit-identical; the pool counters follow the
cache's invariants (moe.zig:711-741)."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from colizig_amd import _lib, moe, synth
from tests.helpers import f32_bits

pytestmark = pytest.mark.gpu

H, E, K, I = 512, 160, 4, 256
D = moe.dims(H, E, K, I)
SLOT = 3 * I * H + 3 * moe.nblk(I) * moe.nblk(H) * 4
NSLOTS = 24  # fewer than one layer's experts: misses and evictions
_keep = []


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def pool(gpu):
    """A pool of this module's shape, freed (with its streamed layers) after
    it; the resident side runs the three-kernel decode (more than 128
    experts: the one-launch decode does not take these layers)."""
    moe.stream_pool_init(D, NSLOTS * SLOT)
    yield True
    moe.stream_pool_free()


def _layers(base_res, base_str, nl, seed, bf16_router=False):
    for l in range(nl):
        h = synth.make_layer(H, E, K, I, 0, True, seed=seed + l)
        h["router_bias"] = synth.zipf_router_bias(E, 1.2, seed=seed + l)
        if bf16_router:  # BF16 bits: registered as a NativeMatrix bf16 router
            h["router"] = synth.f32_to_bf16_bits(h["router"])
        moe.register_layer(base_res + l, h)
        moe.register_layer(base_str + l, h)
        wb, sb = moe.host_expert_slab(D, h["experts"])
        moe.stream_layer_from_host(base_str + l, wb, sb)
        _keep.extend([wb, sb])  # pinned slabs live as long as the layers


@pytest.mark.parametrize("bf16_router", [False, True])
def test_stream_routing_launch_bit_identical_to_resident(pool, bf16_router):
    say(f"stream chain vs resident, E {E}, {NSLOTS}-slot pool, BF16 router {bf16_router}")
    nl = 3
    base_res, base_str = (3000, 3100) if not bf16_router else (3200, 3300)
    _layers(base_res, base_str, nl, seed=61 + (7 if bf16_router else 0), bf16_router=bf16_router)
    hip = _lib.hip()
    assert hip.colizig_hip_fused_decode_active(base_res, nl, 1) == 0
    x0 = synth.hidden_states(1, H, seed=63)
    xr, xs = moe.DeviceBuffer(x0.nbytes), moe.DeviceBuffer(x0.nbytes)
    xr.upload(x0)
    xs.upload(x0)
    st0 = moe.stream_stats()
    steps = 6
    for t in range(steps):
        assert hip.colizig_hip_chain_decode(base_res, nl, xr.ptr, 1, 1e-6, None, None, None, None) == 0
        assert hip.colizig_hip_stream_decode(base_str, nl, xs.ptr, 1, 1e-6) == 0, _lib.last_error()
        assert hip.colizig_hip_sync() == 0
        a = xr.download(np.empty_like(x0))
        b = xs.download(np.empty_like(x0))
        assert np.all(np.isfinite(a))
        assert np.array_equal(f32_bits(a), f32_bits(b)), f"step {t}"
    st = {k: v - st0[k] for k, v in moe.stream_stats().items() if k not in ("slots", "resident")}
    say(f"  {st}")
    assert st["hits"] + st["misses"] == steps * nl * K  # S = 1: K distinct experts per layer step
    assert st["loads"] == st["misses"] + st["prefetch_issued"]
    assert st["bytes_h2d"] == st["loads"] * SLOT
    assert st["misses"] > 0
