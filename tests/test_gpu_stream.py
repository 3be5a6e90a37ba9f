"""Streaming tier: experts in pinned host memory, an HBM pool smaller than
the working set.  A streamed layer runs the same three-kernel decode on the
same bytes as a resident one with the one-launch decode switched off, so
outputs are bit-identical; the pool counters follow
the cache's invariants (moe.zig:711-741: hits + misses = uses, every miss
and prefetch is one load)."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from colizig_amd import _lib, moe, synth
from tests.helpers import f32_bits

pytestmark = pytest.mark.gpu

H, E, K, I = 512, 16, 4, 256
D = moe.dims(H, E, K, I)
SLOT = 3 * I * H + 3 * moe.nblk(I) * moe.nblk(H) * 4
_state = {}


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


NSLOTS = 16  # = E: one layer's whole selection fits at any S; 4 layers x 16 experts do not


@pytest.fixture(scope="module")
def pool(gpu):
    """One pool per context, freed (with its streamed layers) after the
    module.  The resident side of every comparison runs the streamed tier's
    three-kernel decode: the one-launch decode is switched off while this
    module runs and restored after it."""
    moe.stream_pool_init(D, NSLOTS * SLOT)
    hip = _lib.hip()
    prev = hip.colizig_hip_set_fused_decode(0)
    yield True
    hip.colizig_hip_set_fused_decode(prev)
    moe.stream_pool_free()


def _layers(base_res, base_str, nl, seed, zipf=True):
    hosts, keep = [], []
    for l in range(nl):
        h = synth.make_layer(H, E, K, I, 0, True, seed=seed + l)
        if zipf:
            h["router_bias"] = synth.zipf_router_bias(E, 1.2, seed=seed + l)
        hosts.append(h)
        moe.register_layer(base_res + l, h)
        moe.register_layer(base_str + l, h)
        wb, sb = moe.host_expert_slab(D, h["experts"])
        moe.stream_layer_from_host(base_str + l, wb, sb)
        keep += [wb, sb]
    _state.setdefault("keep", []).extend(keep)  # pinned slabs live as long as the layers
    return hosts


def test_stream_chain_bit_identical_to_resident(pool):
    say("stream chain vs resident, 4 layers, 16-slot pool")
    nl = 4
    _layers(2000, 2100, nl, seed=31)
    hip = _lib.hip()
    x0 = synth.hidden_states(1, H, seed=31)
    xr, xs = moe.DeviceBuffer(x0.nbytes), moe.DeviceBuffer(x0.nbytes)
    xr.upload(x0)
    xs.upload(x0)
    st0 = moe.stream_stats()
    steps = 8
    for t in range(steps):
        assert hip.colizig_hip_chain_decode(2000, nl, xr.ptr, 1, 1e-6, None, None, None, None) == 0
        assert hip.colizig_hip_stream_decode(2100, nl, xs.ptr, 1, 1e-6) == 0, _lib.last_error()
        assert hip.colizig_hip_sync() == 0
        a = xr.download(np.empty_like(x0))
        b = xs.download(np.empty_like(x0))
        assert np.array_equal(f32_bits(a), f32_bits(b)), f"step {t}"
    st = {k: v - st0[k] for k, v in moe.stream_stats().items() if k not in ("slots", "resident")}
    say(f"  {st}")
    uses = steps * nl * K  # S=1: K distinct experts per layer per step
    assert st["hits"] + st["misses"] == uses
    assert st["loads"] == st["misses"] + st["prefetch_issued"]
    assert st["bytes_h2d"] == st["loads"] * SLOT
    assert st["misses"] > 0
    if st["loads"] > NSLOTS:
        assert st["evictions"] > 0


def test_stream_moe_forward_bit_identical(pool):
    say("stream moe_forward vs resident, S=1 and S=32")
    _layers(2200, 2300, 1, seed=41)
    Lr = moe.Layer(2200, D, True)
    Ls = moe.Layer(2300, D, True)
    for S in (1, 3, 32):  # S = 32 takes the grouped regime
        x = synth.hidden_states(S, H, seed=41 + S)
        a, ia, ga = Lr.forward(x)
        b, ib, gb = Ls.forward(x)
        assert np.array_equal(ia, ib) and np.array_equal(f32_bits(ga), f32_bits(gb))
        assert np.array_equal(f32_bits(a), f32_bits(b)), f"S={S}"


def test_stream_refused_by_plain_chain(pool):
    _layers(2400, 2500, 1, seed=51, zipf=False)
    hip = _lib.hip()
    xb = moe.DeviceBuffer(H * 4)
    xb.upload(np.zeros((1, H), np.float32))
    assert hip.colizig_hip_chain_decode(2500, 1, xb.ptr, 1, 1e-6, None, None, None, None) == -1
    assert hip.colizig_hip_chain_graph_create(2500, 1, xb.ptr, 1, 1e-6) < 0


def test_stream_priors_warm_the_pool(pool):
    """Learned priors (expert_usage.zig): the pool's routing counts, an empty
    pool (a fresh run), then a warm start from the counts: the warmed experts
    are prefetches that later steps hit, and results stay bit-identical to
    the resident layers."""
    from colizig_amd.usage import ExpertUsage
    say("stream priors: count, evict, warm")
    nl = 2
    _layers(2300, 2400, nl, seed=57)
    hip = _lib.hip()
    x0 = synth.hidden_states(1, H, seed=57)
    xr, xs = moe.DeviceBuffer(x0.nbytes), moe.DeviceBuffer(x0.nbytes)
    xr.upload(x0)
    xs.upload(x0)

    def step(t):
        assert hip.colizig_hip_chain_decode(2300, nl, xr.ptr, 1, 1e-6, None, None, None, None) == 0
        assert hip.colizig_hip_stream_decode(2400, nl, xs.ptr, 1, 1e-6) == 0, _lib.last_error()
        assert hip.colizig_hip_sync() == 0
        a, b = xr.download(np.empty_like(x0)), xs.download(np.empty_like(x0))
        assert np.array_equal(f32_bits(a), f32_bits(b)), f"step {t}"

    for t in range(6):
        step(t)
    u = ExpertUsage.from_pool(2400, nl, E)
    assert int(u.counts.sum()) == 6 * nl * K  # one count per selected expert per layer step
    assert hip.colizig_hip_stream_evict_all() == 0
    assert moe.stream_stats()["resident"] == 0
    hot = int((u.counts > 0).sum())
    st0 = moe.stream_stats()
    warmed = u.warm_pool(2400)
    assert warmed == min(NSLOTS, hot)
    st1 = moe.stream_stats()
    assert st1["prefetch_issued"] - st0["prefetch_issued"] == warmed
    assert st1["resident"] == warmed
    for t in range(6, 9):
        step(t)
    st2 = moe.stream_stats()
    assert st2["prefetch_hits"] > st1["prefetch_hits"]
    say(f"  warmed {warmed} of {hot}; prefetch hits {st2['prefetch_hits'] - st1['prefetch_hits']}")


def test_stream_stats_window(pool):
    """colizig_hip_stream_stats_reset opens a window with its own counters:
    the warmed pool's prefetches were issued before the window, so the
    window's hits on them are hits but not prefetch hits; inside the window
    prefetch hits plus wasted never exceed the prefetches issued, every miss
    and prefetch is one load, and the queue peak is the window's."""
    from colizig_amd.usage import ExpertUsage
    say("stream stats window after a warm start")
    nl = 2
    _layers(2600, 2700, nl, seed=61)
    hip = _lib.hip()
    xs = moe.DeviceBuffer(H * 4)
    xs.upload(synth.hidden_states(1, H, seed=61))
    for _ in range(4):
        assert hip.colizig_hip_stream_decode(2700, nl, xs.ptr, 1, 1e-6) == 0, _lib.last_error()
    assert hip.colizig_hip_sync() == 0
    u = ExpertUsage.from_pool(2700, nl, E)
    assert hip.colizig_hip_stream_evict_all() == 0
    warmed = u.warm_pool(2700)
    assert warmed > 0
    assert hip.colizig_hip_stream_stats_reset() == 0
    st = moe.stream_stats()
    assert all(st[k] == 0 for k in st if k not in ("slots", "resident", "sched_queue_peak"))
    steps = 6
    for _ in range(steps):
        assert hip.colizig_hip_stream_decode(2700, nl, xs.ptr, 1, 1e-6) == 0, _lib.last_error()
    assert hip.colizig_hip_sync() == 0
    st = moe.stream_stats()
    say(f"  {st}")
    assert st["hits"] + st["misses"] == steps * nl * K
    assert st["hits"] > 0  # the warmed experts
    assert st["prefetch_hits"] + st["prefetch_wasted"] <= st["prefetch_issued"]
    assert st["loads"] == st["misses"] + st["prefetch_issued"]
    assert st["bytes_h2d"] == st["loads"] * SLOT
