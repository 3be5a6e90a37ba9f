"""Grouped regime (many tokens per layer: prefill, batch decode) through the
C-ABI vs the oracle's forwardGrouped restatement (moe.zig:597-665).  Bar:
routing indices and gates bit-exact; outputs within 1e-3 relative L2."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from colizig_amd import _lib, moe, synth
from tests.helpers import f32_bits, rel_l2


@pytest.fixture(autouse=True)
def mfma_mode(gpu):
    """These cases run the grouped GEMMs on f16 MFMA (test_gpu_prefill_fp8.py
    runs them again on FP8 MFMA, the library's default)."""
    hip = _lib.hip()
    prev = hip.colizig_hip_set_prefill_fp8(0)
    yield
    hip.colizig_hip_set_prefill_fp8(prev)

pytestmark = pytest.mark.gpu

RTOL_L2 = 1e-3


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _check(Lg, Lo, x, what):
    out, idx, gates = Lg.forward(x)
    ro, ri, rg = Lo.forward(x)
    assert np.array_equal(idx, ri), f"{what}: routing differs"
    assert np.array_equal(f32_bits(gates), f32_bits(rg)), f"{what}: gates differ"
    err = rel_l2(out, ro)
    assert err < RTOL_L2, f"{what}: rel L2 {err}"
    return err


@pytest.mark.parametrize("S", [16, 64, 512])
def test_grouped_tiny_shapes_zipf(gpu, oracle_lib, S):
    """c1 shapes (hidden 512, 16 experts, top-4, inter 256) with Zipf(1.1)
    routing skew: dispatch + grouped MFMA GEMMs + ascending-id combine."""
    say(f"grouped c1 shapes S={S}")
    host = synth.make_layer(512, 16, 4, 256, 0, True, seed=1000 + S)
    host["router_bias"] = synth.zipf_router_bias(16, 1.1, seed=S)
    Lg = moe.register_layer(1000 + S, host)
    Lo = oracle_lib.OracleLayer(host)
    err = _check(Lg, Lo, synth.hidden_states(S, 512, seed=S), f"S={S}")
    say(f"  rel L2 {err:.2e}")


def test_grouped_shared_expert(gpu, oracle_lib):
    """Routed experts + the sigmoid-gated shared expert in the grouped regime."""
    say("grouped shared expert S=48")
    host = synth.make_layer(512, 32, 4, 256, 512, True, seed=77)
    Lg = moe.register_layer(1100, host)
    Lo = oracle_lib.OracleLayer(host)
    _check(Lg, Lo, synth.hidden_states(48, 512, seed=77), "shared S=48")


def test_grouped_norm_topk_false_and_ragged(gpu, oracle_lib):
    """norm_topk off, S not a multiple of the 32-row tile, one expert hot."""
    say("grouped norm_topk false, S=37")
    host = synth.make_layer(256, 64, 6, 256, 0, False, seed=5)
    bias = np.zeros(64, np.float32)
    bias[17] = 6.0  # nearly every token picks expert 17
    host["router_bias"] = bias
    Lg = moe.register_layer(1200, host)
    Lo = oracle_lib.OracleLayer(host)
    _check(Lg, Lo, synth.hidden_states(37, 256, seed=5), "S=37")


def test_grouped_many_experts_two_rounds(gpu, oracle_lib):
    """512 experts, top-10, 160 tokens with Zipf(1.1) skew: 1600 slots, more
    than the dispatch ranks in one round at 512 experts (1024 slots)."""
    say("grouped 512 experts top-10 S=160")
    host = synth.make_layer(256, 512, 10, 128, 0, True, seed=88)
    host["router_bias"] = synth.zipf_router_bias(512, 1.1, seed=88)
    Lg = moe.register_layer(1700, host)
    Lo = oracle_lib.OracleLayer(host)
    err = _check(Lg, Lo, synth.hidden_states(160, 256, seed=88), "E=512 S=160")
    say(f"  rel L2 {err:.2e}")


@pytest.mark.parametrize("E,S", [(128, 256), (128, 512), (256, 64)])
def test_grouped_router_tile_sizes(gpu, oracle_lib, E, S):
    """The many-token router picks 16, 8 or 4 tokens per workgroup from E and
    S (128 experts x 256 tokens: 8; x 512: 16; 256 experts x 64 tokens: 4);
    every size gives the decode router's logits, so routing stays bit-exact."""
    say(f"grouped router tiles E={E} S={S}")
    host = synth.make_layer(256, E, 8, 128, 0, True, seed=E + S)
    host["router_bias"] = synth.zipf_router_bias(E, 1.1, seed=E + S)
    Lg = moe.register_layer(1800 + S + E, host)
    Lo = oracle_lib.OracleLayer(host)
    _check(Lg, Lo, synth.hidden_states(S, 256, seed=E + S), f"E={E} S={S}")


def test_grouped_deterministic(gpu):
    say("grouped determinism")
    host = synth.make_layer(512, 16, 4, 256, 0, True, seed=9)
    Lg = moe.register_layer(1300, host)
    x = synth.hidden_states(96, 512, seed=9)
    a = Lg.forward(x)[0]
    b = Lg.forward(x)[0]
    assert np.array_equal(f32_bits(a), f32_bits(b))


def test_grouped_matches_decode_per_token(gpu):
    """Grouped (S=32) vs the decode kernels token by token: same routing, the
    same outputs to 1e-3 (the reference's own grouped-vs-dense bar is 1e-3
    abs, moe.zig:720-728)."""
    say("grouped vs decode per token")
    host = synth.make_layer(512, 16, 4, 256, 0, True, seed=21)
    Lg = moe.register_layer(1400, host)
    x = synth.hidden_states(32, 512, seed=21)
    og, ig, _ = Lg.forward(x)
    for t in range(32):
        od, id_, _ = Lg.forward(x[t:t + 1])
        assert np.array_equal(id_[0], ig[t])
        assert np.max(np.abs(od[0] - og[t])) < 1e-3


def test_grouped_chain_routing(gpu, oracle_lib):
    """x <- x + MoE(rms(x)) over 2 layers with S=32 tokens in the grouped
    regime: each layer's routing bit-exact on the GPU's own router input."""
    say("grouped chain S=32")
    H, S, nl = 512, 32, 2
    hosts = [synth.make_layer(H, 16, 4, 256, 0, True, seed=60 + l) for l in range(nl)]
    for l, h in enumerate(hosts):
        moe.register_layer(1500 + l, h)
    orcs = [oracle_lib.OracleLayer(h) for h in hosts]
    hip = _lib.hip()
    x0 = synth.hidden_states(S, H, seed=60)
    xb = moe.DeviceBuffer(x0.nbytes)
    xn_t = moe.DeviceBuffer(nl * x0.nbytes)
    idx_t = moe.DeviceBuffer(nl * S * 4 * 4)
    xb.upload(x0)
    assert hip.colizig_hip_chain_decode(1500, nl, xb.ptr, S, 1e-6, xn_t.ptr, idx_t.ptr, None, None) == 0
    assert hip.colizig_hip_sync() == 0
    xn = xn_t.download(np.empty((nl, S, H), np.float32))
    idx = idx_t.download(np.empty((nl, S, 4), np.uint32))
    for l in range(nl):
        for s in range(S):
            ri, _, _ = orcs[l].route(xn[l, s])
            assert np.array_equal(idx[l, s], ri), f"layer {l} token {s}"
        out_g = moe.Layer(1500 + l, moe.Dims(**hosts[l]["dims"]), True).forward(xn[l])[0]
        assert rel_l2(out_g, orcs[l].forward(xn[l])[0]) < RTOL_L2


def test_grouped_chain_shared_expert(gpu, oracle_lib):
    """x <- x + MoE(rms(x)) over 2 layers with a shared expert, S=32 tokens in
    the grouped regime: the RMS rows kernel also forms the shared-expert gate;
    the chained result matches the oracle layers applied to the GPU's own
    router inputs (routing bit-exact, outputs within the bar)."""
    say("grouped chain with shared expert S=32")
    H, S, nl = 512, 32, 2
    hosts = [synth.make_layer(H, 32, 4, 256, 512, True, seed=70 + l) for l in range(nl)]
    for l, h in enumerate(hosts):
        moe.register_layer(1900 + l, h)
    orcs = [oracle_lib.OracleLayer(h) for h in hosts]
    hip = _lib.hip()
    x0 = synth.hidden_states(S, H, seed=70)
    xb = moe.DeviceBuffer(x0.nbytes)
    xn_t = moe.DeviceBuffer(nl * x0.nbytes)
    idx_t = moe.DeviceBuffer(nl * S * 4 * 4)
    xb.upload(x0)
    assert hip.colizig_hip_chain_decode(1900, nl, xb.ptr, S, 1e-6, xn_t.ptr, idx_t.ptr, None, None) == 0
    assert hip.colizig_hip_sync() == 0
    xn = xn_t.download(np.empty((nl, S, H), np.float32))
    idx = idx_t.download(np.empty((nl, S, 4), np.uint32))
    x_gpu = xb.download(np.empty((S, H), np.float32))
    x_ref = x0.astype(np.float64)
    for l in range(nl):
        out, ri, _ = orcs[l].forward(xn[l])
        assert np.array_equal(idx[l], ri), f"layer {l}: routing differs"
        x_ref = x_ref + out
    err = rel_l2(x_gpu, x_ref.astype(np.float32))
    say(f"  rel L2 {err:.2e}")
    assert err < RTOL_L2


def test_prefill_qwen3_30b_shapes_zipf(gpu, oracle_lib):
    """One Qwen3-30B-A3B-shape layer (hidden 2048, 128 experts, top-8, inter
    768) at a 512-token prefill with Zipf(1.1) routing skew, GPU-generated
    weights read back for the oracle."""
    say("prefill c3 shapes S=512")
    H, E, K, I, S = 2048, 128, 8, 768, 512
    L = moe.Layer.load(1600, moe.dims(H, E, K, I), np.zeros((E, H), np.float32))
    L.synth(seed=4242)
    bias = synth.zipf_router_bias(E, 1.1, seed=3)
    L.set_router_bias(bias)
    host = dict(dims=dict(hidden=H, experts=E, topk=K, inter=I, shared_inter=0, norm_topk=1),
                router=L.read_router(), experts=[L.read_expert(e) for e in range(E)], shared=None,
                router_bias=bias)
    Lo = oracle_lib.OracleLayer(host)
    x = synth.hidden_states(S, H, seed=11)
    out, idx, gates = L.forward(x)
    counts = np.bincount(idx.ravel(), minlength=E)
    say(f"  hottest expert {counts.max()} slots, experts touched {int((counts > 0).sum())}")
    ro, ri, rg = Lo.forward(x)
    assert np.array_equal(idx, ri)
    assert np.array_equal(f32_bits(gates), f32_bits(rg))
    err = rel_l2(out, ro)
    say(f"  rel L2 {err:.2e}")
    assert err < RTOL_L2
