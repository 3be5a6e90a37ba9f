"""The decode chain x <- x + MoE(rms(x)) (qwen3moe/model.zig:228-232 with a
unit-weight rms, rmsnorm.zig:32-40) on the GPU against the oracle's own chain
run from the same x0: per layer the router input, the routing and the
residual stream.

Routing bits: both sides evaluate the same correctly rounded f32 exp; the bits
of the reference's @exp (Zig compiler-rt) and its @reduce lane order cannot be
observed here.  The near-tie census below records, for every routing decision
of the oracle, the gap in f32 ulps between consecutive values among the top
K+1; a gap of at least CENSUS_MIN_ULPS means an exp or a logit off by a few
ulps on either side cannot reorder the picks, so the indices do not depend on
those unobserved bits.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from colizig_amd import _lib, moe, synth
from tests.helpers import f32_bits, rel_l2

pytestmark = pytest.mark.gpu

RTOL_L2 = 1e-3       # MoE outputs / residual stream vs the CPU path
CENSUS_MIN_ULPS = 8  # required gap between consecutive top-(K+1) values


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def census_min_gap(v: np.ndarray, K: int) -> int:
    """Smallest gap, in f32 ulps, between consecutive values of the top K+1
    (value descending, lowest id first among equals) of the post-exp values v
    (all >= 0, so their bit patterns order like the values)."""
    E = v.size
    order = sorted(range(E), key=lambda e: (-float(v[e]), e))[:min(K + 1, E)]
    b = f32_bits(v[order]).astype(np.int64)
    return int(np.min(b[:-1] - b[1:]))


def chain_vs_oracle(oracle_lib, hosts, base, S, tokens, eps=1e-6, seed=0, label=""):
    """Runs the GPU chain and the oracle chain side by side from the same x0;
    returns (min census gap, max xn rel diff, max residual rel L2).  The
    device's routed-selection counters (bumpUsage, moe.zig:428-432) must
    equal the counts of the oracle chain's picks."""
    nl = len(hosts)
    H, K = hosts[0]["dims"]["hidden"], hosts[0]["dims"]["topk"]
    layers = [moe.register_layer(base + l, h) if "registered" not in h else h["registered"]
              for l, h in enumerate(hosts)]
    orcs = [oracle_lib.OracleLayer(h) for h in hosts]
    hip = _lib.hip()
    x0 = synth.hidden_states(S, H, seed=seed)
    xb = moe.DeviceBuffer(x0.nbytes)
    xn_t = moe.DeviceBuffer(nl * x0.nbytes)
    idx_t = moe.DeviceBuffer(nl * S * K * 4)
    g_t = moe.DeviceBuffer(nl * S * K * 4)
    xb.upload(x0)
    xo = x0.copy()
    E = hosts[0]["dims"]["experts"]
    assert hip.colizig_hip_usage_reset() == 0
    picks = np.zeros((nl, E), np.uint64)
    min_gap, worst_xn, worst_x = 1 << 30, 0.0, 0.0
    for tok in range(tokens):
        say(f"  {label} token {tok}")
        rc = hip.colizig_hip_chain_decode(base, nl, xb.ptr, S, eps, xn_t.ptr, idx_t.ptr, g_t.ptr, None)
        assert rc == 0, _lib.last_error()
        assert hip.colizig_hip_sync() == 0, _lib.last_error()
        xn_g = xn_t.download(np.empty((nl, S, H), np.float32))
        idx_g = idx_t.download(np.empty((nl, S, K), np.uint32))
        gates_g = g_t.download(np.empty((nl, S, K), np.float32))
        for l in range(nl):
            xn_o, idx_o, gates_o = orcs[l].chain(xo, eps)
            np.add.at(picks[l], idx_o.reshape(-1).astype(np.int64), 1)
            if tok == 0 and l == 0:  # the same x0 on both sides: the same router input, bit for bit
                assert np.array_equal(f32_bits(xn_g[0]), f32_bits(xn_o)), f"{label}: rms of x0"
            worst_xn = max(worst_xn, rel_l2(xn_g[l], xn_o))
            assert rel_l2(xn_g[l], xn_o) < RTOL_L2, f"{label} token {tok} layer {l}: router input"
            for s in range(S):
                # the GPU's routing of its own router input == the oracle's, bit for bit
                ri, rg, _ = orcs[l].route(xn_g[l, s])
                assert np.array_equal(idx_g[l, s], ri), f"{label} token {tok} layer {l} row {s}: routing"
                assert np.array_equal(f32_bits(gates_g[l, s]), f32_bits(rg)), f"{label} t{tok} l{l}: gates"
                # and the same experts as the oracle's own chain picks
                assert np.array_equal(idx_g[l, s], idx_o[s]), f"{label} token {tok} layer {l} row {s}: picks"
                _, _, v = orcs[l].route(xn_o[s])
                min_gap = min(min_gap, census_min_gap(v, K))
        x_g = xb.download(np.empty_like(x0))
        worst_x = max(worst_x, rel_l2(x_g, xo))
        assert rel_l2(x_g, xo) < RTOL_L2, f"{label} token {tok}: residual stream"
    usage = np.zeros((nl, E), np.uint64)
    assert hip.colizig_hip_usage_read(base, nl, E, usage.ctypes.data) == 0
    assert np.array_equal(usage, picks), f"{label}: routed-selection counters"
    assert int(usage.sum()) == tokens * nl * S * K
    assert min_gap >= CENSUS_MIN_ULPS, f"{label}: a routing decision within {min_gap} ulps of a tie"
    say(f"  {label}: census min gap {min_gap} ulps, xn rel diff <= {worst_xn:.2e}, x rel L2 <= {worst_x:.2e}")
    for b in (xb, xn_t, idx_t, g_t):
        b.free()
    return min_gap, worst_xn, worst_x


@pytest.mark.parametrize("S", [1, 2, 20])
def test_chain_vs_oracle_chain_tiny(gpu, oracle_lib, S):
    """Config-1 shapes (hidden 512, 16 experts, top-4, inter 256), 3 chained
    layers, 3 steps; S = 1, 2 (decode kernels) and 20 (grouped regime)."""
    say(f"chain vs oracle chain, tiny S={S}")
    hosts = [synth.make_layer(512, 16, 4, 256, 0, True, seed=61 + l) for l in range(3)]
    chain_vs_oracle(oracle_lib, hosts, 1100 + 10 * S, S, tokens=3, seed=S, label=f"tiny S={S}")


def test_chain_vs_oracle_chain_qwen3_30b(gpu, oracle_lib):
    """Qwen3-30B-A3B shapes (hidden 2048, 128 experts, top-8, inter 768) on
    GPU-generated weights read back for the oracle: 3 chained layers, 4 steps
    at batch 1, the headline workload's own chain."""
    say("chain vs oracle chain, qwen3-30b shapes")
    H, E, K, I = 2048, 128, 8, 768
    d = moe.dims(H, E, K, I)
    hosts = []
    for l in range(3):
        L = moe.Layer.load(1200 + l, d, np.zeros((E, H), np.float32))
        L.synth(seed=4321 + l)
        hosts.append(dict(dims=dict(hidden=H, experts=E, topk=K, inter=I, shared_inter=0, norm_topk=1),
                          router=L.read_router(), experts=[L.read_expert(e) for e in range(E)], shared=None,
                          registered=L))
    chain_vs_oracle(oracle_lib, hosts, 1200, 1, tokens=4, seed=3, label="qwen3-30b")


def test_graph_refuses_changed_layers(gpu):
    """A captured chain graph holds the layers' device pointers: after a layer
    is re-registered, or its router bias is removed, the graph is refused
    (-1) and never launched."""
    say("graph refuses changed layers")
    hip = _lib.hip()
    hosts = [synth.make_layer(512, 16, 4, 256, 0, True, seed=71 + l) for l in range(2)]
    for l, h in enumerate(hosts):
        moe.register_layer(1300 + l, h)
    Lb = moe.Layer(1301, moe.Dims(**hosts[1]["dims"]), True)
    Lb.set_router_bias(np.zeros(16, np.float32))
    x0 = synth.hidden_states(1, 512, seed=7)
    xb = moe.DeviceBuffer(x0.nbytes)
    xb.upload(x0)
    gh = hip.colizig_hip_chain_graph_create(1300, 2, xb.ptr, 1, 1e-6)
    assert gh > 0, _lib.last_error()
    assert hip.colizig_hip_graph_launch(gh, None) == 0
    assert hip.colizig_hip_sync() == 0
    Lb.set_router_bias(None)  # frees the bias buffer the graph captured
    assert hip.colizig_hip_graph_launch(gh, None) == -1
    assert "changed since capture" in _lib.last_error()
    hip.colizig_hip_graph_destroy(gh)
    gh = hip.colizig_hip_chain_graph_create(1300, 2, xb.ptr, 1, 1e-6)
    assert gh > 0 and hip.colizig_hip_graph_launch(gh, None) == 0
    assert hip.colizig_hip_sync() == 0
    moe.register_layer(1300, hosts[0])  # re-registration frees the layer's weights
    assert hip.colizig_hip_graph_launch(gh, None) == -1
    hip.colizig_hip_graph_destroy(gh)
    xb.free()


def test_matmul_fp8_key_holding_other_matrix(gpu, oracle_lib):
    """colizig_cuda_matmul_fp8 with a key whose cache slot holds BF16 rows or
    an FP8 matrix of another shape: the resident slot is not used as is; the
    result matches the oracle."""
    say("keyed matmul over a mismatched slot")
    rng = np.random.default_rng(17)
    moe.set_vram_budget(1 << 30)
    key = moe.Fp8Matrix.expert_key(40, 3, 1)
    moe.matrix_load_bf16(key, rng.integers(0, 1 << 16, size=(64, 256), dtype=np.uint16))
    for (O, I) in [(128, 256), (300, 512), (64, 256)]:
        x = rng.normal(size=(2, I)).astype(np.float32)
        w, s = synth.block_quantize(rng.normal(0, 0.02, size=(O, I)).astype(np.float32))
        y = moe.matmul_fp8(x, w, s, 2, I, O, key=key)
        assert rel_l2(y, oracle_lib.matmul_fp8(x, w, s, 2, I, O)) < 1e-5, (O, I)
    moe.set_vram_budget(0)


def _run_chain(hip, base, nl, x0, K, eps=1e-6):
    H = x0.shape[-1]
    xb = moe.DeviceBuffer(x0.nbytes)
    xn_t = moe.DeviceBuffer(nl * x0.nbytes)
    idx_t = moe.DeviceBuffer(nl * K * 4)
    g_t = moe.DeviceBuffer(nl * K * 4)
    xb.upload(x0)
    assert hip.colizig_hip_chain_decode(base, nl, xb.ptr, 1, eps, xn_t.ptr, idx_t.ptr, g_t.ptr, None) == 0
    assert hip.colizig_hip_sync() == 0, _lib.last_error()
    out = (xb.download(np.empty_like(x0)), xn_t.download(np.empty((nl, H), np.float32)),
           idx_t.download(np.empty((nl, K), np.uint32)), g_t.download(np.empty((nl, K), np.float32)))
    for b in (xb, xn_t, idx_t, g_t):
        b.free()
    return out


@pytest.mark.parametrize("shape", ["tiny", "qwen3-30b"])
def test_one_launch_decode_matches_three_kernel_decode(gpu, oracle_lib, shape):
    """The one-launch-per-layer batch-1 decode is the path the chain takes at
    these shapes; its router inputs, routing and residual stream equal the
    three-kernel decode's (routing and gates bit for bit, x within 1e-5)."""
    say(f"one-launch vs three-kernel decode, {shape}")
    hip = _lib.hip()
    if shape == "tiny":
        H, E, K, I, nl, base = 512, 16, 4, 256, 4, 1400
        for l in range(nl):
            moe.register_layer(base + l, synth.make_layer(H, E, K, I, 0, True, seed=81 + l))
    else:
        H, E, K, I, nl, base = 2048, 128, 8, 768, 6, 1500
        for l in range(nl):
            moe.Layer.load(base + l, moe.dims(H, E, K, I), np.zeros((E, H), np.float32)).synth(seed=99 + l)
    assert hip.colizig_hip_fused_decode_active(base, nl, 1) == 1
    x0 = synth.hidden_states(1, H, seed=13)
    xf, xnf, idf, gf = _run_chain(hip, base, nl, x0, K)
    prev = hip.colizig_hip_set_fused_decode(0)
    try:
        assert hip.colizig_hip_fused_decode_active(base, nl, 1) == 0
        xc, xnc, idc, gc = _run_chain(hip, base, nl, x0, K)
    finally:
        hip.colizig_hip_set_fused_decode(prev)
    # layer 0 sees the same router input on both paths: the same routing, bit for bit; later
    # layers' inputs differ by the rounding of the two paths' down/combine sums
    assert np.array_equal(f32_bits(xnf[0]), f32_bits(xnc[0]))
    assert np.array_equal(f32_bits(gf[0]), f32_bits(gc[0]))
    assert np.array_equal(idf, idc)
    assert np.max(np.abs(gf - gc) / gc) < 1e-5
    assert rel_l2(xnf, xnc) < 1e-5
    assert rel_l2(xf, xc) < 1e-5, rel_l2(xf, xc)
    say(f"  x rel L2 one-launch vs three-kernel {rel_l2(xf, xc):.2e}")


def test_one_launch_decode_graph_replay(gpu):
    """The one-launch decode captured in a graph and replayed 4 times gives
    the eager chain's bits after every replay (each replay advances the run
    counter that tags the exchanged values)."""
    say("one-launch decode graph replay")
    hip = _lib.hip()
    H, E, K, I, nl, base = 2048, 128, 8, 768, 3, 1600
    for l in range(nl):
        moe.Layer.load(base + l, moe.dims(H, E, K, I), np.zeros((E, H), np.float32)).synth(seed=123 + l)
    assert hip.colizig_hip_fused_decode_active(base, nl, 1) == 1
    x0 = synth.hidden_states(1, H, seed=21)
    xe, xg = moe.DeviceBuffer(x0.nbytes), moe.DeviceBuffer(x0.nbytes)
    xe.upload(x0)
    xg.upload(x0)
    gh = hip.colizig_hip_chain_graph_create(base, nl, xg.ptr, 1, 1e-6)
    assert gh > 0, _lib.last_error()
    for rep in range(4):
        assert hip.colizig_hip_chain_decode(base, nl, xe.ptr, 1, 1e-6, None, None, None, None) == 0
        assert hip.colizig_hip_graph_launch(gh, None) == 0
        assert hip.colizig_hip_sync() == 0, _lib.last_error()
        a = xe.download(np.empty_like(x0))
        b = xg.download(np.empty_like(x0))
        assert np.array_equal(f32_bits(a), f32_bits(b)), f"replay {rep}"
    hip.colizig_hip_graph_destroy(gh)
    xe.free()
    xg.free()


@pytest.mark.parametrize("shape", ["tiny", "qwen3-30b"])
def test_one_launch_decode_predicted_experts(gpu, oracle_lib, shape):
    """The one-launch decode requests each layer's predicted experts (the
    previous layer's kernel takes the next layer's top-k on its own router
    input) before its routing.  With the prediction off, as computed, spoiled
    (no slot keeps its prediction: every slot loads after the routing) and
    half spoiled (slot 0 never keeps it): routing and gates equal bit for
    bit, router inputs and the residual stream within 1e-5 relative L2 (only
    the order of the down sums changes).  The hit counters count one
    prediction per slot of every layer after the first; none is kept when
    spoiled, slot 0's never when half spoiled."""
    say(f"predicted experts, {shape}")
    hip = _lib.hip()
    if shape == "tiny":
        H, E, K, I, nl, base = 512, 16, 4, 256, 5, 1700
        for l in range(nl):
            moe.register_layer(base + l, synth.make_layer(H, E, K, I, 0, True, seed=181 + l))
    else:
        H, E, K, I, nl, base = 2048, 128, 8, 768, 6, 1800
        for l in range(nl):
            moe.Layer.load(base + l, moe.dims(H, E, K, I), np.zeros((E, H), np.float32)).synth(seed=199 + l)
    assert hip.colizig_hip_fused_decode_active(base, nl, 1) == 1
    x0 = synth.hidden_states(1, H, seed=17)
    st = np.zeros(2, np.uint64)
    runs = {}
    prev = hip.colizig_hip_set_fused_predict(1)
    try:
        for mode in (0, 1, 2, 3):
            assert hip.colizig_hip_set_fused_predict(mode) >= 0
            hip.colizig_hip_fused_predict_stats(st.ctypes.data)  # zero the counters
            runs[mode] = _run_chain(hip, base, nl, x0, K)
            assert hip.colizig_hip_fused_predict_stats(st.ctypes.data) == 0
            if mode == 0:
                assert st[0] == 0
            else:
                assert st[0] == (nl - 1) * K, st
            if mode == 2:
                assert st[1] == 0, st
            if mode == 3:
                assert st[1] <= (nl - 1) * (K - 1), st
            say(f"  mode {mode}: predictions {int(st[0])}, picked {int(st[1])}")
        assert hip.colizig_hip_set_fused_predict(4) == -1
    finally:
        hip.colizig_hip_set_fused_predict(prev)
    x_ref, xn_ref, id_ref, g_ref = runs[0]
    for mode in (1, 2, 3):
        x, xn, idx, gates = runs[mode]
        assert np.array_equal(idx, id_ref), f"mode {mode}: routing"
        assert np.array_equal(f32_bits(gates[0]), f32_bits(g_ref[0])), f"mode {mode}: layer-0 gates"
        assert np.max(np.abs(gates - g_ref) / g_ref) < 1e-5
        assert rel_l2(xn, xn_ref) < 1e-5, f"mode {mode}: router inputs"
        assert rel_l2(x, x_ref) < 1e-5, f"mode {mode}: x rel L2 {rel_l2(x, x_ref):.2e}"
    say(f"  x rel L2 vs no prediction: " + ", ".join(f"{m}: {rel_l2(runs[m][0], x_ref):.1e}" for m in (1, 2, 3)))


def test_one_launch_decode_ties_and_nan_routers(gpu, oracle_lib):
    """Predicted experts where the routing is least regular: a layer whose
    router has four identical rows (exact ties: the lowest id wins) and a
    layer whose router rows are NaN but for experts 0 and 1 (two valid
    experts for top-4: the scan's remaining picks are expert 0, twice, and so
    are the predicted ones).  With the prediction on, off, spoiled and half
    spoiled, and on the three-kernel decode: the same routing and gates bit
    for bit, and every layer's routing equals the oracle's on the GPU's own
    router input."""
    say("one-launch decode: ties and NaN router rows")
    hip = _lib.hip()
    H, E, K, I, nl, base = 512, 16, 4, 256, 4, 1900
    hosts = [synth.make_layer(H, E, K, I, 0, True, seed=211 + l) for l in range(nl)]
    r1 = hosts[1]["router"].copy()
    r1[3] = r1[4] = r1[5] = r1[2]
    hosts[1]["router"] = r1
    r2 = hosts[2]["router"].copy()
    r2[2:] = np.nan
    hosts[2]["router"] = r2
    for l in range(nl):
        moe.register_layer(base + l, hosts[l])
    assert hip.colizig_hip_fused_decode_active(base, nl, 1) == 1
    orcs = [oracle_lib.OracleLayer(h) for h in hosts]
    x0 = synth.hidden_states(1, H, seed=23)
    runs = {}
    prev = hip.colizig_hip_set_fused_predict(1)
    try:
        for mode in (1, 0, 2, 3):
            hip.colizig_hip_set_fused_predict(mode)
            runs[mode] = _run_chain(hip, base, nl, x0, K)
    finally:
        hip.colizig_hip_set_fused_predict(prev)
    fprev = hip.colizig_hip_set_fused_decode(0)
    try:
        runs["three"] = _run_chain(hip, base, nl, x0, K)
    finally:
        hip.colizig_hip_set_fused_decode(fprev)
    x1, xn1, id1, g1 = runs[1]
    assert list(id1[2][2:]) == [0, 0], id1[2]  # two valid experts: expert 0 fills the rest
    for l in range(nl):
        ri, rg, _ = orcs[l].route(xn1[l])
        assert np.array_equal(id1[l], ri), f"layer {l}: routing vs the oracle's"
        assert np.array_equal(f32_bits(g1[l]), f32_bits(rg)), f"layer {l}: gates vs the oracle's"
    for key, (x, xn, idx, gates) in runs.items():
        assert np.array_equal(idx, id1), f"{key}: routing"
        assert np.array_equal(f32_bits(gates[0]), f32_bits(g1[0])), f"{key}: layer-0 gates"
        assert np.all(np.isfinite(x)), f"{key}: x"
        assert rel_l2(x, x1) < 1e-5, f"{key}: x rel L2 {rel_l2(x, x1):.2e}"
    say(f"  picks of the NaN layer {id1[2].tolist()}; tied layer {id1[1].tolist()}")
