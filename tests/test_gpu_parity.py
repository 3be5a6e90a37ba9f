"""Parity of the HIP library (through its C-ABI) with the oracle on the same
seeded inputs.  Bar: dequantised weights, routing indices and gates bit-exact;
MoE outputs within 1e-3 relative L2 (fp32 accumulation)."""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest

from colizig_amd import _lib, moe, synth
from tests.helpers import f32_bits, rel_l2, tiny_qwen3_layer

pytestmark = pytest.mark.gpu

RTOL_L2 = 1e-3  # MoE outputs vs the CPU path


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def bits_equal_nan_aware(a, b) -> bool:
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(f32_bits(a[~na]), f32_bits(b[~nb])))


def test_device(gpu):
    say(f"device: {gpu}")


# ---------------------------------------------------------------- dequant ----
@pytest.mark.parametrize("rows,cols", [(3, 256), (130, 260), (5, 205), (129, 2048)])
def test_dequant_bit_exact(gpu, oracle_lib, rows, cols):
    """e4m3(b)*scale on the GPU == the reference's dequantRow (fp8.zig:123-130)
    bit for bit, every byte value, several 128-blocks."""
    say(f"dequant {rows}x{cols}")
    rng = np.random.default_rng(rows * 1000 + cols)
    w = (np.arange(rows * cols) % 256).astype(np.uint8).reshape(rows, cols)
    w[1:] = rng.integers(0, 256, size=(rows - 1, cols), dtype=np.uint8)
    s = rng.uniform(1e-5, 3.0, size=(moe.nblk(rows), moe.nblk(cols))).astype(np.float32)
    s.flat[0] = 1.0
    got = moe.dequant_fp8(w, s)
    want = oracle_lib.dequant_matrix(w, s)
    assert bits_equal_nan_aware(got, want)


# -------------------------------------------------------------------- exp ----
def test_expf_device_bitwise(gpu, oracle_lib):
    """The router's exp on the GPU equals the oracle's f32 exp bit for bit."""
    say("expf device")
    rng = np.random.default_rng(7)
    xs = [np.linspace(-30.0, 0.0, 1 << 20, dtype=np.float32),
          rng.uniform(-104, 89, size=1 << 20).astype(np.float32),
          np.arange(0, 1 << 32, 4099, dtype=np.uint64).astype(np.uint32).view(np.float32)]
    x = np.concatenate(xs)
    x = x[~np.isnan(x)]
    out = np.empty_like(x)
    rc = _lib.hip().colizig_hip_expf_dev(_p(x), _p(out), x.size)
    assert rc == 0, _lib.last_error()
    assert bits_equal_nan_aware(out, oracle_lib.expf(x))


# ------------------------------------------------------- per-matmul ABI ----
def test_matmul_fp8_reference_shapes(gpu, oracle_lib):
    """fp8.zig:273-353 shapes through colizig_cuda_matmul_fp8."""
    say("matmul_fp8 reference shapes")
    rng = np.random.default_rng(0xF8)
    S, I, O = 3, 200, 5
    x = (rng.random((S, I)) * 2 - 1).astype(np.float32)
    w = np.array([0x38, 0x34, 0x30, 0x3C, 0xB8, 0xB4, 0x40, 0x2C], np.uint8)[rng.integers(0, 8, size=(O, I))]
    s = (0.5 + rng.random((1, 2))).astype(np.float32)
    y = moe.matmul_fp8(x, w, s, S, I, O)
    assert np.max(np.abs(y - oracle_lib.matmul_fp8(x, w, s, S, I, O))) < 1e-4
    rng = np.random.default_rng(0x5115)
    I, O = 384, 6
    x = (rng.random(I) * 2 - 1).astype(np.float32)
    w = rng.integers(0, 256, size=(O, I), dtype=np.uint8)
    w[(w == 0x7F) | (w == 0xFF)] = 0
    s = (0.25 + rng.random((1, 3))).astype(np.float32)
    y = moe.matmul_fp8(x, w, s, 1, I, O)[0]
    ref = oracle_lib.matmul_fp8(x, w, s, 1, I, O)[0]
    assert np.all(np.abs(y - ref) <= 1e-4 * np.abs(ref) + 1e-6)
    # an expert-sized GEMV (c2 gate: 768 x 2048) and a down (2048 x 768)
    for (O, I) in [(768, 2048), (2048, 768)]:
        x = rng.normal(size=(1, I)).astype(np.float32)
        w, s = synth.block_quantize(rng.normal(0, 0.02, size=(O, I)).astype(np.float32))
        y = moe.matmul_fp8(x, w, s, 1, I, O)
        assert rel_l2(y, oracle_lib.matmul_fp8(x, w, s, 1, I, O)) < 1e-5


def test_matmul_keyed_cache(gpu):
    """colizig_cuda.cu:228-284 cache semantics: budget 0 uploads every call;
    keyed calls hit after the first; stats count them."""
    say("keyed cache")
    rng = np.random.default_rng(1)
    S, I, O = 1, 256, 128
    x = rng.normal(size=(S, I)).astype(np.float32)
    w, s = synth.block_quantize(rng.normal(0, 0.02, size=(O, I)).astype(np.float32))
    moe.set_vram_budget(0)
    st0 = moe.stats()
    y0 = moe.matmul_fp8(x, w, s, S, I, O, key=0)
    moe.matmul_fp8(x, w, s, S, I, O, key=moe.Fp8Matrix.expert_key(0, 1, 0))
    st1 = moe.stats()
    assert st1["hits"] == st0["hits"] and st1["misses"] == st0["misses"]
    moe.set_vram_budget(1 << 30)
    k = moe.Fp8Matrix.expert_key(3, 7, 2)
    y1 = moe.matmul_fp8(x, w, s, S, I, O, key=k)
    y2 = moe.matmul_fp8(x, w, s, S, I, O, key=k)
    st2 = moe.stats()
    assert st2["misses"] == st1["misses"] + 1 and st2["hits"] == st1["hits"] + 1
    assert st2["resident"] >= 1
    assert np.array_equal(f32_bits(y0), f32_bits(y1)) and np.array_equal(f32_bits(y1), f32_bits(y2))
    moe.set_vram_budget(0)


# ---------------------------------------------------------------- MoE layer --
def _check_forward(L_gpu, L_orc, x, what):
    out, idx, gates = L_gpu.forward(x)
    ro, ri, rg = L_orc.forward(x)
    assert np.array_equal(idx, ri), f"{what}: routing differs"
    assert np.array_equal(f32_bits(gates), f32_bits(rg)), f"{what}: gates differ"
    err = rel_l2(out, ro)
    assert err < RTOL_L2, f"{what}: rel L2 {err}"
    return err


def test_c1_tiny_layer_64_decode_steps(gpu, oracle_lib):
    """Tiny layer (hidden 512, 16 experts, top-4, inter 256), 64 decode
    steps from seed 0: every token's experts and gates bit-exact."""
    say("c1 64 decode steps")
    host = synth.make_layer(512, 16, 4, 256, 0, True, seed=0)
    Lg = moe.register_layer(100, host)
    Lo = oracle_lib.OracleLayer(host)
    x = synth.hidden_states(64, 512, seed=0)
    worst = 0.0
    for t in range(64):
        worst = max(worst, _check_forward(Lg, Lo, x[t:t + 1], f"token {t}"))
    say(f"  worst rel L2 {worst:.3e}")


def test_tiny_qwen3_fixture_generic_path(gpu, oracle_lib):
    """The reference fixture's shapes (hidden 32, inter 16) run the generic
    kernels; routing equals the oracle and the f64 golden."""
    say("tiny-qwen3 fixture")
    for li in range(4):
        host, gold = tiny_qwen3_layer(li)
        Lg = moe.register_layer(200 + li, host)
        Lo = oracle_lib.OracleLayer(host)
        out, idx, _ = Lg.forward(gold["x"])
        assert np.array_equal(idx, gold["idx"])
        assert rel_l2(out, gold["out"]) < RTOL_L2
        _check_forward(Lg, Lo, gold["x"], f"layer {li}")
        for t in range(4):
            _check_forward(Lg, Lo, gold["x"][t:t + 1], f"layer {li} token {t}")


@pytest.mark.parametrize("S", [2, 5, 32])
def test_batch_decode(gpu, oracle_lib, S):
    """S tokens at once vs the reference's grouped path (moe.zig:597-665)."""
    say(f"batch decode S={S}")
    host = synth.make_layer(512, 16, 4, 256, 0, True, seed=S)
    Lg = moe.register_layer(300 + S, host)
    Lo = oracle_lib.OracleLayer(host)
    _check_forward(Lg, Lo, synth.hidden_states(S, 512, seed=S), f"S={S}")


@pytest.mark.parametrize("S,SI", [(8, 0), (3, 2048)])
def test_batch_decode_two_rows_per_wave(gpu, oracle_lib, S, SI):
    """Hidden 2048 with enough gate/up rows that the gate/up kernel takes two
    rows of each matrix per wave (>= 1024 workgroups of 8 rows)."""
    say(f"batch decode H=2048 S={S} SI={SI}")
    host = synth.make_layer(2048, 16, 4, 256, SI, True, seed=40 + S)
    Lg = moe.register_layer(340 + S, host)
    Lo = oracle_lib.OracleLayer(host)
    _check_forward(Lg, Lo, synth.hidden_states(S, 2048, seed=S), f"H=2048 S={S}")


@pytest.mark.parametrize("SI,S", [(512, 1), (512, 3), (384, 2)])
def test_shared_expert(gpu, oracle_lib, SI, S):
    """Qwen4-Exp style: routed experts plus an always-on sigmoid-gated shared
    expert (moe.zig:467-479).  SI=384 takes the generic down kernel."""
    say(f"shared SI={SI} S={S}")
    host = synth.make_layer(512, 32, 4, 256, SI, True, seed=SI + S)
    Lg = moe.register_layer(400 + SI + S, host)
    Lo = oracle_lib.OracleLayer(host)
    _check_forward(Lg, Lo, synth.hidden_states(S, 512, seed=SI), f"SI={SI}")


def test_norm_topk_false(gpu, oracle_lib):
    say("norm_topk false")
    host = synth.make_layer(256, 64, 6, 256, 0, False, seed=9)
    Lg = moe.register_layer(500, host)
    Lo = oracle_lib.OracleLayer(host)
    x = synth.hidden_states(4, 256, seed=9)
    for t in range(4):
        _check_forward(Lg, Lo, x[t:t + 1], f"token {t}")


def test_deterministic(gpu):
    say("determinism")
    host = synth.make_layer(512, 16, 4, 256, 0, True, seed=11)
    Lg = moe.register_layer(600, host)
    x = synth.hidden_states(3, 512, seed=11)
    a = Lg.forward(x)[0]
    b = Lg.forward(x)[0]
    assert np.array_equal(f32_bits(a), f32_bits(b))


def test_misaligned_activations_rejected(gpu):
    """Device activations move as float4: a pointer off 16-byte alignment is
    refused (-1, with a message) before anything is launched."""
    say("misaligned activation pointers")
    host = synth.make_layer(512, 16, 4, 256, 0, True, seed=12)
    moe.register_layer(650, host)
    hip = _lib.hip()
    xb = moe.DeviceBuffer(2 * 512 * 4 + 64)
    ob = moe.DeviceBuffer(2 * 512 * 4 + 64)
    assert hip.colizig_hip_moe_forward_dev(650, xb.ptr + 4, 2, ob.ptr, None, None, None) == -1
    assert "16-byte" in _lib.last_error()
    assert hip.colizig_hip_moe_forward_dev(650, xb.ptr, 2, ob.ptr + 8, None, None, None) == -1
    assert hip.colizig_hip_chain_decode(650, 1, xb.ptr + 4, 1, 1e-6, None, None, None, None) == -1
    assert hip.colizig_hip_chain_graph_create(650, 1, xb.ptr + 4, 1, 1e-6) < 0
    # aligned: accepted
    xb.upload(synth.hidden_states(2, 512, seed=12))
    assert hip.colizig_hip_moe_forward_dev(650, xb.ptr, 2, ob.ptr, None, None, None) == 0
    assert hip.colizig_hip_sync() == 0


# ------------------------------------------------------------- layer chain --
def _chain_case(oracle_lib, dims, nl, base, seed, S=1, tokens=3):
    H, E, K, I, SI = dims
    hosts = [synth.make_layer(H, E, K, I, SI, True, seed=seed + l) for l in range(nl)]
    for l, h in enumerate(hosts):
        moe.register_layer(base + l, h)
    orcs = [oracle_lib.OracleLayer(h) for h in hosts]
    hip = _lib.hip()
    x0 = synth.hidden_states(S, H, seed=seed)
    xb = moe.DeviceBuffer(x0.nbytes)
    xn_t = moe.DeviceBuffer(nl * x0.nbytes)
    idx_t = moe.DeviceBuffer(nl * S * K * 4)
    g_t = moe.DeviceBuffer(nl * S * K * 4)
    xb.upload(x0)
    eps = 1e-6
    x = x0.copy()
    for tok in range(tokens):
        rc = hip.colizig_hip_chain_decode(base, nl, xb.ptr, S, eps, xn_t.ptr, idx_t.ptr, g_t.ptr, None)
        assert rc == 0, _lib.last_error()
        assert hip.colizig_hip_sync() == 0
        xn = xn_t.download(np.empty((nl, S, H), np.float32))
        idx = idx_t.download(np.empty((nl, S, K), np.uint32))
        gates = g_t.download(np.empty((nl, S, K), np.float32))
        for l in range(nl):
            for s in range(S):
                ri, rg, _ = orcs[l].route(xn[l, s])
                assert np.array_equal(idx[l, s], ri), f"token {tok} layer {l} row {s}: routing"
                assert np.array_equal(f32_bits(gates[l, s]), f32_bits(rg)), f"token {tok} layer {l}: gates"
            # the layer's MoE output on the GPU's own router input
            Lg = moe.Layer(base + l, moe.Dims(**hosts[l]["dims"]), True)
            out_g = Lg.forward(xn[l])[0]
            out_o = orcs[l].forward(xn[l])[0]
            assert rel_l2(out_g, out_o) < RTOL_L2
    return base, nl, xb, x0, S


def test_chain_routing_bit_exact_per_layer(gpu, oracle_lib):
    """x <- x + MoE(rms(x)) over 3 layers: each layer's routing (taken on the
    GPU's own router input) bit-exact vs the oracle; outputs within 1e-3."""
    say("chain per-layer parity")
    _chain_case(oracle_lib, (512, 16, 4, 256, 0), 3, 700, seed=21)


def test_chain_graph_replay_matches_eager(gpu, oracle_lib):
    """A captured chain replayed 3 times gives the eager chain's bits after
    every replay (no memset nodes: counters are reset by the kernels)."""
    say("chain graph replay")
    H, nl, S = 512, 3, 2
    hosts = [synth.make_layer(H, 16, 4, 256, 0, True, seed=40 + l) for l in range(nl)]
    for l, h in enumerate(hosts):
        moe.register_layer(800 + l, h)
    hip = _lib.hip()
    x0 = synth.hidden_states(S, H, seed=40)
    xe = moe.DeviceBuffer(x0.nbytes)
    xg = moe.DeviceBuffer(x0.nbytes)
    xe.upload(x0)
    xg.upload(x0)
    gh = hip.colizig_hip_chain_graph_create(800, nl, xg.ptr, S, 1e-6)
    assert gh > 0, _lib.last_error()
    for rep in range(3):
        assert hip.colizig_hip_chain_decode(800, nl, xe.ptr, S, 1e-6, None, None, None, None) == 0
        assert hip.colizig_hip_graph_launch(gh, None) == 0
        assert hip.colizig_hip_sync() == 0
        a = xe.download(np.empty_like(x0))
        b = xg.download(np.empty_like(x0))
        assert np.array_equal(f32_bits(a), f32_bits(b)), f"replay {rep}"
    hip.colizig_hip_graph_destroy(gh)


def test_qwen3_30b_shape_two_layers(gpu, oracle_lib):
    """Full Qwen3-30B-A3B MoE shapes (hidden 2048, 128 experts, top-8, inter
    768) on GPU-generated weights read back for the oracle: 2 chained layers,
    4 tokens, routing bit-exact per layer, outputs within 1e-3."""
    say("c2 shapes, 2 layers")
    H, E, K, I = 2048, 128, 8, 768
    d = moe.dims(H, E, K, I)
    hip = _lib.hip()
    layers = []
    for l in range(2):
        L = moe.Layer.load(900 + l, d, np.zeros((E, H), np.float32))
        L.synth(seed=1234 + l)
        layers.append(L)
    hosts = []
    for L in layers:
        ex = [L.read_expert(e) for e in range(E)]
        hosts.append(dict(dims=dict(hidden=H, experts=E, topk=K, inter=I, shared_inter=0, norm_topk=1),
                          router=L.read_router(), experts=ex, shared=None))
    orcs = [oracle_lib.OracleLayer(h) for h in hosts]
    x0 = synth.hidden_states(1, H, seed=5)
    xb = moe.DeviceBuffer(x0.nbytes)
    xn_t = moe.DeviceBuffer(2 * x0.nbytes)
    idx_t = moe.DeviceBuffer(2 * K * 4)
    xb.upload(x0)
    for tok in range(4):
        assert hip.colizig_hip_chain_decode(900, 2, xb.ptr, 1, 1e-6, xn_t.ptr, idx_t.ptr, None, None) == 0
        assert hip.colizig_hip_sync() == 0
        xn = xn_t.download(np.empty((2, 1, H), np.float32))
        idx = idx_t.download(np.empty((2, 1, K), np.uint32))
        for l in range(2):
            ri, rg, _ = orcs[l].route(xn[l, 0])
            assert np.array_equal(idx[l, 0], ri), f"token {tok} layer {l}"
            out_g = layers[l].forward(xn[l])[0]
            out_o = orcs[l].forward(xn[l])[0]
            assert rel_l2(out_g, out_o) < RTOL_L2


@pytest.mark.parametrize("S", [1, 20])
def test_routing_exact_ties_pick_lowest_id(gpu, oracle_lib, S):
    """Router rows duplicated so several experts get bit-identical logits:
    the scan's strict '>' keeps the lowest id first (moe.zig:447-460), in the
    decode (S=1) and grouped (S=20) regimes."""
    say(f"exact ties S={S}")
    host = synth.make_layer(512, 64, 8, 256, 0, True, seed=123)
    r = host["router"]
    for a, b in [(3, 40), (7, 8), (8, 63), (20, 21), (21, 22)]:
        r[b] = r[a]
    host["router"] = r
    Lg = moe.register_layer(650 + S, host)
    Lo = oracle_lib.OracleLayer(host)
    x = synth.hidden_states(S, 512, seed=5)
    _check_forward(Lg, Lo, x, f"ties S={S}")
    # the tie groups really occur in the selected sets
    _, idx, _ = Lo.forward(x)
    assert any(len({3, 40} & set(row)) == 2 or len({7, 8, 63} & set(row)) >= 2 or len({20, 21, 22} & set(row)) >= 2
               for row in idx.tolist()) or S == 1


@pytest.mark.parametrize("S", [1, 32])
def test_qwen4_exp_shape_layer(gpu, oracle_lib, S):
    """Qwen4-Exp-style layer at full size: hidden 4096, 512 experts, top-10,
    moe_intermediate 512, one sigmoid-gated shared expert of 4096 (FP8), at
    batch 1 (decode kernels) and batch 32 (grouped regime); GPU-generated
    weights read back for the oracle."""
    say(f"qwen4-exp shapes S={S}")
    H, E, K, I, SI = 4096, 512, 10, 512, 4096
    L = moe.Layer.load(950, moe.dims(H, E, K, I, SI), np.zeros((E, H), np.float32))
    L.synth(seed=777)
    host = dict(dims=dict(hidden=H, experts=E, topk=K, inter=I, shared_inter=SI, norm_topk=1),
                router=L.read_router(), experts=[L.read_expert(e) for e in range(E)], shared=L.read_shared())
    Lo = oracle_lib.OracleLayer(host)
    err = _check_forward(L, Lo, synth.hidden_states(S, H, seed=S + 1), f"qwen4 S={S}")
    say(f"  rel L2 {err:.2e}")
