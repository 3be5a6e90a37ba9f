"""Pins the oracle (oracle/cz_oracle.c) against the reference's own golden
vectors and known-answer tests, library routines and what the mathematics
fixes.  CPU only."""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from tests.helpers import deq_f64, e4m3_f64, f32_bits, moe_f64, rel_l2, tiny_qwen3_layer

# fp8.zig:263-264 demo bytes and their exact values
DEMO_BYTES = [0x38, 0x34, 0x30, 0x3C, 0xB8, 0xB4, 0x40, 0x2C]
DEMO_VALUES = [1.0, 0.75, 0.5, 1.5, -1.0, -0.75, 2.0, 0.375]


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------- E4M3 ----
def test_e4m3_demo_bytes(oracle_lib):
    """fp8.zig:266-271"""
    lut = oracle_lib.lut()
    for b, v in zip(DEMO_BYTES, DEMO_VALUES):
        assert lut[b] == np.float32(v)
        assert oracle_lib.lib().czo_e4m3_decode(b) == np.float32(v)
    assert lut[0] == 0.0


def test_e4m3_lut_closed_form_all_bytes(oracle_lib):
    lut = oracle_lib.lut()
    ref = e4m3_f64(np.arange(256))
    for b in range(256):
        if np.isnan(ref[b]):
            assert np.isnan(lut[b]), b
        else:
            assert lut[b] == np.float32(ref[b]), b  # exact: every E4M3 value is an f32
    assert np.isnan(lut[0x7F]) and np.isnan(lut[0xFF])
    assert lut[0x7E] == 448.0 and lut[0x01] == 2.0 ** -9


def test_e4m3_lut_matches_torch(oracle_lib):
    torch = pytest.importorskip("torch")
    lut = oracle_lib.lut()
    t = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    for b in range(256):
        if np.isnan(t[b]):
            assert np.isnan(lut[b])
        else:
            assert f32_bits(lut[b]) == f32_bits(t[b]), b


def test_dequant_row_bit_identical_to_lut(oracle_lib):
    """fp8.zig:355-377: I = 128 + 77 covers every byte, a lane-chunk tail and two
    scale blocks; SIMD bit-build * scale == lut[b] * scale."""
    I = 128 + 77
    w = (np.arange(I) % 256).astype(np.uint8)
    scale_row = np.array([0.5, 1.75], np.float32)
    out = np.empty(I, np.float32)
    oracle_lib.lib().czo_dequant_row(_p(out), _p(w), _p(scale_row), I)
    lut = oracle_lib.lut()
    for i in range(I):
        want = np.float32(lut[w[i]] * scale_row[i // 128])
        if np.isnan(want):
            assert np.isnan(out[i])
        else:
            assert f32_bits(out[i]) == f32_bits(want), i


def test_decode_lane_all_bytes_many_scales(oracle_lib):
    lut = oracle_lib.lut()
    rng = np.random.default_rng(3)
    out = np.empty(8, np.float32)
    for sc in [1.0, 0.5, 1.75, 3.0517578e-05, 2.2e-4, float(rng.uniform(1e-5, 1))]:
        for b0 in range(0, 256, 8):
            w = np.arange(b0, b0 + 8, dtype=np.uint8)
            oracle_lib.lib().czo_decode_lane(_p(w), sc, _p(out))
            for l in range(8):
                want = np.float32(np.float32(lut[w[l]]) * np.float32(sc))
                if np.isnan(want):
                    assert np.isnan(out[l])
                else:
                    assert f32_bits(out[l]) == f32_bits(want)


def test_nblk(oracle_lib):
    """fp8.zig:379-384"""
    f = oracle_lib.lib().czo_nblk
    assert (f(1), f(128), f(129), f(2560)) == (1, 1, 2, 20)


# ---------------------------------------------------------------- dots ----
def test_simd_dots_equal_scalar_lane_emulation(oracle_lib):
    """The AVX2 kernels and the scalar 8-lane emulations agree bit for bit,
    for every length 1..300 (tails of every size) and I = 2048 / 768."""
    lib = oracle_lib.lib()
    rng = np.random.default_rng(11)
    for n in list(range(1, 301)) + [768, 2048, 4096]:
        x = rng.normal(size=n).astype(np.float32)
        y = rng.normal(size=n).astype(np.float32)
        w = rng.integers(0, 256, size=n, dtype=np.uint8)
        w[(w & 0x7F) == 0x7F] = 0x01
        s = rng.uniform(1e-4, 2, size=(n + 127) // 128).astype(np.float32)
        a = lib.czo_dot_fp8_row(_p(x), _p(w), _p(s), n)
        b = lib.czo_dot_fp8_row_scalar(_p(x), _p(w), _p(s), n)
        assert f32_bits(a) == f32_bits(b), n
        a = lib.czo_dot_f32(_p(x), _p(y), n)
        b = lib.czo_dot_f32_scalar(_p(x), _p(y), n)
        assert f32_bits(a) == f32_bits(b), n


def test_dots_exact_on_integer_inputs(oracle_lib):
    """Integer-valued data with small sums: every rounding is exact, so any
    summation order gives the mathematical value."""
    lib = oracle_lib.lib()
    rng = np.random.default_rng(5)
    ints = np.array([0x38, 0x40, 0x48, 0xB8, 0xC0, 0x00], np.uint8)  # 1, 2, 4, -1, -2, 0
    for n in [1, 7, 8, 9, 16, 31, 32, 33, 200, 2048]:
        x = rng.integers(-8, 9, size=n).astype(np.float32)
        w = rng.choice(ints, size=n).astype(np.uint8)
        s = np.ones((n + 127) // 128, np.float32)
        want = float(np.dot(x.astype(np.float64), e4m3_f64(w)))
        assert lib.czo_dot_fp8_row(_p(x), _p(w), _p(s), n) == want
        y = rng.integers(-8, 9, size=n).astype(np.float32)
        assert lib.czo_dot_f32(_p(x), _p(y), n) == float(np.dot(x.astype(np.float64), y))


def test_dot_order_is_the_reference_lane_order(oracle_lib):
    """A planted cancellation that only the reference's chain assignment keeps:
    element 0 (acc0, lane 0) = 2^24, element 8 (acc1, lane 0) = -2^24, element
    1 (acc0, lane 1) = 1.  dotFp8Row: v_0 = 2^24 + -2^24 = 0, sum = 1.
    A plain left-to-right sum would give (2^24 + 1) - 2^24 = 0."""
    lib = oracle_lib.lib()
    n = 16
    x = np.zeros(n, np.float32)
    x[0], x[8], x[1] = 2.0 ** 24, -(2.0 ** 24), 1.0
    w = np.full(n, 0x38, np.uint8)  # 1.0
    s = np.ones(1, np.float32)
    assert lib.czo_dot_fp8_row(_p(x), _p(w), _p(s), n) == 1.0
    # dotF32: acc0 lane0 += 2^24 (i=0), acc1 lane0 += 1 (i=8), acc2 lane 0 -2^24 (i=16)
    n = 32
    a = np.zeros(n, np.float32)
    a[0], a[8], a[16] = 2.0 ** 24, 1.0, -(2.0 ** 24)
    b = np.ones(n, np.float32)
    # total_0 = ((0 + 2^24) + 1) + -2^24 = 0 (2^24 + 1 rounds to 2^24)
    assert lib.czo_dot_f32(_p(a), _p(b), n) == 0.0


def test_matmul_bf16_lane_order_and_widening(oracle_lib):
    """dotBf16 (matmul.zig:84-110): dotF32's chains with each weight widened
    as bits << 16.  Planted: x[0] = 1 (acc0 lane 0), x[8] = 2^24 (acc1 lane
    0), x[16] = -2^24 (acc2 lane 0), x[1] = 1 (acc0 lane 1), weights 1.0 (BF16
    0x3F80).  Lane 0: (1 + 2^24) rounds to 2^24 (ties to even), - 2^24 = 0;
    lane 1: 1; the sum is 1.  A left-to-right sum gives 2.  Then random finite
    BF16 rows against a float64 dot of the widened values."""
    n = 32
    x = np.zeros((1, n), np.float32)
    x[0, 0], x[0, 8], x[0, 16], x[0, 1] = 1.0, 2.0 ** 24, -(2.0 ** 24), 1.0
    w = np.full((1, n), 0x3F80, np.uint16)
    assert oracle_lib.matmul_bf16(x, w, 1, n, 1)[0, 0] == 1.0
    rng = np.random.default_rng(0xBF16)
    S, I, O = 3, 256, 7
    bits = (rng.normal(0.0, 0.02, size=(O, I)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    wf = (bits.astype(np.uint32) << 16).view(np.float32)
    x = rng.normal(size=(S, I)).astype(np.float32)
    y = oracle_lib.matmul_bf16(x, bits, S, I, O)
    ref = x.astype(np.float64) @ wf.astype(np.float64).T
    assert np.all(np.abs(y - ref) <= 1e-5 * np.abs(ref).max() + 1e-30)


def test_matmul_fp8_vs_dequant_reference(oracle_lib):
    """fp8.zig:273-311: S=3, I=200, O=5, demo bytes, scales 0.5+U -> 1e-4 abs."""
    rng = np.random.default_rng(0xF8)
    S, I, O = 3, 200, 5
    x = (rng.random((S, I)) * 2 - 1).astype(np.float32)
    w = np.array(DEMO_BYTES, np.uint8)[rng.integers(0, 8, size=(O, I))]
    s = (0.5 + rng.random((1, 2))).astype(np.float32)
    y = oracle_lib.matmul_fp8(x, w, s, S, I, O)
    ref = x.astype(np.float64) @ deq_f64(w, s).T
    assert np.max(np.abs(y - ref)) < 1e-4


def test_matmul_fp8_s1_fused_any_finite_byte(oracle_lib):
    """fp8.zig:313-353: S=1, I=384, O=6, any finite byte incl. subnormals,
    scales 0.25+U -> 1e-4 rel."""
    rng = np.random.default_rng(0x5115)
    I, O = 384, 6
    x = (rng.random(I) * 2 - 1).astype(np.float32)
    w = rng.integers(0, 256, size=(O, I), dtype=np.uint8)
    w[(w == 0x7F) | (w == 0xFF)] = 0
    s = (0.25 + rng.random((1, 3))).astype(np.float32)
    y = oracle_lib.matmul_fp8(x, w, s, 1, I, O)[0]
    ref = deq_f64(w, s) @ x.astype(np.float64)
    assert np.all(np.abs(y - ref) <= 1e-4 * np.abs(ref) + 1e-6)


def test_matmul_f32_naive_and_threaded_bit_identity(oracle_lib):
    """matmul.zig:133-155 (1e-4 rel vs naive) and :191-216 (threaded ==
    serial, bit for bit)."""
    lib = oracle_lib.lib()
    rng = np.random.default_rng(0xC0FFEE)
    S, I, O = 5, 37, 9
    x = (rng.random((S, I)) * 2 - 1).astype(np.float32)
    w = (rng.random((O, I)) * 2 - 1).astype(np.float32)
    y = np.empty((S, O), np.float32)
    lib.czo_matmul_f32(_p(y), _p(x), _p(w), S, I, O)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.all(np.abs(y - ref) <= 1e-4 * np.abs(ref) + 1e-6)
    S, I, O = 2, 256, 512
    x = (rng.random((S, I)) * 2 - 1).astype(np.float32)
    w = (rng.random((O, I)) * 2 - 1).astype(np.float32)
    ys, yp = np.empty((S, O), np.float32), np.empty((S, O), np.float32)
    lib.czo_parallel_disable()
    lib.czo_matmul_f32(_p(ys), _p(x), _p(w), S, I, O)
    lib.czo_parallel_enable(8)
    try:
        lib.czo_matmul_f32(_p(yp), _p(x), _p(w), S, I, O)
    finally:
        lib.czo_parallel_disable()
    assert np.array_equal(f32_bits(ys), f32_bits(yp))


# ----------------------------------------------------------- exp / act ----
def _audit(oracle_lib, lo, hi, threads=8):
    out = (ctypes.c_uint64 * 5)()
    oracle_lib.lib().czo_exp_audit(oracle_lib.fn_ptr("czo_expf"), lo, hi, threads, out)
    return list(out)


def _bits(f):
    return int(np.array([f], np.float32).view(np.uint32)[0])


@pytest.mark.parametrize("start", [0.0, -1.0, -7.25, -0.001, 1.0, 20.0, 88.0, -87.0, -100.0, -1e-30])
def test_expf_correctly_rounded_windows(oracle_lib, start):
    """czo_expf equals the correctly rounded exp (expl, ambiguity-checked) on
    2^20 consecutive f32 inputs from each start point."""
    b = _bits(start)
    checked, ambiguous, mism, max_ulp, first = _audit(oracle_lib, b, b + (1 << 20))
    assert checked > 0 and mism == 0, (hex(first), max_ulp)


def test_expf_correctly_rounded_strided(oracle_lib):
    """Every 997th bit pattern over the whole f32 range."""
    lib = oracle_lib.lib()
    f = lib.czo_expf
    bits = np.arange(0, 1 << 32, 997, dtype=np.uint64).astype(np.uint32)
    xs = bits.view(np.float32)
    xs = xs[~np.isnan(xs)][::7]
    # f64 exp rounded to f32: correct unless within 2^-29 relative of a midpoint
    for x in xs[:20000]:
        got = f(float(x))
        ref = np.exp(np.float64(x))
        assert got == np.float32(ref) or abs(got - ref) <= 2.0 ** -52 * abs(ref) * 2 ** 29, x


@pytest.mark.skipif(not os.environ.get("CZ_SLOW"), reason="exhaustive 2^32 audit takes minutes (CZ_SLOW=1)")
def test_expf_exhaustive(oracle_lib):
    checked, ambiguous, mism, max_ulp, first = _audit(oracle_lib, 0, 1 << 32, threads=os.cpu_count() or 8)
    assert mism == 0, (mism, max_ulp, hex(first))


def test_sigmoid_silu_points(oracle_lib):
    """activation.zig:42-47"""
    lib = oracle_lib.lib()
    assert abs(lib.czo_sigmoid(0.0) - 0.5) <= 1e-6
    assert abs(lib.czo_sigmoid(1.0) - 0.7310586) <= 1e-5
    assert abs(lib.czo_silu(0.0)) <= 1e-6
    assert abs(lib.czo_sigmoid(-3.0) - (1.0 - lib.czo_sigmoid(3.0))) <= 1e-6
    for v in np.linspace(-30, 30, 1201):
        ref = 1.0 / (1.0 + np.exp(-np.float64(np.float32(v))))
        assert abs(lib.czo_sigmoid(float(v)) - ref) <= 2e-7 * max(ref, 1e-30) + 1e-30


# ---------------------------------------------------------------- route ----
def _layer(H=512, E=16, K=4, I=256, SI=0, seed=0, norm=True):
    from colizig_amd.synth import make_layer
    return make_layer(H, E, K, I, SI, norm, seed=seed)


def test_route_vs_bruteforce_topk(oracle_lib):
    host = _layer()
    L = oracle_lib.OracleLayer(host)
    rng = np.random.default_rng(1)
    for _ in range(64):
        x = rng.normal(size=512).astype(np.float32)
        idx, gates, v = L.route(x)
        lg = L.router_logits(x)
        mx = np.max(lg)
        ref_v = np.exp((lg - mx).astype(np.float64)).astype(np.float32)
        assert np.array_equal(v, ref_v)  # correctly rounded exp of the f32 difference
        order = sorted(range(16), key=lambda e: (-v[e], e))[:4]
        assert list(idx) == order
        assert abs(float(np.sum(gates, dtype=np.float64)) - 1.0) < 1e-6
        assert np.all(np.diff(gates) <= 0)


def test_route_ties_pick_lowest_index(oracle_lib):
    host = _layer(E=8, K=3)
    r = host["router"]
    r[5] = r[2]
    r[7] = r[2]  # experts 2, 5, 7 always tie
    r[2] *= 0
    r[2] += 10 * np.abs(r[1])  # and make them clearly the largest for a positive x
    r[5] = r[2]
    r[7] = r[2]
    L = oracle_lib.OracleLayer(host)
    x = np.abs(np.random.default_rng(2).normal(size=512)).astype(np.float32)
    idx, gates, _ = L.route(x)
    assert list(idx) == [2, 5, 7]
    assert gates[0] == gates[1] == gates[2]


def test_route_without_norm_topk_uses_all(oracle_lib):
    host = _layer(norm=False)
    L = oracle_lib.OracleLayer(host)
    x = np.random.default_rng(3).normal(size=512).astype(np.float32)
    idx, gates, v = L.route(x)
    all_ = float(np.sum(v.astype(np.float64)))
    for z in range(4):
        assert gates[z] == np.float32(np.float64(v[idx[z]]) / all_)


# ------------------------------------------------------------- forward ----
@pytest.mark.parametrize("SI", [0, 256])
def test_moe_forward_vs_f64(oracle_lib, SI):
    host = _layer(SI=SI, seed=4)
    L = oracle_lib.OracleLayer(host)
    x = np.random.default_rng(4).normal(size=(3, 512)).astype(np.float32)
    for S in (1, 3):
        out, idx, _ = L.forward(x[:S])
        ref, ridx = moe_f64(host, x[:S])
        assert np.array_equal(idx, ridx)
        assert rel_l2(out, ref) < 1e-5


@pytest.mark.parametrize("shared", ["f32", "bf16"])
def test_native_shared_and_bf16_router_vs_f64(oracle_lib, shared):
    """NativeMatrix weights (tensors.zig:65-120): a BF16 router and an f32 or
    BF16 shared expert evaluated as dense rows (moe.zig:467-479), against the
    independent float64 MoE that widens BF16 bits itself.  Zeroing the shared
    gate's weights moves the output (the shared term is present), and the
    BF16 router's logits are the widened rows' dots (routing agrees)."""
    from colizig_amd import synth
    host = synth.with_native(_layer(SI=256, seed=41), seed=42, shared=shared)
    assert host["router"].dtype == np.uint16
    L = oracle_lib.OracleLayer(host)
    x = np.random.default_rng(43).normal(size=(3, 512)).astype(np.float32)
    for S in (1, 3):
        out, idx, _ = L.forward(x[:S])
        ref, ridx = moe_f64(host, x[:S])
        assert np.array_equal(idx, ridx)
        assert rel_l2(out, ref) < 1e-5
    no_sh = dict(host, shared=dict(host["shared"], down=np.zeros_like(host["shared"]["down"])))
    out0, _, _ = oracle_lib.OracleLayer(no_sh).forward(x)
    ref0, _ = moe_f64(no_sh, x)
    assert rel_l2(out0, ref0) < 1e-5
    assert rel_l2(out0, out) > 1e-3


def test_grouped_equals_dense_per_token(oracle_lib):
    """moe.zig:720-728: grouped prefill ~= per-token dense within 1e-3 abs,
    and (moe.zig:717-718) deterministic across fresh runs."""
    host = _layer(seed=5)
    L = oracle_lib.OracleLayer(host)
    x = np.random.default_rng(0x30E).uniform(-1, 1, size=(9, 512)).astype(np.float32)
    o1, i1, g1 = L.forward(x)
    o2, i2, g2 = L.forward(x)
    assert np.array_equal(f32_bits(o1), f32_bits(o2))
    od, idd, gd = L.forward(x, dense_each=True)
    assert np.array_equal(i1, idd) and np.array_equal(f32_bits(g1), f32_bits(gd))
    assert np.max(np.abs(o1 - od)) < 1e-3
    assert np.all(np.isfinite(o1))


def test_threaded_forward_bit_identical(oracle_lib):
    host = _layer(seed=6)
    L = oracle_lib.OracleLayer(host)
    x = np.random.default_rng(6).normal(size=(4, 512)).astype(np.float32)
    lib = oracle_lib.lib()
    lib.czo_parallel_disable()
    a = [L.forward(x[:1])[0], L.forward(x)[0]]
    lib.czo_parallel_enable(8)
    try:
        b = [L.forward(x[:1])[0], L.forward(x)[0]]
    finally:
        lib.czo_parallel_disable()
    for u, v in zip(a, b):
        assert np.array_equal(f32_bits(u), f32_bits(v))


def test_tiny_qwen3_fixture(oracle_lib):
    """The reference fixture's MoE layers (tools/gen_tiny_fixture.zig restated):
    routing equals the f64 golden, outputs within 1e-5 rel L2."""
    for li in range(4):
        host, gold = tiny_qwen3_layer(li)
        L = oracle_lib.OracleLayer(host)
        out, idx, _ = L.forward(gold["x"])
        assert np.array_equal(idx, gold["idx"])
        assert rel_l2(out, gold["out"]) < 1e-5
        od, _, _ = L.forward(gold["x"], dense_each=True)
        assert np.max(np.abs(out - od)) < 1e-3


# ---------------------------------------------------------- decode chain ----
def test_rms_unit_closed_form(oracle_lib):
    """czo_rms_unit (rmsnorm.zig:32-40 with a unit weight) against the float64
    closed form x / sqrt(mean(x^2) + eps): a sum in place of the mean, eps
    outside the square root or a dropped square each miss this by far more
    than 2e-6."""
    rng = np.random.default_rng(3)
    for H, scale in [(512, 1.0), (2048, 1.0), (4096, 30.0), (2048, 1e-3), (7, 2.0)]:
        x = (rng.normal(size=(3, H)) * scale).astype(np.float32)
        for eps in (1e-6, 1e-5, 0.1):
            got = oracle_lib.rms_unit(x, eps)
            x64 = x.astype(np.float64)
            want = x64 / np.sqrt(np.mean(x64 * x64, axis=1, keepdims=True) + eps)
            assert np.max(np.abs(got - want) / np.abs(want)) < 2e-6, (H, scale, eps)
    # rmsnorm.zig:67-73 with a unit (not zero-centred) weight: +-1 rows, eps 0
    got = oracle_lib.rms_unit(np.array([[1, -1, 1, -1]], np.float32), 0.0)
    assert np.array_equal(np.abs(got), np.ones((1, 4), np.float32))
    # eps is added to the mean inside the root: a constant row c -> c / sqrt(c^2 + eps)
    got = oracle_lib.rms_unit(np.full((1, 16), 3.0, np.float32), 0.25)
    assert abs(float(got[0, 0]) - 3.0 / np.sqrt(9.25)) < 1e-6


def test_rms_unit_is_the_reference_arithmetic(oracle_lib):
    """Bit-exact against the reference's steps done in numpy: f64 sum of
    f64(v)*v, mean cast to f32, r = 1/sqrt(mean+eps) in f32, v*r."""
    rng = np.random.default_rng(9)
    for H in (512, 2048, 4096):
        x = rng.normal(size=(4, H)).astype(np.float32)
        eps = np.float32(1e-6)
        got = oracle_lib.rms_unit(x, float(eps))
        for r in range(4):
            ss = 0.0
            for v in x[r].astype(np.float64):
                ss += v * v
            mean = np.float32(ss / H)
            inv = np.float32(1.0) / np.sqrt(np.float32(mean + eps), dtype=np.float32)
            assert np.array_equal(f32_bits(got[r]), f32_bits(x[r] * inv))


def test_chain_layer_is_rms_moe_residual(oracle_lib):
    """czo_chain_layer = rms, then moe.forward on it, then the residual add
    (qwen3moe/model.zig:228-232), bit for bit; and within 1e-5 of the float64
    pipeline x + moe_f64(x / sqrt(mean(x^2) + eps))."""
    host = _layer(seed=5)
    L = oracle_lib.OracleLayer(host)
    x = np.random.default_rng(11).normal(size=(3, 512)).astype(np.float32)
    eps = 1e-6
    for S in (1, 3):
        xc = x[:S].copy()
        xn, idx, gates = L.chain(xc, eps)
        xn2 = oracle_lib.rms_unit(x[:S], eps)
        assert np.array_equal(f32_bits(xn), f32_bits(xn2))
        out, ri, rg = L.forward(xn2)
        assert np.array_equal(idx, ri) and np.array_equal(f32_bits(gates), f32_bits(rg))
        assert np.array_equal(f32_bits(xc), f32_bits(x[:S] + out))
        x64 = x[:S].astype(np.float64)
        xn64 = x64 / np.sqrt(np.mean(x64 * x64, axis=1, keepdims=True) + eps)
        ref, _ = moe_f64(host, xn64)
        assert rel_l2(xc, x64 + ref) < 1e-5


# ------------------------------------------------------- cache / chunks ----
def _replay(oracle_lib, cap, ids):
    ids = np.array(ids, np.uint32)
    slots = np.empty(len(ids), np.int32)
    st = oracle_lib.CCacheStats()
    res = oracle_lib.lib().czo_cache_replay(cap, _p(ids), len(ids), _p(slots), ctypes.byref(st))
    return res, list(slots), st


def test_cache_policy(oracle_lib):
    """moe.zig:141-249 / :730-741: empty slots first, LRU victim, cap-1 evicts
    every distinct expert, warm replay is all hits."""
    res, slots, st = _replay(oracle_lib, 3, [5, 6, 7, 5, 8, 6, 9])
    # 5->0, 6->1, 7->2, hit 5 (slot 0 used=4), 8 evicts LRU slot 1 (6), 6 evicts slot 2 (7), 9 evicts slot 0 (5)
    assert slots == [0, 1, 2, 0, 1, 2, 0]
    assert (st.hits, st.misses, st.evictions, st.loads) == (1, 6, 3, 6)
    res, slots, st = _replay(oracle_lib, 1, [1, 2, 1, 3])
    assert res == 1 and st.evictions == 3 and st.hits == 0
    ids = [3, 1, 2, 0]
    res, _, st = _replay(oracle_lib, 4, ids + ids)
    assert st.misses == 4 and st.hits == 4 and st.evictions == 0


def test_chunk_bounds(oracle_lib):
    """parallel.zig:50-76 / :348-375"""
    lib = oracle_lib.lib()
    buf = np.zeros(2 * 64, np.uint32)
    lib.czo_parallel_enable(8)
    try:
        n = lib.czo_chunk_bounds(1000, 1 << 20, _p(buf), 64)
        pairs = buf[: 2 * n].reshape(-1, 2)
        assert n == 8 and pairs[0][0] == 0 and pairs[-1][1] == 1000
        assert all(pairs[i][1] == pairs[i + 1][0] for i in range(n - 1))
        assert all(p[1] - p[0] == 125 for p in pairs)
        assert lib.czo_chunk_bounds(1000, 10, _p(buf), 64) == 1  # below min_work
        assert lib.czo_chunk_bounds(5, 1 << 20, _p(buf), 64) == 5  # tasks capped at n
    finally:
        lib.czo_parallel_disable()


def test_router_bias_is_one_add_after_the_dot(oracle_lib):
    """The optional router bias (workload shaping) adds bias[e] to each logit
    with one f32 add after the dotF32 logit; without it routing is the
    reference's."""
    from colizig_amd import synth
    host = synth.make_layer(256, 32, 4, 128, 0, True, seed=3)
    plain = oracle_lib.OracleLayer(host)
    bias = synth.zipf_router_bias(32, 1.1, seed=1)
    biased = oracle_lib.OracleLayer(dict(host, router_bias=bias))
    x = synth.hidden_states(1, 256, seed=4)[0]
    want = (plain.router_logits(x) + bias).astype(np.float32)
    assert np.array_equal(biased.router_logits(x).view(np.uint32), want.view(np.uint32))
    # the biased route is the reference route on the biased logits: brute force
    idx, _, _ = biased.route(x)
    v = np.exp(want.astype(np.float64) - want.max())
    order = sorted(range(32), key=lambda e: (-v[e], e))[:4]
    assert list(idx) == order


def test_zipf_bias_skews_popularity(oracle_lib):
    """Zipf(1.1) bias: over many tokens the most popular expert is picked far
    more often than the median one (a property of the workload generator)."""
    from colizig_amd import synth
    host = synth.make_layer(128, 64, 4, 128, 0, True, seed=8)
    host["router_bias"] = synth.zipf_router_bias(64, 1.1, seed=2)
    O = oracle_lib.OracleLayer(host)
    _, idx, _ = O.forward(synth.hidden_states(256, 128, seed=8))
    c = np.bincount(idx.ravel(), minlength=64)
    assert c.max() > 4 * max(np.median(c), 1)


def _ops(*rows):
    return np.array(rows, np.uint32).reshape(-1, 4)


GET, PRE, WARM, CLEAR, EPOCH = 1, 2, 3, 4, 0
HIT = 0x80000000


def test_pool_replay_is_the_reference_lru_without_pins(oracle_lib):
    """With every get in a layer of its own (no pins held across gets) and no
    prefetch, the pool replay is the reference's per-layer LRU: the same slot
    for every get as czo_cache_replay on a random trace (whose own policy the
    hand-worked traces of test_cache_policy pin)."""
    rng = np.random.default_rng(7)
    for cap in (1, 3, 8):
        ids = rng.integers(0, 12, size=200).astype(np.uint32)
        _, slots, cst = _replay(oracle_lib, cap, ids)
        ops = []
        for e in ids:
            ops += [(EPOCH, 0, 0, 0), (GET, 5, int(e), 0)]
        r, res, st = oracle_lib.pool_replay(cap, _ops(*ops))
        gets = res[1::2]
        assert [int(x) & 0x7fffffff for x in gets] == [int(s) for s in slots]
        assert (st["hits"], st["misses"], st["evictions"], st["loads"]) == (cst.hits, cst.misses, cst.evictions,
                                                                          cst.loads)
        assert int(sum(int(x) >> 31 for x in gets)) == cst.hits


def test_pool_replay_pins_and_prefetch(oracle_lib):
    """Hand-worked: pins of the layer in flight are spared, a prefetch of a
    resident key is a no-op, one with every slot pinned is dropped, a
    prefetched slot consumed by a get is a prefetch hit, one evicted unused
    is wasted; keys of different layers never alias."""
    r, res, st = oracle_lib.pool_replay(3, _ops(
        (EPOCH, 0, 0, 0), (GET, 0, 1, 0), (GET, 0, 2, 0),      # slots 0, 1 pinned
        (PRE, 1, 1, 0),                                          # free slot 2
        (PRE, 1, 1, 0),                                          # resident: no-op
        (PRE, 1, 2, 0),                                          # LRU unpinned = slot 2 (just filled): evicts it, wasted
        (EPOCH, 1, 0, 0), (GET, 1, 2, 0),                        # layer 1 expert 2: hit on slot 2, prefetch hit
        (GET, 1, 1, 0),                                          # evicted above: miss, victim LRU unpinned = slot 0
        (GET, 1, 3, 0),                                          # slots 0 and 2 pinned: victim slot 1
        (PRE, 2, 0, 0),                                          # every slot pinned: dropped
    ))
    assert r == 3
    assert list(res) == [0, 0, 1, 2, 0xfffffffe, 2, 0, 2 | HIT, 0, 1, 0xffffffff]
    assert st == dict(hits=1, misses=4, loads=6, evictions=3, prefetch_issued=2, prefetch_hits=1, prefetch_wasted=1)


def test_pool_replay_warm_clear_and_full_pin(oracle_lib):
    """Warm fills take free slots only; clear frees every slot (counters
    kept); a get with every slot pinned is an error (-1)."""
    r, res, st = oracle_lib.pool_replay(2, _ops((WARM, 0, 4, 0), (WARM, 0, 5, 0), (WARM, 0, 6, 0),
                                                (EPOCH, 0, 0, 0), (GET, 0, 5, 0), (CLEAR, 0, 0, 0),
                                                (EPOCH, 0, 0, 0), (GET, 0, 5, 0)))
    assert list(res) == [0, 1, 0xffffffff, 0, 1 | HIT, 0, 0, 0]
    assert st["prefetch_issued"] == 2 and st["prefetch_hits"] == 1 and st["misses"] == 1 and r == 1
    r, _, _ = oracle_lib.pool_replay(1, _ops((EPOCH, 0, 0, 0), (GET, 0, 1, 0), (GET, 0, 2, 0)))
    assert r == -1


def test_pool_replay_invariants(oracle_lib):
    """The cache invariants (moe.zig:711-741) on random logs: hits + misses =
    gets; loads = misses + prefetch fills; evictions = loads - resident -
    (slots freed by clears); resident <= slots."""
    rng = np.random.default_rng(11)
    for nslots in (4, 16):
        ops = []
        for step in range(60):
            for layer in range(3):
                ops.append((EPOCH, layer, 0, 0))
                for e in rng.choice(10, size=3, replace=False):
                    ops.append((GET, layer, int(e), 0))
                for e in rng.choice(10, size=2, replace=False):
                    ops.append((PRE, (layer + 1) % 3, int(e), 0))
        r, res, st = oracle_lib.pool_replay(nslots, _ops(*ops))
        a = _ops(*ops)
        gets = int((a[:, 0] == GET).sum())
        fills_pre = int(((a[:, 0] == PRE) & (res < 0xfffffffe)).sum())
        assert st["hits"] + st["misses"] == gets
        assert st["loads"] == st["misses"] + fills_pre == st["misses"] + st["prefetch_issued"]
        assert st["evictions"] == st["loads"] - r
        assert 0 <= r <= nslots
        assert st["prefetch_hits"] + st["prefetch_wasted"] <= st["prefetch_issued"]
