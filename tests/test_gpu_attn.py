"""Keyed FP8 GEMV on device pointers (colizig_hip_matrix_load +
colizig_hip_matmul_fp8_dev): the Qwen3-30B-A3B attention projections
(attn.zig:55-58 shapes, q/k/v/o keyed by attnKey, attn.zig:47-50) and other
Fp8Matrix shapes vs the oracle's matmulFp8 (fp8.zig:182 semantics).  Bar:
relative L2 1e-5 (the same per-128-block partial sums as the decode kernels;
the oracle sums every product in order)."""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest

from colizig_amd import _lib, moe, synth
from tests.helpers import f32_bits, rel_l2

pytestmark = pytest.mark.gpu

RTOL_L2 = 1e-5
H, QD, KVD = 2048, 32 * 128, 4 * 128  # hidden, q_heads*head_dim, kv_heads*head_dim


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _dev_matmul(x: np.ndarray, key: int, I: int, O: int) -> np.ndarray:
    S = x.shape[0]
    xb = moe.DeviceBuffer(x.nbytes)
    yb = moe.DeviceBuffer(S * O * 4)
    try:
        xb.upload(x)
        moe.matmul_fp8_dev(yb.ptr, xb.ptr, S, I, O, key)
        assert _lib.hip().colizig_hip_sync() == 0
        return yb.download(np.empty((S, O), np.float32))
    finally:
        xb.free()
        yb.free()


@pytest.mark.parametrize("S", [1, 3, 5])
def test_attention_projections(gpu, oracle_lib, S):
    """q [4096 x 2048], k and v [512 x 2048], o [2048 x 4096] of one layer,
    loaded under their attention keys, S tokens (several passes of the
    kernel's token staging when S exceeds it)."""
    say(f"attention projections S={S}")
    moe.set_vram_budget(1 << 30)
    rng = np.random.default_rng(100 + S)
    shapes = [(QD, H), (KVD, H), (KVD, H), (H, QD)]  # (O, I) for roles q, k, v, o
    try:
        for role, (O, I) in enumerate(shapes):
            w, s = synth.block_quantize(rng.normal(0, 0.02, size=(O, I)).astype(np.float32))
            key = moe.Fp8Matrix.attn_key(7, role)
            moe.matrix_load(key, w, s)
            x = rng.normal(size=(S, I)).astype(np.float32)
            y = _dev_matmul(x, key, I, O)
            ref = oracle_lib.matmul_fp8(x, w, s, S, I, O)
            err = rel_l2(y, ref)
            say(f"  role {role} {O}x{I}: rel L2 {err:.2e}")
            assert err < RTOL_L2
    finally:
        moe.set_vram_budget(0)


@pytest.mark.parametrize("O,I,S", [(130, 256, 2), (7, 200, 3), (300, 3072, 1)])
def test_matmul_dev_other_shapes(gpu, oracle_lib, O, I, S):
    """Rows not a multiple of the workgroup's 4, a row width off the 128-bit
    path (I = 200: the generic kernel), and I = 3072."""
    say(f"matmul_fp8_dev {O}x{I} S={S}")
    moe.set_vram_budget(1 << 30)
    try:
        rng = np.random.default_rng(O * 7 + I)
        w, s = synth.block_quantize(rng.normal(0, 0.02, size=(O, I)).astype(np.float32))
        key = moe.Fp8Matrix.expert_key(9, O, 1)
        moe.matrix_load(key, w, s)
        x = rng.normal(size=(S, I)).astype(np.float32)
        assert rel_l2(_dev_matmul(x, key, I, O), oracle_lib.matmul_fp8(x, w, s, S, I, O)) < RTOL_L2
    finally:
        moe.set_vram_budget(0)


def test_matmul_dev_same_key_as_host_path(gpu):
    """A matrix cached by the host keyed matmul serves the device call, and a
    reload under the same key replaces it; both paths agree to the bar."""
    say("matmul_fp8_dev shares the keyed cache")
    moe.set_vram_budget(1 << 30)
    try:
        rng = np.random.default_rng(5)
        O, I, S = 256, 2048, 2
        key = moe.Fp8Matrix.attn_key(11, 0)
        w, s = synth.block_quantize(rng.normal(0, 0.02, size=(O, I)).astype(np.float32))
        x = rng.normal(size=(S, I)).astype(np.float32)
        y_host = moe.matmul_fp8(x, w, s, S, I, O, key=key)
        assert rel_l2(_dev_matmul(x, key, I, O), y_host) < RTOL_L2
        w2, s2 = synth.block_quantize(rng.normal(0, 0.02, size=(O, I)).astype(np.float32))
        moe.matrix_load(key, w2, s2)
        y2 = _dev_matmul(x, key, I, O)
        assert rel_l2(y2, moe.matmul_fp8(x, w2, s2, S, I, O, key=0)) < RTOL_L2
        assert not np.array_equal(f32_bits(y2), f32_bits(y_host))
    finally:
        moe.set_vram_budget(0)


def test_matmul_dev_errors(gpu):
    """A key that is not resident (-7), a shape other than the resident one
    (-1), no cache budget for a load (-8): errors, no launch."""
    say("matmul_fp8_dev errors")
    hip = _lib.hip()
    xb = moe.DeviceBuffer(4 * 2048 * 4)
    yb = moe.DeviceBuffer(4 * 2048 * 4)
    try:
        assert hip.colizig_hip_matmul_fp8_dev(yb.ptr, xb.ptr, 1, 2048, 512, 0xDEADBEEF, None) == -7
        moe.set_vram_budget(1 << 30)
        rng = np.random.default_rng(3)
        w, s = synth.block_quantize(rng.normal(0, 0.02, size=(512, 2048)).astype(np.float32))
        key = moe.Fp8Matrix.attn_key(12, 1)
        moe.matrix_load(key, w, s)
        assert hip.colizig_hip_matmul_fp8_dev(yb.ptr, xb.ptr, 1, 2048, 256, key, None) == -1
        assert hip.colizig_hip_matmul_fp8_dev(yb.ptr, xb.ptr, 1, 1024, 512, key, None) == -1
        moe.set_vram_budget(0)
        assert hip.colizig_hip_matrix_load(moe.Fp8Matrix.attn_key(12, 2), w.ctypes.data, s.ctypes.data, 2048,
                                           512) == -8
    finally:
        moe.set_vram_budget(0)
        xb.free()
        yb.free()


@pytest.mark.parametrize("S", [1, 5])
def test_qkv_in_one_launch(gpu, oracle_lib, S):
    """colizig_hip_matmul_fp8_dev_multi: a layer's q, k and v projections on
    the same input rows in one launch give, for each matrix, the bits of its
    own colizig_hip_matmul_fp8_dev call, and the oracle's matmulFp8 to the
    bar.  Also a row width off the 128-bit path (one launch per matrix
    there) and the argument checks."""
    say(f"q/k/v in one launch S={S}")
    hip = _lib.hip()
    moe.set_vram_budget(1 << 30)
    rng = np.random.default_rng(300 + S)
    bufs = []
    try:
        for I, Os in ((H, (QD, KVD, KVD)), (200, (130, 7))):
            mats, keys = [], []
            for role, O in enumerate(Os):
                w, s = synth.block_quantize(rng.normal(0, 0.02, size=(O, I)).astype(np.float32))
                key = moe.Fp8Matrix.attn_key(21 if I == H else 22, role)
                moe.matrix_load(key, w, s)
                mats.append((w, s))
                keys.append(key)
            x = rng.normal(size=(S, I)).astype(np.float32)
            xb = moe.DeviceBuffer(x.nbytes)
            xb.upload(x)
            ybs = [moe.DeviceBuffer(S * O * 4) for O in Os]
            bufs += [xb] + ybs
            moe.matmul_fp8_dev_multi([b.ptr for b in ybs], xb.ptr, S, I, Os, keys)
            assert hip.colizig_hip_sync() == 0
            for m, O in enumerate(Os):
                y = ybs[m].download(np.empty((S, O), np.float32))
                single = _dev_matmul(x, keys[m], I, O)
                assert np.array_equal(f32_bits(y), f32_bits(single)), f"I={I} matrix {m}: bits"
                ref = oracle_lib.matmul_fp8(x, mats[m][0], mats[m][1], S, I, O)
                assert rel_l2(y, ref) < RTOL_L2
        # argument checks: too many matrices, a key not resident, a shape other than the resident one
        y3 = (ctypes.c_void_p * 5)(*([bufs[1].ptr] * 5))
        k3 = (ctypes.c_uint64 * 5)(*([keys[0]] * 5))
        o3 = (ctypes.c_int * 5)(*([130] * 5))
        assert hip.colizig_hip_matmul_fp8_dev_multi(5, y3, k3, o3, bufs[0].ptr, 1, 200, None) == -1
        k3[0] = 0xDEADBEEF
        assert hip.colizig_hip_matmul_fp8_dev_multi(1, y3, k3, o3, bufs[0].ptr, 1, 200, None) == -7
        k3[0] = keys[0]
        o3[0] = 131
        assert hip.colizig_hip_matmul_fp8_dev_multi(1, y3, k3, o3, bufs[0].ptr, 1, 200, None) == -1
    finally:
        moe.set_vram_budget(0)
        for b in bufs:
            b.free()
