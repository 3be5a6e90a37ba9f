"""BF16 GEMV on device pointers (colizig_hip_matrix_load_bf16 +
colizig_hip_matmul_bf16_dev) vs the oracle's dotBf16 rows (matmul.zig:84-110):
bit-identical, at lm_head-like and Qwen4-Exp router-like shapes."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from colizig_amd import _lib, moe
from tests.helpers import f32_bits

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _bf16(rng, O, I):
    return (rng.normal(0.0, 0.02, size=(O, I)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)


# the last three widths are not a multiple of 256 x 32 tiles: the any-width
# kernel, dotBf16's 8-wide steps and scalar tail included (200 = 6*32 + 8,
# 45 = 32 + 8 + 5)
@pytest.mark.parametrize("O,I,S", [(1000, 2048, 1), (4099, 2048, 3), (512, 4096, 2), (33, 256, 5), (96, 3072, 1),
                                   (8, 200, 3), (17, 45, 2), (64, 384, 1)])
def test_bf16_rows_bit_exact(gpu, oracle_lib, O, I, S):
    say(f"bf16 gemv {O}x{I} S={S}")
    moe.set_vram_budget(1 << 30)
    rng = np.random.default_rng(O + I + S)
    w = _bf16(rng, O, I)
    key = moe.Fp8Matrix.expert_key(40, O % 500, 3)
    xb = moe.DeviceBuffer(S * I * 4)
    yb = moe.DeviceBuffer(S * O * 4)
    try:
        moe.matrix_load_bf16(key, w)
        x = rng.normal(size=(S, I)).astype(np.float32)
        xb.upload(x)
        moe.matmul_bf16_dev(yb.ptr, xb.ptr, S, I, O, key)
        assert _lib.hip().colizig_hip_sync() == 0
        y = yb.download(np.empty((S, O), np.float32))
        ref = oracle_lib.matmul_bf16(x, w, S, I, O)
        assert np.array_equal(f32_bits(y), f32_bits(ref))
    finally:
        xb.free()
        yb.free()
        moe.set_vram_budget(0)


def test_bf16_key_type_checks(gpu):
    """A BF16 key is not an FP8 matrix and the reverse (-1); a call with
    another shape than the resident one (-1); a missing key (-7)."""
    say("bf16 key checks")
    hip = _lib.hip()
    moe.set_vram_budget(1 << 30)
    rng = np.random.default_rng(9)
    xb = moe.DeviceBuffer(4096 * 4)
    yb = moe.DeviceBuffer(4096 * 4)
    try:
        kb = moe.Fp8Matrix.expert_key(41, 0, 3)
        moe.matrix_load_bf16(kb, _bf16(rng, 64, 2048))
        assert hip.colizig_hip_matmul_fp8_dev(yb.ptr, xb.ptr, 1, 2048, 64, kb, None) == -1
        assert hip.colizig_hip_matmul_bf16_dev(yb.ptr, xb.ptr, 1, 2048, 64, kb, None) == 0
        kw = moe.Fp8Matrix.expert_key(41, 1, 3)
        moe.matrix_load_bf16(kw, _bf16(rng, 8, 200))
        assert hip.colizig_hip_matmul_bf16_dev(yb.ptr, xb.ptr, 1, 200, 8, kw, None) == 0
        assert hip.colizig_hip_matmul_bf16_dev(yb.ptr, xb.ptr, 1, 192, 8, kw, None) == -1
        assert hip.colizig_hip_matmul_bf16_dev(yb.ptr, xb.ptr, 1, 2048, 64, 0xBADBAD, None) == -7
        assert hip.colizig_hip_sync() == 0
    finally:
        xb.free()
        yb.free()
        moe.set_vram_budget(0)
