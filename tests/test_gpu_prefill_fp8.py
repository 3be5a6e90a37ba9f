"""The grouped regime with its GEMMs on FP8 MFMA (colizig_hip_set_prefill_fp8):
every case of tests/test_gpu_grouped.py run again in that mode, against the
same oracle and bar (routing bit-exact, outputs within 1e-3 relative L2),
at the config-1 shapes, with a shared expert, ragged tiles and the
Qwen3-30B-A3B 512-token Zipf(1.1) prefill."""
from __future__ import annotations

import pytest

from colizig_amd import _lib
from tests.test_gpu_grouped import *  # noqa: F401,F403  (the cases, collected again in this mode)

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def fp8_mode(gpu):
    hip = _lib.hip()
    prev = hip.colizig_hip_set_prefill_fp8(1)
    yield
    hip.colizig_hip_set_prefill_fp8(prev)
