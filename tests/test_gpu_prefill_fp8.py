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
def mfma_mode(gpu):  # shadows test_gpu_grouped's f16 fixture of the same name
    hip = _lib.hip()
    prev = hip.colizig_hip_set_prefill_fp8(1)
    yield
    hip.colizig_hip_set_prefill_fp8(prev)


@pytest.mark.parametrize("SI", [0, 256])
def test_fp8_chain_vs_oracle_chain(gpu, oracle_lib, SI):
    """The chained grouped regime on FP8 MFMA, where the RMS rows kernel writes
    the gate/up GEMM's E4M3 terms of xn (with and without a shared expert):
    3 layers x 2 steps of 20 tokens against the oracle's own chain from the
    same x0 (routing bit-exact on the GPU's router inputs and against the
    oracle chain's picks, router inputs and residual stream within 1e-3)."""
    from colizig_amd import synth
    from tests.test_gpu_chain import chain_vs_oracle
    hosts = [synth.make_layer(512, 16, 4, 256, SI, True, seed=331 + l + SI) for l in range(3)]
    chain_vs_oracle(oracle_lib, hosts, 2100 + SI, 20, tokens=2, seed=5, label=f"fp8 chain SI={SI}")


def test_fp8_prefill_48_layers_vs_oracle_chain(gpu):
    """The default FP8 prefill at depth: bench.py's prefill leg (48
    Qwen3-30B-A3B-shape layers, 512 tokens, Zipf(1.1) routing skew) checks the
    first 64 tokens' rows against the oracle's own 48-layer chain of those
    tokens from the same x0, in FP8 and in f16 mode.  Both must route
    bit-exactly at every layer, keep the router inputs and the final residual
    stream within 1e-3 relative L2, and the oracle's decisions must sit at
    least 8 ulps from a tie."""
    import json
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-u", os.path.join(root, "bench.py"), "--workload", "prefill", "--steps", "1",
                        "--warmup", "1"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]
    line = json.loads(r.stdout.strip().splitlines()[-1])
    res = line["parity"]["oracle_chain"]
    print(res, flush=True)
    assert res["layers_checked"] == 48 and res["tokens_checked"] == 64
    assert res["near_tie_min_gap_ulps"] >= 8
    for mode in ("fp8", "f16"):
        assert res[mode]["routing_bit_exact"], mode
        assert res[mode]["max_router_input_rel_l2"] < 1e-3, mode
        assert res[mode]["residual_rel_l2"] < 1e-3, mode
    assert line["parity"]["token_independence"]["bit_identical"]
    assert line["cpu_baseline"]["kind"] == "port" and line["cpu_baseline"]["value"] > 0
