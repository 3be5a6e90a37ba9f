"""NativeMatrix weights in the MoE layer (src/model/tensors.zig:65-120): a
BF16 router (logits in dotBf16's order, matmul.zig:84-110) and a shared
expert of f32 or BF16 rows (moe.zig:300-303, 316-325, 467-479), as the
reference loads them, against the oracle (BF16 widened exactly, dotF32):
routing bit-exact, outputs within 1e-3 relative L2, at the config-1 and the
Qwen4-Exp-style (config-4) shapes."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from colizig_amd import _lib, moe, synth
from tests.helpers import f32_bits, rel_l2
from tests.test_gpu_chain import chain_vs_oracle

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _check_forward(L, O, x, label):
    out, idx, gates = L.forward(x)
    ro, ri, rg = O.forward(x)
    assert np.array_equal(idx, ri), f"{label}: routing"
    assert np.array_equal(f32_bits(gates), f32_bits(rg)), f"{label}: gates"
    err = rel_l2(out, ro)
    assert err < 1e-3, f"{label}: rel L2 {err:.2e}"
    return err


@pytest.mark.parametrize("shared", [None, "bf16", "f32"])
def test_native_tiny_forward(gpu, oracle_lib, shared):
    """Config-1 shapes (shared expert of 384 rows when asked): S = 1, 2
    (decode kernels) and 20 (grouped regime)."""
    say(f"native weights tiny, shared={shared}")
    SI = 384 if shared else 0
    host = synth.with_native(synth.make_layer(512, 16, 4, 256, SI, True, seed=91), seed=92, shared=shared)
    assert host["router"].dtype == np.uint16
    L = moe.register_layer(4000 + (SI and (1 if shared == "bf16" else 2)), host)
    O = oracle_lib.OracleLayer(host)
    x = synth.hidden_states(20, 512, seed=93)
    for S in (1, 2, 20):
        err = _check_forward(L, O, x[:S], f"S={S}")
        say(f"  S={S}: rel L2 {err:.2e}")


def test_bf16_router_chain_vs_oracle(gpu, oracle_lib):
    """A chain of three BF16-router layers (the three-kernel decode, not the
    one-launch one) against the oracle's own chain, at S = 1."""
    say("bf16 router chain")
    hosts = [synth.with_native(synth.make_layer(512, 16, 4, 256, 0, True, seed=71 + l), seed=0) for l in range(3)]
    chain_vs_oracle(oracle_lib, hosts, 4100, 1, tokens=3, seed=5, label="bf16 router")
    assert _lib.hip().colizig_hip_fused_decode_active(4100, 3, 1) == 0


@pytest.mark.parametrize("shared", ["bf16", "f32"])
def test_native_qwen4_shapes(gpu, oracle_lib, shared):
    """Qwen4-Exp-style shapes (hidden 4096, 512 experts, top-10, inter 512,
    shared 4096): GPU-generated experts read back for the oracle, a BF16
    router and a NativeMatrix shared expert; batch 1 and batch 32."""
    say(f"native weights qwen4 shapes, shared={shared}")
    H, E, K, I, SI = 4096, 512, 10, 512, 4096
    d = moe.dims(H, E, K, I, SI)
    lid = 4200 + (0 if shared == "bf16" else 1)
    L = moe.Layer.load(lid, d, np.zeros((E, H), np.float32))
    L.synth(seed=444)
    router = L.read_router()
    base = dict(dims=dict(hidden=H, experts=E, topk=K, inter=I, shared_inter=SI, norm_topk=1), router=router,
                experts=[L.read_expert(e) for e in range(E)], shared=None)
    host = synth.with_native(base, seed=445, shared=shared)
    L.set_router_bf16(host["router"])
    s = host["shared"]
    L.set_shared_native(s["gate"], s["up"], s["down"], s["sh_gate"])
    O = oracle_lib.OracleLayer(host)
    x = synth.hidden_states(32, H, seed=446)
    for S in (1, 32):
        err = _check_forward(L, O, x[:S], f"S={S}")
        say(f"  S={S}: rel L2 {err:.2e}")
