"""A checkpoint on disk -> HBM (colizig_amd.ingest.load_layer) -> the MoE
layer on the GPU vs the oracle on the same tensors: routing and gates
bit-exact, outputs within 1e-3 relative L2."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from colizig_amd import ingest, moe, synth
from tests.helpers import f32_bits, rel_l2

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("SI,router_dt", [(0, "BF16"), (512, "F32")])
def test_layer_from_safetensors(gpu, oracle_lib, tmp_path, SI, router_dt):
    say(f"ingest SI={SI} router {router_dt}")
    H, E, K, I = 512, 16, 4, 256
    host = synth.make_layer(H, E, K, I, SI, True, seed=31 + SI)
    if router_dt == "BF16":  # a BF16 router: the oracle sees the same widened values
        bits = (host["router"].view(np.uint32) >> 16).astype(np.uint16)
        host["router"] = (bits.astype(np.uint32) << 16).view(np.float32)
        rt = ("BF16", bits)
    else:
        rt = ("F32", host["router"])
    t = {"model.layers.5.mlp.gate.weight": rt}
    for e, ex in enumerate(host["experts"]):
        for proj, k in (("gate_proj", "gate"), ("up_proj", "up"), ("down_proj", "down")):
            t[f"model.layers.5.mlp.experts.{e}.{proj}.weight"] = ("F8_E4M3", ex[f"{k}_w"])
            t[f"model.layers.5.mlp.experts.{e}.{proj}.weight_scale_inv"] = ("F32", ex[f"{k}_s"])
    if SI:
        sh = host["shared"]
        for proj, k in (("gate_proj", "gate"), ("up_proj", "up"), ("down_proj", "down")):
            t[f"model.layers.5.mlp.shared_expert.{proj}.weight"] = ("F8_E4M3", sh[f"{k}_w"])
            t[f"model.layers.5.mlp.shared_expert.{proj}.weight_scale_inv"] = ("F32", sh[f"{k}_s"])
        t["model.layers.5.mlp.shared_expert_gate.weight"] = ("F32", sh["sh_gate"].reshape(1, H))
    path = str(tmp_path / "layer5.safetensors")
    ingest.write_safetensors(path, t)
    L = ingest.load_layer(ingest.Checkpoint(path), 5, moe.dims(H, E, K, I, SI), layer_id=2500 + SI)
    Lo = oracle_lib.OracleLayer(host)
    for S in (1, 24):
        x = synth.hidden_states(S, H, seed=S)
        out, idx, gates = L.forward(x)
        ro, ri, rg = Lo.forward(x)
        assert np.array_equal(idx, ri), f"S={S}: routing differs"
        assert np.array_equal(f32_bits(gates), f32_bits(rg)), f"S={S}: gates differ"
        err = rel_l2(out, ro)
        say(f"  S={S}: rel L2 {err:.2e}")
        assert err < 1e-3
