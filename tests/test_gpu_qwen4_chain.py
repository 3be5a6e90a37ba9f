"""The Qwen4-Exp-style stack (hidden 4096, 512 experts top-10, inter 512,
one FP8 shared expert of 4096) at batch 1 (the three-kernel decode): two
chained layers over two tokens against the oracle's own chain from the same
x0 (routing bit-exact on the GPU's router inputs and the same picks as the
oracle chain, router inputs and residual within 1e-3, the routed-selection
counters equal to the oracle chain's picks)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from colizig_amd import _lib, moe
from tests.test_gpu_chain import chain_vs_oracle, say

pytestmark = pytest.mark.gpu

H, E, K, I, SI = 4096, 512, 10, 512, 4096


def _host(L: moe.Layer) -> dict:
    """A GPU-generated layer copied back in the oracle's layout."""
    nb = moe.nblk
    mat, nsc = I * H, nb(I) * nb(H)
    ew = np.empty(E * 3 * mat, np.uint8)
    es = np.empty(E * 3 * nsc, np.float32)
    assert _lib.hip().colizig_hip_expert_slab_read(L.layer, ew.ctypes.data_as(ctypes.c_void_p),
                                                   es.ctypes.data_as(ctypes.c_void_p)) == 0
    ew = ew.reshape(E, 3, mat)
    es = es.reshape(E, 3, nsc)
    experts = [dict(gate_w=ew[e, 0].reshape(I, H), gate_s=es[e, 0].reshape(nb(I), nb(H)),
                    up_w=ew[e, 1].reshape(I, H), up_s=es[e, 1].reshape(nb(I), nb(H)),
                    down_w=ew[e, 2].reshape(H, I), down_s=es[e, 2].reshape(nb(H), nb(I))) for e in range(E)]
    return dict(dims=dict(hidden=H, experts=E, topk=K, inter=I, shared_inter=SI, norm_topk=1),
                router=L.read_router(), experts=experts, shared=L.read_shared(), registered=L)


@pytest.fixture(scope="module")
def qwen4_layers(gpu):
    d = moe.dims(H, E, K, I, SI, True)
    layers = []
    for l in range(2):
        L = moe.Layer.load(3100 + l, d, np.zeros((E, H), np.float32))
        L.synth(seed=4100 + l)
        layers.append(L)
    return [_host(L) for L in layers]


def test_qwen4_chain_vs_oracle_chain(oracle_lib, qwen4_layers):
    say("qwen4 chain vs oracle chain, 2 layers, batch 1")
    chain_vs_oracle(oracle_lib, qwen4_layers, 3100, 1, tokens=2, seed=41, label="qwen4")
