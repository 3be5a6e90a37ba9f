"""The expert-streaming tier at the Qwen3-30B-A3B expert shapes (hidden
2048, 128 experts, top-8, inter 768): 4 streamed layers whose experts sit in
pinned host memory (packed slabs, one copy per fill), an HBM pool of 64
slots (the working set is 512 experts), routing Zipf(1.2)-skewed over a
seeded permutation per layer with 10% of the experts swapping ranks after
every step, 32 decode steps at batch 1.  Two routing-prediction modes:
both predictions (next layer, and every later layer from the token's first
router input), and the token-level one with the later layers run with the
host off their path (speculative runs: a pick without a slot stops the run,
that layer goes through the per-layer path, and a new run follows).

Against the oracle:
- every layer's demand gets (its picks, in pick order, repeats dropped)
  equal the picks of the oracle's own chain run from the same x0;
- the residual stream after every step is within 1e-3 relative L2;
- the pool's op log replayed by the oracle's restatement of the cache
  policy (czo_pool_replay: ExpertCache, moe.zig:141-249, over (layer,
  expert) keys with the in-flight layer's slots pinned) gives the same slot
  for every op and the same counters as the library's.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from colizig_amd import _lib, moe, synth
from tests.helpers import rel_l2

pytestmark = pytest.mark.gpu

H, E, K, I = 2048, 128, 8, 768
NL, NSLOTS, STEPS, BASE = 4, 64, 32, 3100
ZIPF_S, DRIFT = 1.2, 0.1
EPS = 1e-6


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def zipf_bias(ranks: np.ndarray) -> np.ndarray:
    lp = -ZIPF_S * np.log(ranks.astype(np.float64) + 1.0)
    return (lp - lp.mean()).astype(np.float32)


def host_layer(L: moe.Layer, d: moe.Dims, bias: np.ndarray):
    """The layer's weights read back from HBM: the oracle's layer dict and
    the packed pinned host slab the stream reads."""
    mat, nsc = I * H, moe.nblk(I) * moe.nblk(H)
    ew = np.empty(E * 3 * mat, np.uint8)
    es = np.empty(E * 3 * nsc, np.float32)
    assert _lib.hip().colizig_hip_expert_slab_read(L.layer, ew.ctypes.data, es.ctypes.data) == 0
    ew3, es3 = ew.reshape(E, 3, mat), es.reshape(E, 3, nsc)
    experts = [dict(gate_w=ew3[e, 0].reshape(I, H), gate_s=es3[e, 0].reshape(moe.nblk(I), moe.nblk(H)),
                    up_w=ew3[e, 1].reshape(I, H), up_s=es3[e, 1].reshape(moe.nblk(I), moe.nblk(H)),
                    down_w=ew3[e, 2].reshape(H, I), down_s=es3[e, 2].reshape(moe.nblk(H), moe.nblk(I)))
               for e in range(E)]
    host = dict(dims=dict(hidden=H, experts=E, topk=K, inter=I, shared_inter=0, norm_topk=1),
                router=L.read_router(), experts=experts, shared=None, router_bias=bias.copy(), _keep=(ew, es))
    packed = moe.host_expert_slab_packed(d, ew3.reshape(E, -1), es3.reshape(E, -1))
    return host, packed


@pytest.fixture(scope="module", params=[3, 6], ids=["predict3", "predict6_speculative"])
def c5(gpu, oracle_lib, request):
    d = moe.dims(H, E, K, I)
    moe.stream_pool_init(d, NSLOTS * moe.packed_expert_bytes(d))
    assert moe.stream_stats()["slots"] == NSLOTS
    hip = _lib.hip()
    hip.colizig_hip_stream_log(1)
    rng = np.random.default_rng(2025)
    ranks = [rng.permutation(E) for _ in range(NL)]
    hosts, packs, layers = [], [], []
    for l in range(NL):
        L = moe.Layer.load(BASE + l, d, np.zeros((E, H), np.float32))
        L.synth(seed=777 + l)
        bias = zipf_bias(ranks[l])
        L.set_router_bias(bias)
        host, packed = host_layer(L, d, bias)
        moe.stream_layer_from_host_packed(BASE + l, packed)
        hosts.append(host)
        packs.append(packed)
        layers.append(L)
    prev = hip.colizig_hip_stream_set_predict(request.param)
    yield dict(d=d, hosts=hosts, packs=packs, layers=layers, ranks=ranks, rng=rng, mode=request.param)
    hip.colizig_hip_stream_set_predict(prev)
    hip.colizig_hip_stream_log(0)
    moe.stream_pool_free()
    for p in packs:
        p.free()


def test_c5_stream_vs_oracle_chain_and_policy(c5, oracle_lib):
    mode = c5["mode"]
    say(f"c5: 4 streamed layers, 64-slot pool, Zipf(1.2) with 10% drift, 32 steps, prediction mode {mode}")
    hip = _lib.hip()
    orcs = [oracle_lib.OracleLayer(h) for h in c5["hosts"]]
    rng, ranks = c5["rng"], c5["ranks"]
    x0 = synth.hidden_states(1, H, seed=55)
    xb = moe.DeviceBuffer(x0.nbytes)
    xb.upload(x0)
    xo = x0.copy()
    worst = 0.0
    picks_o = []
    for t in range(STEPS):
        rc = hip.colizig_hip_stream_decode(BASE, NL, xb.ptr, 1, EPS)
        assert rc == 0, _lib.last_error()
        assert hip.colizig_hip_sync() == 0, _lib.last_error()
        for l in range(NL):
            _, idx_o, _ = orcs[l].chain(xo, EPS)
            sel = []
            for e in idx_o[0].tolist():
                if e not in sel:
                    sel.append(e)
            picks_o.append((BASE + l, sel))
        x_g = xb.download(np.empty_like(x0))
        err = rel_l2(x_g, xo)
        worst = max(worst, err)
        assert err < 1e-3, f"step {t}: residual stream rel L2 {err:.2e}"
        for l in range(NL):  # drift: 10% of the experts swap ranks
            pick = rng.choice(E, size=int(E * DRIFT), replace=False)
            ranks[l][pick] = ranks[l][rng.permutation(pick)]
            bias = zipf_bias(ranks[l])
            c5["layers"][l].set_router_bias(bias)
            orcs[l].router_bias[:] = bias
        if t % 8 == 0:
            say(f"  step {t}: x rel L2 {err:.2e}")
    xb.free()

    ops = moe.stream_log_read()
    # demand gets, grouped by layer epoch, against the oracle chain's picks
    got = []
    for op, layer, e, _ in ops.tolist():
        if op == 0:
            got.append((layer, []))
        elif op == 1:
            got[-1][1].append(e)
    assert len(got) == STEPS * NL
    for i, (a, b) in enumerate(zip(got, picks_o)):
        assert a == b, f"layer step {i}: demand gets {a} vs oracle picks {b}"

    r, res, st = oracle_lib.pool_replay(NSLOTS, ops)
    assert r >= 0
    assert np.array_equal(res, ops[:, 3]), "pool policy: slot decisions differ from the oracle's replay"
    lib_st = moe.stream_stats()
    for k, v in st.items():
        assert lib_st[k] == v, (k, lib_st[k], v)
    assert lib_st["resident"] == r
    assert lib_st["hits"] + lib_st["misses"] == sum(len(s) for _, s in picks_o)
    # every layer but the first of each step
    assert lib_st["next_predicted"] == ((STEPS * NL - STEPS) * K if mode & 1 else 0)
    assert lib_st["tok_predicted"] == (STEPS * NL - STEPS) * K
    if mode & 4:  # speculative runs ran layers, and missing slots stopped some (their layers re-ran above)
        assert lib_st["spec_layers"] > 0 and lib_st["spec_stops"] > 0, lib_st
        assert lib_st["spec_layers"] + lib_st["spec_stops"] <= STEPS * (NL - 1)
        say(f"  speculative: {lib_st['spec_layers']} layers ran, {lib_st['spec_stops']} runs stopped")
    else:
        assert lib_st["spec_layers"] == 0
    acc = lib_st["next_correct"] / max(lib_st["next_predicted"], 1)
    say(f"  x rel L2 <= {worst:.2e}; {len(ops)} pool ops replayed; hits {lib_st['hits']} misses "
        f"{lib_st['misses']} evictions {lib_st['evictions']}; prefetch issued {lib_st['prefetch_issued']} hits "
        f"{lib_st['prefetch_hits']} wasted {lib_st['prefetch_wasted']}; next-layer prediction {acc:.3f}")
    assert lib_st["prefetch_hits"] > 0
