#!/usr/bin/env python3
"""Benchmark: colizig's MoE expert path, Qwen3-30B-A3B decode shape, 1 MI355X.

Workload (one "step" = one decode token through all layers):
  48 MoE layers, hidden 2048, 128 experts, top-8 renormalised, no shared
  expert, moe_intermediate 768; block-FP8 E4M3 expert weights N(0,0.02) with
  128x128 f32 scales and an f32 N(0,0.02) router, all resident in HBM (29 GB),
  generated on the GPU from a seed; batch 1, hidden state N(0,1).  Layers are
  chained x <- x + MoE_l(rmsnorm(x)) so every layer depends on the previous.
The timed region replays a HIP graph of one step K times, inputs already in
HBM.  At batch 1 every layer is one kernel launch (router, routing, gate/up,
SiLU, down and combine); a second graph of the layer launches alone, timed
with events on the library stream, gives that kernel's mean duration, the
roofline kernel's.  The parity line runs the oracle's own chain from the same
x0 over the first layers.  The CPU baseline runs the oracle (the C
restatement of the reference's CPU SIMD path, threaded like its
parallel.chunks) on the same weights copied to host memory, for a bounded
number of tokens.

    python bench.py [--steps 256] [--warmup 10] [--cpu-seconds 15] [--no-cpu]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published

# HBM bytes per launch of the one-launch layer kernel on this workload,
# measured with rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE and scaled by
# what the same counters read for a plain 256 MiB copy (FETCH_SIZE x 2.0,
# WRITE_SIZE x 1.0): 24430.4 KiB fetched, 134.5 KiB written per dispatch
# (the mean over a step's 47 launches with predicted experts and its first).
LAYER_TRAFFIC_BYTES = int(round((24430.4 * 2.0 + 134.5) * 1024))

# HBM bytes per 512-token prefill step (48 layers: router, routing, dispatch,
# the two grouped GEMMs and the combine, which forms the next layer's RMS
# rows in 47 of them; the first layer's RMS rows), measured the same way:
# 12057994.9 KiB fetched and 2593636.8 KiB written per step, the sums of the
# kernels' per-dispatch means.
PREFILL_STEP_TRAFFIC_BYTES = int(round((12057994.9 * 2.0 + 2593636.8) * 1024))

CONFIG = dict(workload="qwen3-30b-a3b-moe-decode", layers=48, hidden=2048, experts=128, topk=8, inter=768,
              shared_inter=0, norm_topk=1, batch=1, weights="block-fp8-e4m3-128x128", seed=0)


def nblk(x):
    return (x + 127) // 128


def per_token_bytes(c) -> dict:
    """Algorithmic HBM bytes per token per layer (weights + scales of the K
    selected experts, the router, activations)."""
    H, I, E, K = c["hidden"], c["inter"], c["experts"], c["topk"]
    mat = H * I
    sc_up = nblk(I) * nblk(H) * 4
    up = K * 2 * (mat + sc_up)            # gate + up weights and scales
    down = K * (mat + nblk(H) * nblk(I) * 4)
    router = E * H * 4
    act = (2 * H + 2 * K * I) * 4
    return dict(up=up, down=down, router=router, act=act, total=up + down + router + act)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default 256; 512 for --workload stream, config 5's length)")
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=CONFIG["layers"])
    ap.add_argument("--profile-steps", type=int, default=32)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--parity-layers", type=int, default=48,
                    help="decode: layers of the parity check against the oracle's own chain (one token)")
    ap.add_argument("--workload", choices=["decode", "prefill", "stream", "qwen4", "attn", "lmhead", "dropin",
                                           "microbench"],
                    default="decode",
                    help="decode: the 48-layer batch-1 decode line (default); prefill: 48 layers x "
                         "512 tokens with Zipf(1.1) routing skew (grouped regime); stream: batch-1 decode "
                         "with the expert set in pinned host memory and a 16 GB HBM expert pool; qwen4: "
                         "Qwen4-Exp-style stack (36 layers, H4096, E512 top-10, shared 4096) at batch 1 and 32; "
                         "attn: the FP8 attention projections q/k/v/o of 48 Qwen3-30B-A3B layers at batch 1 "
                         "(keyed device GEMV); lmhead: the BF16 lm_head GEMV (151936 x 2048) at batch 1, "
                         "dotBf16 order; dropin: the unchanged engine's per-matmul calls (colizig_cuda_matmul_fp8 "
                         "on host buffers, keyed hits) at the Qwen3-30B-A3B expert and attention shapes")
    ap.add_argument("--pool-gb", type=float, default=16.0, help="stream: HBM expert pool cap (GB)")
    ap.add_argument("--priors", action="store_true",
                    help="stream: warm the pool from learned priors (.colizig_usage written by an untimed "
                         "previous session of --steps tokens on the same workload) before the timed tokens")
    ap.add_argument("--predict", type=int, default=6, choices=list(range(8)),
                    help="stream: routing prediction for prefetch (bit 0: next layer from the current layer's "
                         "router input; bit 1: every later layer from the token's first router input; bit 2, "
                         "with bit 1: the later layers enqueued at once, the host off their path); 0: only "
                         "the last token's routing")
    ap.add_argument("--split-slabs", action="store_true",
                    help="stream: weights and scales in two host slabs (two copies per fill) instead of one packed slab")
    ap.add_argument("--fused-predict", type=int, default=None, choices=[0, 1],
                    help="decode: request each layer's predicted experts before its routing (1, the library's "
                         "default) or after it (0)")
    ap.add_argument("--attn-separate", action="store_true",
                    help="attn: q, k and v as three launches (the reference's three calls) instead of one")
    ap.add_argument("--tokens", type=int, default=512, help="prefill tokens per step")
    ap.add_argument("--prefill-mfma", choices=["f16", "fp8"], default=None,
                    help="prefill/qwen4: the grouped GEMMs on f16 MFMA (weights widened, activations f16 hi + lo) "
                         "or FP8 MFMA (E4M3 weights, activations as three E4M3 terms); default: the library's")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB (HBM counter calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (--gpus must be 1)", file=sys.stderr)
        sys.exit(2)

    if args.steps is None:
        args.steps = 512 if args.workload == "stream" else 256
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
        return
    if args.workload == "prefill":
        prefill_bench(args)
        return
    if args.workload == "stream":
        stream_bench(args)
        return
    if args.workload == "qwen4":
        qwen4_bench(args)
        return
    if args.workload == "attn":
        attn_bench(args)
        return
    if args.workload == "lmhead":
        lmhead_bench(args)
        return
    if args.workload == "microbench":
        microbench(args)
        return
    if args.workload == "dropin":
        dropin_bench(args)
        return

    from colizig_amd import _lib, moe

    c = dict(CONFIG)
    c["layers"] = args.layers
    H, E, K, I, NL = c["hidden"], c["experts"], c["topk"], c["inter"], c["layers"]
    name = moe.init()
    log(f"device: {name}")
    hip = _lib.hip()
    if args.fused_predict is not None:
        hip.colizig_hip_set_fused_predict(args.fused_predict)
    predict = hip.colizig_hip_set_fused_predict(0)
    hip.colizig_hip_set_fused_predict(predict)
    c["expert_prediction"] = "next layer's top-k on this layer's router input" if predict else "off"
    d = moe.dims(H, E, K, I, 0, True)
    t0 = time.time()
    layers = []
    zero_router = np.zeros((E, H), np.float32)
    for l in range(NL):
        L = moe.Layer.load(l, d, zero_router)
        L.synth(seed=c["seed"] * 1000003 + l)
        layers.append(L)
    log(f"weights generated in HBM: {NL} layers in {time.time() - t0:.1f}s")

    x0 = np.random.default_rng(c["seed"]).normal(0.0, 1.0, size=(1, H)).astype(np.float32)
    xb = moe.DeviceBuffer(x0.nbytes)
    xb.upload(x0)
    eps = 1e-6
    gh = hip.colizig_hip_chain_graph_create(0, NL, xb.ptr, 1, eps)
    if gh <= 0:
        raise RuntimeError(f"graph capture failed: {_lib.last_error()}")

    # warmup
    for _ in range(args.warmup):
        assert hip.colizig_hip_graph_launch(gh, None) == 0
    assert hip.colizig_hip_sync() == 0

    # timed region: K steps, synchronised on both sides
    ev0, ev1 = hip.colizig_hip_event_create(), hip.colizig_hip_event_create()
    pst = np.zeros(2, np.uint64)
    hip.colizig_hip_fused_predict_stats(pst.ctypes.data)  # zeroes the prediction counters
    assert hip.colizig_hip_sync() == 0
    w0 = time.perf_counter()
    hip.colizig_hip_event_record(ev0, None)
    for _ in range(args.steps):
        hip.colizig_hip_graph_launch(gh, None)
    hip.colizig_hip_event_record(ev1, None)
    assert hip.colizig_hip_sync() == 0
    wall = time.perf_counter() - w0
    ms_total = hip.colizig_hip_event_elapsed_ms(ev0, ev1)
    ms_per_step = ms_total / args.steps
    tok_s = 1000.0 / ms_per_step
    log(f"timed: {args.steps} steps, {ms_per_step * 1000:.1f} us/token, {tok_s:.1f} tok/s (wall {wall:.3f}s)")
    pred_rate = None
    if hip.colizig_hip_fused_predict_stats(pst.ctypes.data) == 0 and pst[0] > 0:
        pred_rate = round(float(pst[1]) / float(pst[0]), 4)
        log(f"predicted experts picked: {int(pst[1])} of {int(pst[0])} ({pred_rate:.3f})")

    # the layer kernel's duration: a HIP graph of the layer launches replayed
    # between two events on the library stream (minus the chain's final
    # residual kernel, timed alone the same way)
    if hip.colizig_hip_fused_decode_active(0, NL, 1) != 1:
        raise RuntimeError("the batch-1 chain is not served by the one-launch layer kernel")
    us2 = (ctypes.c_float * 2)()
    rc = hip.colizig_hip_chain_fused_times(0, NL, xb.ptr, eps, args.profile_steps, us2)
    if rc != 0:
        raise RuntimeError(f"kernel timing pass failed: {_lib.last_error()}")
    layer_us, final_us = float(us2[0]), float(us2[1])
    b = per_token_bytes(c)
    layer_bytes = b["total"]
    layer_gbs = layer_bytes / (layer_us * 1e-6) / 1e9
    tok_bytes = NL * b["total"]
    log(f"kernels: layer {layer_us:.2f} us ({layer_gbs:.0f} GB/s of {layer_bytes} algorithmic bytes), "
        f"final residual {final_us:.2f} us")

    # host copies of the layers for the oracle (parity and CPU baseline)
    hosts, copy_s = None, 0.0
    if args.parity_layers > 0 or not args.no_cpu:
        from oracle import oracle as orc
        t1 = time.time()
        n_host = NL if not args.no_cpu else min(args.parity_layers, NL)
        hosts = [orc.OracleLayer(host_layer(hip, L, c)) for L in layers[:n_host]]
        copy_s = time.time() - t1
    # parity: the oracle's own chain from the same x0 over the first layers
    parity = None
    if args.parity_layers > 0:
        parity = parity_check(hip, moe, hosts[:min(args.parity_layers, NL)], x0, c, eps)
        log(f"parity: {parity}")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(hosts, x0, eps, args.cpu_seconds, copy_s)
        log(f"cpu baseline: {cpu}")

    line = {
        "metric": "MoE decode tok/s + achieved HBM GB/s, Qwen3-30B-A3B shape, 1 MI355X",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e4m3-weights/f32-accumulate",
        "data": "synthetic (seeded N(0,0.02) weights generated in HBM, N(0,1) hidden state)",
        "config": {**c, "parallelism": "none (1 GPU)", "global_batch": 1, "seq_len": 1},
        "step_hbm_gbs": round(tok_bytes * tok_s / 1e9, 1),
        "step_hbm_frac": round(tok_bytes * tok_s / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": {
            "bound": "hbm",
            "kernel": "k_layer_fused (one MoE layer: rmsnorm, router, top-8, gate/up, SiLU, down, combine)",
            "achieved": round(layer_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(layer_gbs / HBM_PEAK_GBS, 4),
            "traffic": LAYER_TRAFFIC_BYTES,
            "bytes_per_launch": layer_bytes,
            "avg_launch_us": round(layer_us, 3),
        },
        "kernels_us": {"layer": round(layer_us, 3), "final_residual": round(final_us, 3)},
        "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / tok_bytes, 1),
        "expert_prediction_hit_rate": pred_rate,
        "parity": parity,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def prefill_bench(args) -> None:
    """Qwen3-30B-A3B MoE shapes at prefill: 48 chained layers, `tokens` tokens
    per step, each layer's routing skewed Zipf(1.1) by a per-expert logit bias
    over a seeded permutation.  Runs the grouped regime (dispatch + grouped
    MFMA GEMMs).  Algorithmic bytes per step: every expert a layer's routing
    touches, read once, + routers + activations."""
    from colizig_amd import _lib, moe, synth
    c = dict(CONFIG)
    c.update(workload="qwen3-30b-a3b-moe-prefill-zipf1.1", batch=args.tokens, zipf_s=1.1)
    c["layers"] = args.layers
    H, E, K, I, NL, S = c["hidden"], c["experts"], c["topk"], c["inter"], c["layers"], args.tokens
    name = moe.init()
    log(f"device: {name}")
    hip = _lib.hip()
    if args.prefill_mfma:
        hip.colizig_hip_set_prefill_fp8(1 if args.prefill_mfma == "fp8" else 0)
    fp8 = hip.colizig_hip_set_prefill_fp8(0) == 1
    hip.colizig_hip_set_prefill_fp8(1 if fp8 else 0)
    c["mfma"] = "fp8 (v_mfma_scale_f32_32x32x64_f8f6f4, activations as 3 E4M3 terms)" if fp8 else \
        "f16 (v_mfma_f32_32x32x16_f16, activations as f16 hi + lo)"
    d = moe.dims(H, E, K, I, 0, True)
    zero_router = np.zeros((E, H), np.float32)
    for l in range(NL):
        L = moe.Layer.load(l, d, zero_router)
        L.synth(seed=c["seed"] * 1000003 + l)
        L.set_router_bias(synth.zipf_router_bias(E, 1.1, seed=7919 * l + 1))
    x0 = np.random.default_rng(c["seed"]).normal(0.0, 1.0, size=(S, H)).astype(np.float32)
    xb = moe.DeviceBuffer(x0.nbytes)
    eps = 1e-6
    # one traced pass: the experts each layer touches
    idx_t = moe.DeviceBuffer(NL * S * K * 4)
    xb.upload(x0)
    assert hip.colizig_hip_chain_decode(0, NL, xb.ptr, S, eps, None, idx_t.ptr, None, None) == 0, _lib.last_error()
    assert hip.colizig_hip_sync() == 0
    idx = idx_t.download(np.empty((NL, S, K), np.uint32))
    touched = [int(np.unique(idx[l]).size) for l in range(NL)]
    hottest = [int(np.bincount(idx[l].ravel(), minlength=E).max()) for l in range(NL)]
    per_expert = 3 * H * I + 4 * (2 * nblk(I) * nblk(H) + nblk(H) * nblk(I))
    step_bytes = sum(t * per_expert for t in touched) + NL * (E * H * 4 + 2 * S * H * 4)
    step_flops = NL * S * K * 2 * 3 * H * I
    xb.upload(x0)
    gh = hip.colizig_hip_chain_graph_create(0, NL, xb.ptr, S, eps)
    if gh <= 0:
        raise RuntimeError(f"graph capture failed: {_lib.last_error()}")
    for _ in range(args.warmup):
        assert hip.colizig_hip_graph_launch(gh, None) == 0
    assert hip.colizig_hip_sync() == 0
    ev0, ev1 = hip.colizig_hip_event_create(), hip.colizig_hip_event_create()
    hip.colizig_hip_event_record(ev0, None)
    for _ in range(args.steps):
        hip.colizig_hip_graph_launch(gh, None)
    hip.colizig_hip_event_record(ev1, None)
    assert hip.colizig_hip_sync() == 0
    ms = hip.colizig_hip_event_elapsed_ms(ev0, ev1) / args.steps
    tok_s = S * 1000.0 / ms
    gbs = step_bytes / (ms * 1e-3) / 1e9
    log(f"prefill: {S} tokens x {NL} layers in {ms:.3f} ms ({tok_s:.0f} tok/s); experts touched per layer "
        f"{min(touched)}..{max(touched)}, hottest expert {max(hottest)} of {S} tokens; {gbs:.0f} GB/s; "
        f"{step_flops / (ms * 1e-3) / 1e12:.1f} TFLOP/s")
    # token independence at the full size (after the timed region): the MoE
    # treats tokens independently (per-row activation terms, per-row GEMM
    # sums, each token's combine in its pick order), so the first 64 tokens
    # through the 48 layers on their own (still the grouped regime) must get
    # the bits they got inside the whole step
    parity = None
    if args.parity_layers > 0 and S > 64:
        P = 64
        xa, xp = moe.DeviceBuffer(x0.nbytes), moe.DeviceBuffer(P * H * 4)
        xa.upload(x0)
        xp.upload(np.ascontiguousarray(x0[:P]))
        if hip.colizig_hip_chain_decode(0, NL, xa.ptr, S, eps, None, None, None, None) != 0 or \
                hip.colizig_hip_chain_decode(0, NL, xp.ptr, P, eps, None, None, None, None) != 0:
            raise RuntimeError(f"parity pass failed: {_lib.last_error()}")
        assert hip.colizig_hip_sync() == 0
        a = xa.download(np.empty_like(x0))[:P]
        b = xp.download(np.empty((P, H), np.float32))
        parity = {"property": f"the first {P} tokens through the {NL} layers alone vs inside the {S}-token step",
                  "bit_identical": bool(np.array_equal(a.view(np.uint32), b.view(np.uint32))),
                  "max_abs_diff": float(np.max(np.abs(a - b)))}
        xa.free()
        xp.free()
        log(f"parity: {parity}")
    # the oracle's own chain from the same x0 over all the layers, on the
    # first 64 tokens (tokens are independent, so their rows of the 512-token
    # step are what the oracle's chain of those tokens alone gives), for the
    # FP8 and the f16 GEMM operands; its timing is the line's CPU baseline
    cpu = None
    if args.parity_layers > 0 and S > 64:
        biases = [synth.zipf_router_bias(E, 1.1, seed=7919 * l + 1) for l in range(NL)]
        layers = [moe.Layer(l, d) for l in range(NL)]
        res, cpu = prefill_oracle_parity(hip, moe, layers, biases, x0, c, eps, 64, 1 if fp8 else 0)
        parity = {"token_independence": parity, "oracle_chain": res}
        log(f"parity vs oracle chain: {res}")
        log(f"cpu baseline: {cpu}")
    line = {
        "metric": "MoE prefill tok/s (512-token step, Zipf(1.1) routing), Qwen3-30B-A3B shape, 1 MI355X",
        "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "e4m3-weights/e4m3x3-activations/f32-accumulate" if fp8 else "e4m3-weights/f16x2-activations/f32-accumulate",
        "data": "synthetic (seeded N(0,0.02) weights generated in HBM, N(0,1) hidden states)",
        "config": {**c, "parallelism": "none (1 GPU)", "global_batch": S, "seq_len": S},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": PREFILL_STEP_TRAFFIC_BYTES if (S == 512 and NL == 48) else None,
                     "scope": "whole step", "bytes_per_step": step_bytes},
        "mfma_tflops": round(step_flops / (ms * 1e-3) / 1e12, 2),
        # useful FLOPs / step time against the dense peak of the MFMA in use
        # (FP8 5.0 PFLOP/s, f16 2.5 PFLOP/s; the activation terms multiply the work done)
        "mfma_peak_tflops": 5000.0 if fp8 else 2500.0,
        "mfma_frac": round(step_flops / (ms * 1e-3) / 1e12 / (5000.0 if fp8 else 2500.0), 4),
        "experts_touched_per_layer": [min(touched), max(touched)],
        "parity": parity,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def prefill_oracle_parity(hip, moe, layers, biases, x0, c, eps, P, mode):
    """The 48-layer prefill chain on the GPU (S = len(x0) tokens, in each
    grouped-GEMM mode: the library's current one and f16) against the
    oracle's own chain of the first P tokens from the same x0, layer by layer
    (each layer's weights copied back, checked and dropped): routing bit-exact
    on the GPU's own router inputs and the same picks as the oracle's chain,
    the near-tie census of the oracle's decisions, router inputs and the
    final residual stream within 1e-3 relative L2.  Returns the result per
    mode and the oracle's timing as the CPU baseline (P tokens x all layers
    on the host cores)."""
    from oracle import oracle as orc
    S, H = x0.shape
    K = c["topk"]
    NL = len(layers)
    present = len(os.sched_getaffinity(0))
    threads = min(present, 16)
    orc.lib().czo_parallel_enable(threads)
    modes = [mode, 0] if mode != 0 else [0]
    gpu = {}
    for m in modes:
        hip.colizig_hip_set_prefill_fp8(m)
        xb = moe.DeviceBuffer(x0.nbytes)
        xn_t = moe.DeviceBuffer(NL * S * H * 4)
        idx_t = moe.DeviceBuffer(NL * S * K * 4)
        g_t = moe.DeviceBuffer(NL * S * K * 4)
        xb.upload(x0)
        if hip.colizig_hip_chain_decode(0, NL, xb.ptr, S, eps, xn_t.ptr, idx_t.ptr, g_t.ptr, None) != 0 or \
                hip.colizig_hip_sync() != 0:
            raise RuntimeError(f"prefill parity pass failed: {_lib_err()}")
        gpu[m] = dict(x=xb.download(np.empty_like(x0))[:P].copy(),
                      xn=xn_t.download(np.empty((NL, S, H), np.float32))[:, :P].copy(),
                      idx=idx_t.download(np.empty((NL, S, K), np.uint32))[:, :P].copy(),
                      gates=g_t.download(np.empty((NL, S, K), np.float32))[:, :P].copy())
        for b in (xb, xn_t, idx_t, g_t):
            b.free()
    hip.colizig_hip_set_prefill_fp8(mode)
    xo = np.ascontiguousarray(x0[:P]).copy()
    acc = {m: dict(exact=True, worst_xn=0.0) for m in modes}
    min_gap, oracle_s = 1 << 30, 0.0
    for l, L in enumerate(layers):
        host = host_layer(hip, L, c)
        host["router_bias"] = biases[l]
        O = orc.OracleLayer(host)
        t0 = time.perf_counter()
        xn_o, idx_o, _ = O.chain(xo, eps)
        oracle_s += time.perf_counter() - t0
        for t in range(P):  # route() takes one row
            _, _, v = O.route(xn_o[t])
            top = sorted(range(v.size), key=lambda e: (-float(v[e]), e))[:K + 1]
            b = v[top].view(np.uint32).astype(np.int64)
            min_gap = min(min_gap, int(np.min(b[:-1] - b[1:])))
        for m in modes:
            G = gpu[m]
            a = acc[m]
            a["worst_xn"] = max(a["worst_xn"], float(np.linalg.norm(G["xn"][l] - xn_o) / np.linalg.norm(xn_o)))
            for t in range(P):
                ri, rg, _ = O.route(G["xn"][l, t])
                a["exact"] &= bool(np.array_equal(ri, G["idx"][l, t]) and
                                   np.array_equal(rg.view(np.uint32), G["gates"][l, t].view(np.uint32)))
            a["exact"] &= bool(np.array_equal(G["idx"][l], idx_o))
        del O, host
    names = {0: "f16", 1: "fp8", 2: "fp8"}
    res = {"layers_checked": NL, "tokens_checked": P, "reference": f"oracle chain of the first {P} tokens from the same x0",
           "tolerance": 1e-3, "near_tie_min_gap_ulps": min_gap}
    for m in modes:
        res[names[m]] = {"routing_bit_exact": acc[m]["exact"], "max_router_input_rel_l2": acc[m]["worst_xn"],
                         "residual_rel_l2": float(np.linalg.norm(gpu[m]["x"] - xo) / np.linalg.norm(xo))}
    cpu = {"value": round(P / oracle_s, 2), "unit": "tok/s", "cores": threads, "kind": "port",
           "sample": f"the oracle's chain (cz_oracle.c, the reference's CPU SIMD path restated) of {P} of the "
                     f"{S} tokens through all {NL} layers, {oracle_s:.1f} s; host {cpu_model()}"}
    return res, cpu


def _lib_err() -> str:
    from colizig_amd import _lib
    return _lib.last_error()


def stream_bench(args) -> None:
    """Expert-streaming tier on the Qwen3-30B-A3B shapes: the full block-FP8
    expert set (48 x 128 experts, 29 GB) in pinned host memory, an HBM expert
    pool capped at --pool-gb, batch-1 decode over 48 chained layers whose
    routing is Zipf(1.2)-skewed with a 10% per-step drift of the hot ranks
    (each step a random 10% of every layer's experts swap ranks).  Reports
    tok/s, the pool's hit rate and the host->HBM rate."""
    from colizig_amd import _lib, moe, synth
    c = dict(CONFIG)
    c.update(workload="qwen3-30b-a3b-moe-decode-streamed", zipf_s=1.2, drift=0.1, pool_gb=args.pool_gb,
             routing_prediction=args.predict, host_slabs="split" if args.split_slabs else "packed")
    c["layers"] = args.layers
    H, E, K, I, NL = c["hidden"], c["experts"], c["topk"], c["inter"], c["layers"]
    steps = args.steps
    name = moe.init()
    log(f"device: {name}")
    hip = _lib.hip()
    d = moe.dims(H, E, K, I, 0, True)
    # the HBM plan for a 16 GB expert budget (budget.plan restated for HBM):
    # every layer streams through one pool of that many expert slots
    plan = moe.plan_hbm(d, NL, moe.plan_hbm(d, NL, 1 << 40)["fixed_resident"] + int(args.pool_gb * 1e9))
    assert plan["fits"] and not plan["all_resident"], plan
    moe.stream_pool_init(d, plan["expert_bytes"])
    c["hbm_plan"] = {k: plan[k] for k in ("pool_slots", "expert_cap", "ladder_cap", "fixed_resident", "total")}
    t0 = time.time()
    mat, nsc = I * H, nblk(I) * nblk(H)
    zero_router = np.zeros((E, H), np.float32)
    host = []
    for l in range(NL):
        L = moe.Layer.load(l, d, zero_router)
        L.synth(seed=c["seed"] * 1000003 + l)
        wb, sb = moe.HostBuffer(E * 3 * mat), moe.HostBuffer(E * 3 * nsc * 4)
        rc = hip.colizig_hip_expert_slab_read(l, wb.ptr, sb.ptr)
        assert rc == 0, _lib.last_error()
        if args.split_slabs:
            moe.stream_layer_from_host(l, wb, sb)
            host.append((wb, sb))
        else:
            hb = moe.host_expert_slab_packed(d, wb.view(np.uint8).reshape(E, -1), sb.view(np.float32).reshape(E, -1))
            wb.free()
            sb.free()
            moe.stream_layer_from_host_packed(l, hb)
            host.append((hb,))
    hip.colizig_hip_stream_set_predict(args.predict)
    log(f"expert set in pinned host memory: {NL * E * 3 * mat / 1e9:.1f} GB in {time.time() - t0:.1f}s; "
        f"pool {moe.stream_stats()['slots']} slots")
    # the link on its own: one 1 GiB pinned host->HBM copy
    probe = moe.HostBuffer(1 << 30)
    dprobe = moe.DeviceBuffer(1 << 30)
    hip.colizig_hip_memcpy_htod(dprobe.ptr, probe.ptr, 1 << 30)
    tl = time.perf_counter()
    hip.colizig_hip_memcpy_htod(dprobe.ptr, probe.ptr, 1 << 30)
    link_gbs = (1 << 30) / (time.perf_counter() - tl) / 1e9
    probe.free()
    dprobe.free()
    rng = np.random.default_rng(c["seed"] + 12345)
    ranks = [rng.permutation(E) for _ in range(NL)]  # ranks[l][e]: 0 = hottest

    def set_bias(l):
        lp = -1.2 * np.log(ranks[l].astype(np.float64) + 1.0)
        moe.Layer(l, d, True).set_router_bias((lp - lp.mean()).astype(np.float32))

    def drift(l):
        pick = rng.choice(E, size=max(1, E // 10), replace=False)
        ranks[l][pick] = ranks[l][rng.permutation(pick)]

    for l in range(NL):
        set_bias(l)
    x0 = np.random.default_rng(c["seed"]).normal(0.0, 1.0, size=(1, H)).astype(np.float32)
    xb = moe.DeviceBuffer(x0.nbytes)
    xb.upload(x0)
    eps = 1e-6

    def step() -> float:
        """One decode token; returns its time (the routing drift applied
        afterwards is workload bookkeeping and is not timed)."""
        ts = time.perf_counter()
        rc = hip.colizig_hip_stream_decode(0, NL, xb.ptr, 1, eps)
        if rc != 0:
            raise RuntimeError(f"stream step failed: {_lib.last_error()}")
        assert hip.colizig_hip_sync() == 0
        dt = time.perf_counter() - ts
        for l in range(NL):
            drift(l)
            set_bias(l)
        return dt

    warmed = None
    if args.priors:
        import tempfile
        from colizig_amd.usage import FILENAME, ExpertUsage
        for _ in range(steps):  # the previous session, untimed
            step()
        with tempfile.TemporaryDirectory() as td:
            path = os.path.join(td, FILENAME)
            ExpertUsage.from_pool(0, NL, E).save(path)
            prior = ExpertUsage.load(path, NL, E)
        assert prior is not None and hip.colizig_hip_stream_evict_all() == 0
        warmed = prior.warm_pool(0)
        log(f"priors: pool warmed with {warmed} experts from {int(prior.counts.sum())} routed counts")
        c["priors"] = "warm start from .colizig_usage of a previous untimed session of the same length"
    for _ in range(args.warmup):
        step()
    # the timed window's own counters: a prefetch issued in the warm-up and
    # used in the window is neither issued nor a hit here, and the queue peak
    # is the window's
    assert hip.colizig_hip_stream_stats_reset() == 0
    w0 = time.perf_counter()
    wall = sum(step() for _ in range(steps))
    harness = time.perf_counter() - w0 - wall
    s1 = moe.stream_stats()
    st = {k: s1[k] for k in s1 if k not in ("slots", "resident")}
    uses = st["hits"] + st["misses"]
    hit = st["hits"] / max(uses, 1)
    tok_s = steps / wall
    h2d_gbs = st["bytes_h2d"] / wall / 1e9
    log(f"stream: {steps} steps, {wall * 1e3 / steps:.2f} ms/token, {tok_s:.1f} tok/s; hit rate {hit:.3f}; "
        f"H2D {st['bytes_h2d'] / 1e9:.2f} GB ({h2d_gbs:.1f} GB/s; link {link_gbs:.1f} GB/s); {st}; "
        f"untimed drift bookkeeping {harness * 1e3 / steps:.2f} ms/step")
    # parity at the full size (after the timed region): a streamed layer runs
    # the resident three-kernel decode's kernels on the same bytes, so the 48
    # layers made resident again from the streamed layers' own bytes (router
    # read back, experts from the host slabs, the same current router
    # biases) must give the streamed chain's bits token after token
    parity = None
    if args.parity_layers > 0:
        prev_fd = hip.colizig_hip_set_fused_decode(0)
        try:
            t1 = time.time()
            w_slot, P = 3 * mat, moe.packed_expert_bytes(d)
            for l in range(NL):
                Lr = moe.Layer.load(NL + l, d, moe.Layer(l, d, True).read_router())
                if args.split_slabs:
                    wa = host[l][0].view(np.uint8).reshape(E, w_slot)
                    sa = host[l][1].view(np.float32).reshape(E, 3 * nsc)
                else:
                    a = host[l][0].view(np.uint8).reshape(E, P)
                    wa, sa = a[:, :w_slot], a[:, w_slot:].view(np.float32)
                for e in range(E):
                    w, sc = wa[e], sa[e]
                    Lr.load_expert(e, w[:mat].reshape(I, H), sc[:nsc].reshape(nblk(I), nblk(H)),
                                   w[mat:2 * mat].reshape(I, H), sc[nsc:2 * nsc].reshape(nblk(I), nblk(H)),
                                   w[2 * mat:].reshape(H, I), sc[2 * nsc:].reshape(nblk(H), nblk(I)))
                lp = -1.2 * np.log(ranks[l].astype(np.float64) + 1.0)
                Lr.set_router_bias((lp - lp.mean()).astype(np.float32))
            log(f"parity: {NL} resident copies of the streamed layers in {time.time() - t1:.1f}s")
            xr = moe.DeviceBuffer(x0.nbytes)
            xr.upload(xb.download(np.empty_like(x0)))
            ntok, same = 8, True
            for _ in range(ntok):
                if hip.colizig_hip_stream_decode(0, NL, xb.ptr, 1, eps) != 0 or \
                        hip.colizig_hip_chain_decode(NL, NL, xr.ptr, 1, eps, None, None, None, None) != 0:
                    raise RuntimeError(f"parity pass failed: {_lib.last_error()}")
                assert hip.colizig_hip_sync() == 0
                a, b = xb.download(np.empty_like(x0)), xr.download(np.empty_like(x0))
                same = same and bool(np.array_equal(a.view(np.uint32), b.view(np.uint32)))
            # as timed: the speculative runs on the one-launch decode, the
            # resident chain on it too; the residual differs only in the
            # order of the per-XCD partial sums (a changed pick would show
            # as a difference of order 1e-2)
            hip.colizig_hip_set_fused_decode(prev_fd)
            xr.upload(xb.download(np.empty_like(x0)))
            worst = 0.0
            for _ in range(ntok):
                if hip.colizig_hip_stream_decode(0, NL, xb.ptr, 1, eps) != 0 or \
                        hip.colizig_hip_chain_decode(NL, NL, xr.ptr, 1, eps, None, None, None, None) != 0:
                    raise RuntimeError(f"parity pass failed: {_lib.last_error()}")
                assert hip.colizig_hip_sync() == 0
                a, b = xb.download(np.empty_like(x0)), xr.download(np.empty_like(x0))
                worst = max(worst, float(np.linalg.norm((a - b).astype(np.float64)) /
                                         np.linalg.norm(b.astype(np.float64))))
            parity = {"reference": f"the same {NL} layers resident from the same x",
                      "tokens": ntok, "bit_identical_three_kernel": same,
                      "one_launch_rel_l2": worst, "one_launch_ok": worst < 1e-5}
            xr.free()
        finally:
            hip.colizig_hip_set_fused_decode(prev_fd)
        log(f"parity: {parity}")
    line = {
        "metric": "MoE decode tok/s, expert-streaming tier (16 GB HBM pool, 29 GB pinned host), Qwen3-30B-A3B "
                  "shape, 1 MI355X",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "e4m3-weights/f32-accumulate",
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) hidden state, Zipf(1.2) routing with 10% drift)",
        "config": {**c, "parallelism": "none (1 GPU)", "global_batch": 1, "seq_len": 1},
        "hit_rate": round(hit, 4), "h2d_gbs": round(h2d_gbs, 2), "link_h2d_gbs": round(link_gbs, 2),
        "h2d_link_frac": round(h2d_gbs / link_gbs, 3), "pool": st,
        "next_layer_prediction_accuracy": round(st["next_correct"] / max(st["next_predicted"], 1), 4),
        "token_level_prediction_accuracy": round(st["tok_correct"] / max(st["tok_predicted"], 1), 4),
        "roofline": {"bound": "h2d", "achieved": round(h2d_gbs, 2), "peak": round(link_gbs, 2), "unit": "GB/s",
                     "frac": round(h2d_gbs / link_gbs, 3), "traffic": None, "scope": "host->HBM fills"},
        "parity": parity,
    }
    print(json.dumps(line), flush=True)
    # the pinned slabs in `host` stay allocated until the process ends (the layers point at them)


def qwen4_bench(args) -> None:
    """Qwen4-Exp-style MoE stack (synthetic shapes): 36 layers, hidden 4096,
    512 routed experts top-10 + 1 always-on shared expert, moe_intermediate
    512, shared_intermediate 4096, block-FP8 weights (116 GB resident).
    Decode at batch 1 (decode kernels) and at batch 32 independent rows
    (grouped regime), each a HIP graph of the chained step."""
    from colizig_amd import _lib, moe
    H, E, K, I, SI, NL = 4096, 512, 10, 512, 4096, 36
    c = dict(workload="qwen4-exp-moe-decode", layers=NL, hidden=H, experts=E, topk=K, inter=I, shared_inter=SI,
             norm_topk=1, weights="block-fp8-e4m3-128x128", seed=0)
    name = moe.init()
    log(f"device: {name}")
    hip = _lib.hip()
    d = moe.dims(H, E, K, I, SI, True)
    zero_router = np.zeros((E, H), np.float32)
    t0 = time.time()
    for l in range(NL):
        moe.Layer.load(l, d, zero_router).synth(seed=7 * l + 3)
    log(f"weights generated in HBM: {NL} layers in {time.time() - t0:.1f}s")
    per_expert = 3 * H * I + 4 * 3 * nblk(I) * nblk(H)
    shared = 3 * H * SI + 4 * 3 * nblk(SI) * nblk(H) + H * 4
    router = E * H * 4
    out = {}
    for S in (1, 32):
        x0 = np.random.default_rng(S).normal(0.0, 1.0, size=(S, H)).astype(np.float32)
        xb = moe.DeviceBuffer(x0.nbytes)
        idx_t = moe.DeviceBuffer(NL * S * K * 4)
        xb.upload(x0)
        assert hip.colizig_hip_chain_decode(0, NL, xb.ptr, S, 1e-6, None, idx_t.ptr, None, None) == 0
        assert hip.colizig_hip_sync() == 0
        idx = idx_t.download(np.empty((NL, S, K), np.uint32))
        touched = sum(int(np.unique(idx[l]).size) for l in range(NL))
        step_bytes = touched * per_expert + NL * (shared + router + 2 * S * H * 4)
        xb.upload(x0)
        gh = hip.colizig_hip_chain_graph_create(0, NL, xb.ptr, S, 1e-6)
        assert gh > 0, _lib.last_error()
        for _ in range(args.warmup):
            assert hip.colizig_hip_graph_launch(gh, None) == 0
        assert hip.colizig_hip_sync() == 0
        ev0, ev1 = hip.colizig_hip_event_create(), hip.colizig_hip_event_create()
        steps = max(8, args.steps // (4 if S > 1 else 1))
        hip.colizig_hip_event_record(ev0, None)
        for _ in range(steps):
            hip.colizig_hip_graph_launch(gh, None)
        hip.colizig_hip_event_record(ev1, None)
        assert hip.colizig_hip_sync() == 0
        ms = hip.colizig_hip_event_elapsed_ms(ev0, ev1) / steps
        gbs = step_bytes / (ms * 1e-3) / 1e9
        out[S] = dict(tok_s=round(S * 1000.0 / ms, 1), ms_per_step=round(ms, 4), hbm_gbs=round(gbs, 1),
                      hbm_frac=round(gbs / HBM_PEAK_GBS, 4), experts_touched_per_layer=round(touched / NL, 1),
                      bytes_per_step=step_bytes)
        log(f"qwen4 S={S}: {ms:.3f} ms/step, {S * 1000.0 / ms:.1f} tok/s, {gbs:.0f} GB/s "
            f"({touched / NL:.1f} experts/layer)")
        hip.colizig_hip_graph_destroy(gh)
        xb.free()
        idx_t.free()
    # after the timed regions: the batch-1 chain against the oracle's own
    # chain from the same x0 over the first PL layers (each 3.3 GB layer
    # copied back), and the oracle's per-layer time on the host cores as the
    # CPU baseline, scaled to the 36-layer token
    parity, cpu = None, None
    PL = min(args.parity_layers, 4, NL)
    if PL > 0:
        from oracle import oracle as orc
        threads = min(len(os.sched_getaffinity(0)), 16)
        orc.lib().czo_parallel_enable(threads)
        t1 = time.time()
        hosts = [orc.OracleLayer(host_layer(hip, moe.Layer(l, d), c)) for l in range(PL)]
        copy_s = time.time() - t1
        x0 = np.random.default_rng(101).normal(0.0, 1.0, size=(1, H)).astype(np.float32)
        parity = parity_check(hip, moe, hosts, x0, c, 1e-6)
        log(f"parity: {parity}")
        xo = x0.copy()
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds or n < PL:
            hosts[n % PL].chain(xo, 1e-6)
            n += 1
        per_layer_s = (time.perf_counter() - t0) / n
        cpu = {"value": round(1.0 / (NL * per_layer_s), 3), "unit": "tok/s", "cores": threads, "kind": "port",
               "sample": f"{n} layer steps of the oracle's chain at batch 1 over the first {PL} layers "
                         f"({per_layer_s * 1e3:.1f} ms per layer), scaled to the {NL}-layer token; host "
                         f"{cpu_model()}; {copy_s:.1f} s to copy the {PL} layers back"}
        log(f"cpu baseline: {cpu}")
        del hosts
    line = {
        "metric": "MoE decode tok/s, Qwen4-Exp-style stack (36 L, E512 top-10 + shared), 1 MI355X",
        "value": out[1]["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": out[1]["ms_per_step"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "e4m3-weights/f32-accumulate", "data": "synthetic (seeded N(0,0.02) weights, N(0,1) hidden states)",
        "config": {**c, "parallelism": "none (1 GPU)", "global_batch": 1, "seq_len": 1},
        "batch1": out[1], "batch32": out[32],
        "roofline": {"bound": "hbm", "achieved": out[1]["hbm_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": out[1]["hbm_frac"], "traffic": None, "scope": "whole step, batch 1"},
        "parity": parity,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def attn_bench(args) -> None:
    """The FP8 attention projections of Qwen3-30B-A3B decode at batch 1
    (attn.zig:206-208 q/k/v, :260 o; shapes attn.zig:55-58: q [4096][2048],
    k and v [512][2048], o [2048][4096]) for 48 layers through the keyed
    device GEMV, each matrix resident under its attnKey (attn.zig:47-50).  The
    192 launches of a token are captured in one graph on a torch stream (used
    for the stream and the graph only) and replayed; inputs stay in HBM.
    Synthetic weights: one random block-FP8 matrix per role, uploaded under
    every layer's key (each key holds its own HBM copy, so every launch reads
    its own bytes)."""
    import torch
    from colizig_amd import _lib, moe, synth
    name = moe.init()
    log(f"device: {name}")
    NL, H, QD, KVD = args.layers, 2048, 32 * 128, 4 * 128
    shapes = [(QD, H), (KVD, H), (KVD, H), (H, QD)]  # (O, I) of q, k, v, o
    rng = np.random.default_rng(0)
    mats = [synth.block_quantize(rng.normal(0, 0.02, size=(O, I)).astype(np.float32)) for (O, I) in shapes]
    moe.set_vram_budget(8 << 30)
    for l in range(NL):
        for role, (w, s) in enumerate(mats):
            moe.matrix_load(moe.Fp8Matrix.attn_key(l, role), w, s)
    dev = torch.device("cuda:0")
    x = torch.randn(QD, device=dev)            # x (first H entries) and the attention output
    ys = [torch.empty(O, device=dev) for (O, _) in shapes]
    st = torch.cuda.Stream(device=dev)
    hs = ctypes.c_void_p(st.cuda_stream)

    def token():
        for l in range(NL):
            if args.attn_separate:
                for role, (O, I) in enumerate(shapes):
                    moe.matmul_fp8_dev(ys[role].data_ptr(), x.data_ptr(), 1, I, O, moe.Fp8Matrix.attn_key(l, role), hs)
            else:  # q, k and v share their input: one launch; then o
                moe.matmul_fp8_dev_multi([ys[r].data_ptr() for r in range(3)], x.data_ptr(), 1, H,
                                         [shapes[r][0] for r in range(3)],
                                         [moe.Fp8Matrix.attn_key(l, r) for r in range(3)], hs)
                O, I = shapes[3]
                moe.matmul_fp8_dev(ys[3].data_ptr(), x.data_ptr(), 1, I, O, moe.Fp8Matrix.attn_key(l, 3), hs)

    with torch.cuda.stream(st):
        token()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        token()
    for _ in range(args.warmup):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(st):
        e0.record(st)
        for _ in range(args.steps):
            g.replay()
        e1.record(st)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / args.steps
    per_token = NL * sum(O * I + nblk(O) * nblk(I) * 4 for (O, I) in shapes)
    gbs = per_token / (us * 1e-6) / 1e9
    launches = NL * (4 if args.attn_separate else 2)
    log(f"attn: {NL} layers x q/k/v/o at batch 1 ({launches} launches): {us:.1f} us per token, "
        f"{per_token / 1e6:.1f} MB, {gbs:.0f} GB/s")
    moe.set_vram_budget(0)
    print(json.dumps({
        "metric": "FP8 attention projections q/k/v/o at decode (keyed device GEMV), Qwen3-30B-A3B shape, 1 MI355X",
        "value": round(1e6 / us, 1), "unit": "tok/s (projections only)", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(us / 1000.0, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "e4m3-weights/f32-accumulate", "data": "synthetic (seeded N(0,0.02) weights)",
        "config": {"workload": "qwen3-30b-a3b-attn-proj-decode", "layers": NL, "hidden": H, "q_dim": QD,
                   "kv_dim": KVD, "global_batch": 1, "seq_len": 1, "parallelism": "none (1 GPU)",
                   "qkv": "three launches" if args.attn_separate else "one launch (matmul_fp8_dev_multi)"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "scope": "whole token, 192 launches"},
    }))


# tools/microbench.zig:198-298's FP8 expert matmul and its published single-
# thread figure (docs/BENCHMARK.md:240, "FP8: fused decode+FMA")
MICRO_I, MICRO_O, MICRO_ITERS = 2560, 640, 4000
MICRO_REF_US, MICRO_REF_GFLOPS = 469.0, 7.0


def microbench(args) -> None:
    """The reference's kernel micro-benchmark restated (tools/microbench.zig:
    198-298): one FP8 expert projection y[1, 640] = x[1, 2560] . W[640, 2560]^T
    with 128x128 block scales, timed over 4000 back-to-back matmuls.  GPU: the
    keyed device FP8 GEMV (the matrix resident, the input in HBM), between HIP
    events on the library stream.  CPU: the oracle's matmulFp8 (fp8.zig:
    215-257, the reference's CPU SIMD path restated in C) on one thread, the
    reference's own setting.  Inputs as the reference draws them (x uniform in
    [-1, 1), random weight bytes, scales uniform in [0.01, 0.06)), NaN
    encodings excluded so that the two results can be compared."""
    from colizig_amd import _lib, moe
    from oracle import oracle as orc
    name = moe.init()
    log(f"device: {name}")
    hip = _lib.hip()
    I, O, iters = MICRO_I, MICRO_O, MICRO_ITERS
    rng = np.random.default_rng(42)
    x = (rng.random((1, I), dtype=np.float32) * 2 - 1).astype(np.float32)
    w = rng.integers(0, 256, size=(O, I), dtype=np.uint8)
    w[(w & 0x7f) == 0x7f] = 0x00  # no NaN encodings
    s = (0.01 + rng.random(nblk(O) * nblk(I), dtype=np.float32) * 0.05).astype(np.float32)
    moe.set_vram_budget(1 << 30)
    key = moe.Fp8Matrix.expert_key(0, 1001, 0)
    moe.matrix_load(key, w, s.reshape(nblk(O), nblk(I)))
    xb, yb = moe.DeviceBuffer(I * 4), moe.DeviceBuffer(O * 4)
    xb.upload(x)
    for _ in range(max(args.warmup, 10)):
        moe.matmul_fp8_dev(yb.ptr, xb.ptr, 1, I, O, key)
    assert hip.colizig_hip_sync() == 0
    ev0, ev1 = hip.colizig_hip_event_create(), hip.colizig_hip_event_create()
    hip.colizig_hip_event_record(ev0, None)
    for _ in range(iters):
        moe.matmul_fp8_dev(yb.ptr, xb.ptr, 1, I, O, key)
    hip.colizig_hip_event_record(ev1, None)
    assert hip.colizig_hip_sync() == 0
    gpu_us = hip.colizig_hip_event_elapsed_ms(ev0, ev1) * 1000.0 / iters
    y_gpu = yb.download(np.empty((1, O), np.float32))
    moe.set_vram_budget(0)
    flop = 2.0 * O * I
    # the oracle on one thread, as the reference's micro-benchmark runs
    orc.lib().czo_parallel_disable()
    y_cpu = orc.matmul_fp8(x, w, s, 1, I, O)
    n, t0 = 0, time.perf_counter()
    while n < iters and time.perf_counter() - t0 < 20.0:
        orc.matmul_fp8(x, w, s, 1, I, O)
        n += 1
    cpu_us = (time.perf_counter() - t0) * 1e6 / n
    err = float(np.linalg.norm(y_gpu - y_cpu) / np.linalg.norm(y_cpu))
    log(f"microbench FP8 I={I} O={O} S=1: GPU {gpu_us:.2f} us/matmul ({flop / gpu_us / 1e3:.1f} GFLOP/s); "
        f"oracle, 1 thread {cpu_us:.1f} us/matmul ({flop / cpu_us / 1e3:.2f} GFLOP/s, {n} matmuls); reference "
        f"{MICRO_REF_US:.0f} us ({MICRO_REF_GFLOPS} GFLOP/s); GPU vs oracle rel L2 {err:.2e}")
    wbytes = O * I + 4 * s.size
    print(json.dumps({
        "metric": "FP8 expert matmul (tools/microbench.zig: I=2560, O=640, S=1) us per matmul, 1 MI355X",
        "value": round(gpu_us, 3), "unit": "us/matmul", "n_gpus": 1, "steps": iters, "warmup": max(args.warmup, 10),
        "ms_per_step": round(gpu_us / 1000.0, 6), "higher_is_better": False, "scaling": "strong",
        "vs_baseline": None, "dtype": "e4m3-weights/f32-accumulate",
        "data": "synthetic (x uniform [-1, 1), random E4M3 bytes without NaN, scales uniform [0.01, 0.06))",
        "config": {"workload": "microbench-fp8-expert-matmul", "I": I, "O": O, "S": 1, "matmuls": iters,
                   "parallelism": "none (1 GPU)"},
        "gflops": round(flop / gpu_us / 1e3, 2),
        "roofline": {"bound": "hbm", "achieved": round(wbytes / (gpu_us * 1e-6) / 1e9, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(wbytes / (gpu_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": None, "scope": "one launch; the 1.6 MB matrix stays in the caches between launches"},
        "reference": {"us_per_matmul": MICRO_REF_US, "gflops": MICRO_REF_GFLOPS,
                      "source": "docs/BENCHMARK.md:240 (FP8 fused decode+FMA, one thread)"},
        "cpu_baseline": {"value": round(cpu_us, 2), "unit": "us/matmul", "cores": 1, "kind": "port",
                         "gflops": round(flop / cpu_us / 1e3, 3),
                         "sample": f"{n} matmuls of the oracle's matmulFp8 (cz_oracle.c) on one thread, host "
                                   f"{cpu_model()}"},
        "parity": {"reference": "the oracle's matmulFp8 on the same inputs", "rel_l2": err, "tolerance": 1e-3},
    }))


# HBM bytes per lm_head launch from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
# (303,938 KiB read x 2.0 copy calibration + 594 KiB written)
LMHEAD_TRAFFIC_BYTES = 303938 * 1024 * 2 + 594 * 1024


def lmhead_bench(args) -> None:
    """The BF16 lm_head of Qwen3-30B-A3B at batch 1: vocab 151936 x hidden
    2048 rows (622 MB) through the keyed device BF16 GEMV, every dot in
    dotBf16's order (matmul.zig:84-110), input resident in HBM; back-to-back
    launches between HIP events on the library stream."""
    from colizig_amd import _lib, moe
    name = moe.init()
    log(f"device: {name}")
    hip = _lib.hip()
    V, H = 151936, 2048
    rng = np.random.default_rng(0)
    w = (rng.normal(0.0, 0.02, size=(V, H)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    moe.set_vram_budget(4 << 30)
    key = moe.Fp8Matrix.expert_key(0, 1000, 3)
    moe.matrix_load_bf16(key, w)
    del w
    xb, yb = moe.DeviceBuffer(H * 4), moe.DeviceBuffer(V * 4)
    xb.upload(rng.normal(size=(1, H)).astype(np.float32))
    for _ in range(args.warmup):
        moe.matmul_bf16_dev(yb.ptr, xb.ptr, 1, H, V, key)
    assert hip.colizig_hip_sync() == 0
    ev0, ev1 = hip.colizig_hip_event_create(), hip.colizig_hip_event_create()
    hip.colizig_hip_event_record(ev0, None)
    for _ in range(args.steps):
        moe.matmul_bf16_dev(yb.ptr, xb.ptr, 1, H, V, key)
    hip.colizig_hip_event_record(ev1, None)
    assert hip.colizig_hip_sync() == 0
    us = hip.colizig_hip_event_elapsed_ms(ev0, ev1) * 1000.0 / args.steps
    nbytes = V * H * 2
    gbs = nbytes / (us * 1e-6) / 1e9
    log(f"lmhead: {V} x {H} BF16 at batch 1: {us:.1f} us per token, {nbytes / 1e6:.1f} MB, {gbs:.0f} GB/s")
    moe.set_vram_budget(0)
    print(json.dumps({
        "metric": "BF16 lm_head GEMV at decode (dotBf16 order), Qwen3-30B-A3B shape, 1 MI355X",
        "value": round(1e6 / us, 1), "unit": "tok/s (lm_head only)", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(us / 1000.0, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16-weights/f32-accumulate", "data": "synthetic (seeded N(0,0.02) weights)",
        "config": {"workload": "qwen3-30b-a3b-lm-head-decode", "vocab": V, "hidden": H, "global_batch": 1,
                   "seq_len": 1, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": LMHEAD_TRAFFIC_BYTES, "scope": "one launch"},
    }))


def dropin_bench(args) -> None:
    """The drop-in path as the unchanged engine drives it: Fp8Matrix.matmul ->
    fp8.matmulFp8Keyed -> gpu.matmulFp8 -> colizig_cuda_matmul_fp8 (host
    pointers, synchronous, keyed; fp8.zig:165-194, gpu.zig:175-190), once per
    expert projection: per layer and token 3 x top-k = 24 expert calls at
    batch 1 (gate and up 768 x 2048, down 2048 x 768), plus the four FP8
    attention projections (q 4096 x 2048, k and v 512 x 2048, o 2048 x 4096).
    Every key is resident (a warm-up call uploads it), so each call is a
    keyed hit: x in, y out over PCIe, one kernel, one synchronisation.
    Reports the mean time per call of each shape and the implied MoE + attention
    projection time of a 48-layer token (the engine's own CPU work - router,
    attention, norms - not included)."""
    from colizig_amd import _lib, moe, synth
    name = moe.init()
    log(f"device: {name}")
    hip = _lib.hip()
    moe.set_vram_budget(8 << 30)
    rng = np.random.default_rng(11)
    H, I, K = 2048, 768, 8
    shapes = {"expert_gate_up": (I, H), "expert_down": (H, I), "attn_q": (4096, H), "attn_kv": (512, H),
              "attn_o": (H, 4096)}
    per_token = {"expert_gate_up": 48 * 2 * K, "expert_down": 48 * K, "attn_q": 48, "attn_kv": 48 * 2, "attn_o": 48}
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    res = {}
    for n, (O, Ii) in shapes.items():
        mats = []
        for k in range(8):  # 8 distinct keyed matrices per shape
            w, s = synth.block_quantize(rng.normal(0.0, 0.02, size=(O, Ii)).astype(np.float32))
            mats.append((w, s, moe.Fp8Matrix.expert_key(7, 100 + 8 * list(shapes).index(n) + k, 0)))
        x = rng.normal(size=(1, Ii)).astype(np.float32)
        y = np.zeros((1, O), np.float32)
        for w, s, key in mats:  # uploads (misses)
            assert hip.colizig_cuda_matmul_fp8(p(y), p(x), p(w), p(s), 1, Ii, O, key) == 0
        reps = max(1, args.steps // 4)
        t0 = time.perf_counter()
        for _ in range(reps):
            for w, s, key in mats:
                hip.colizig_cuda_matmul_fp8(p(y), p(x), p(w), p(s), 1, Ii, O, key)
        us = (time.perf_counter() - t0) * 1e6 / (reps * len(mats))
        ref = oracle_matmul(x, mats[-1][0], mats[-1][1], 1, Ii, O)
        err = float(np.linalg.norm(y - ref) / np.linalg.norm(ref))
        res[n] = {"us_per_call": round(us, 2), "calls_per_token": per_token[n], "rel_l2_vs_oracle": err}
        log(f"dropin {n} {O}x{Ii}: {us:.2f} us per call (rel L2 {err:.1e})")
    tok_ms = sum(v["us_per_call"] * v["calls_per_token"] for v in res.values()) / 1000.0
    hits = ctypes.c_uint64()
    misses = ctypes.c_uint64()
    hip.colizig_cuda_stats(ctypes.byref(hits), ctypes.byref(misses), None, None)
    line = {
        "metric": "drop-in per-matmul calls (colizig_cuda_matmul_fp8, keyed hits, host buffers), Qwen3-30B-A3B "
                  "expert and attention shapes, 1 MI355X",
        "value": round(1000.0 / tok_ms, 2), "unit": "tok/s (FP8 matmul calls only)", "n_gpus": 1,
        "steps": args.steps, "warmup": 0, "ms_per_step": round(tok_ms, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "e4m3-weights/f32-accumulate",
        "data": "synthetic (N(0,0.02) block-FP8 weights, N(0,1) inputs)",
        "config": {"workload": "dropin-per-matmul", "layers": 48, "hidden": H, "inter": I, "topk": K,
                   "calls_per_token": sum(per_token.values())},
        "calls": res, "cache_hits": hits.value, "cache_misses": misses.value,
    }
    print(json.dumps(line), flush=True)


def oracle_matmul(x, w, s, S, I, O):
    from oracle import oracle as orc
    return orc.matmul_fp8(x, w, s, S, I, O)


def calibrate_copy(mib: int) -> None:
    """A plain copy kernel of known size: under rocprofv3 --pmc its FETCH_SIZE /
    WRITE_SIZE give the counters' scale (bytes counted per byte moved)."""
    import torch
    n = mib << 20
    a = torch.empty(n, dtype=torch.uint8, device="cuda")
    b = torch.empty(n, dtype=torch.uint8, device="cuda")
    a.fill_(1)
    torch.cuda.synchronize()
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    log(f"copied {mib} MiB x 3")


def parity_check(hip, moe, orcs, x0, c, eps):
    """The GPU chain and the oracle's own chain from the same x0 over the
    first len(orcs) layers, one token: routing bit-exact (on the GPU's router
    input, and the same picks as the oracle's chain), router input and
    residual stream within 1e-3 relative L2."""
    H, K = c["hidden"], c["topk"]
    n = len(orcs)
    xn_t = moe.DeviceBuffer(n * H * 4)
    idx_t = moe.DeviceBuffer(n * K * 4)
    g_t = moe.DeviceBuffer(n * K * 4)
    xtmp = moe.DeviceBuffer(H * 4)
    xtmp.upload(x0)
    assert hip.colizig_hip_chain_decode(0, n, xtmp.ptr, 1, eps, xn_t.ptr, idx_t.ptr, g_t.ptr, None) == 0
    assert hip.colizig_hip_sync() == 0
    xn = xn_t.download(np.empty((n, H), np.float32))
    idx = idx_t.download(np.empty((n, K), np.uint32))
    gates = g_t.download(np.empty((n, K), np.float32))
    x_g = xtmp.download(np.empty((1, H), np.float32))
    xo = x0.copy()
    exact = True
    worst_xn = 0.0
    min_gap = 1 << 30
    for l, O in enumerate(orcs):
        xn_o, idx_o, _ = O.chain(xo, eps)
        worst_xn = max(worst_xn, float(np.linalg.norm(xn[l] - xn_o[0]) / np.linalg.norm(xn_o[0])))
        # near-tie census: the smallest gap, in f32 ulps, between consecutive
        # post-exp values of the oracle's top K+1 (a gap of a few ulps would
        # make the picks depend on the last bit of exp)
        _, _, v = O.route(xn_o[0])
        top = sorted(range(v.size), key=lambda e: (-float(v[e]), e))[:K + 1]
        b = v[top].view(np.uint32).astype(np.int64)
        min_gap = min(min_gap, int(np.min(b[:-1] - b[1:])))
        ri, rg, _ = O.route(xn[l])
        exact &= bool(np.array_equal(ri, idx[l]) and np.array_equal(rg.view(np.uint32), gates[l].view(np.uint32)))
        exact &= bool(np.array_equal(idx[l], idx_o[0]))
    x_err = float(np.linalg.norm(x_g - xo) / np.linalg.norm(xo))
    for buf in (xn_t, idx_t, g_t, xtmp):
        buf.free()
    return {"layers_checked": n, "reference": "oracle chain from the same x0", "routing_bit_exact": exact,
            "max_router_input_rel_l2": worst_xn, "residual_rel_l2": x_err, "tolerance": 1e-3,
            "near_tie_min_gap_ulps": min_gap}


def host_layer(hip, L, c):
    """A registered layer copied to host memory, in the oracle's layout (its
    shared expert too, when c has one)."""
    H, E, K, I = c["hidden"], c["experts"], c["topk"], c["inter"]
    SI = c.get("shared_inter", 0)
    mat = I * H
    nsc = nblk(I) * nblk(H)
    ew = np.empty(E * 3 * mat, np.uint8)
    es = np.empty(E * 3 * nsc, np.float32)
    rc = hip.colizig_hip_expert_slab_read(L.layer, ew.ctypes.data_as(ctypes.c_void_p),
                                          es.ctypes.data_as(ctypes.c_void_p))
    assert rc == 0
    ew = ew.reshape(E, 3, mat)
    es = es.reshape(E, 3, nsc)
    experts = []
    for e in range(E):
        experts.append(dict(gate_w=ew[e, 0].reshape(I, H), gate_s=es[e, 0].reshape(nblk(I), nblk(H)),
                            up_w=ew[e, 1].reshape(I, H), up_s=es[e, 1].reshape(nblk(I), nblk(H)),
                            down_w=ew[e, 2].reshape(H, I), down_s=es[e, 2].reshape(nblk(H), nblk(I))))
    return dict(dims=dict(hidden=H, experts=E, topk=K, inter=I, shared_inter=SI, norm_topk=1),
                router=L.read_router(), experts=experts, shared=L.read_shared() if SI else None, _slabs=(ew, es))


def cpu_baseline(hosts, x0, eps, seconds, copy_s):
    """The oracle's chain on the host cores, same weights, bounded sample."""
    from oracle import oracle as orc
    # at most 16 host threads per GPU (the CPU share of a one-GPU host), whatever the affinity mask shows
    present = len(os.sched_getaffinity(0))
    threads = min(present, 16)
    orc.lib().czo_parallel_enable(threads)
    x = x0.copy()
    n = 0
    t1 = time.perf_counter()
    while n < 256:
        for O in hosts:
            O.chain(x, eps)
        n += 1
        if time.perf_counter() - t1 > seconds:
            break
    el = time.perf_counter() - t1
    orc.lib().czo_parallel_disable()
    return {"value": round(n / el, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "cores_present": present,
            "sample": f"{n} decode tokens x {len(hosts)} layers of the same workload (oracle chain, "
                      f"expert fan-out over min(threads, top-k) tasks as parallel.chunks), {el:.1f}s",
            "cpu_model": cpu_model(), "host_copy_s": round(copy_s, 1)}


def cpu_model() -> str:
    """The host CPU's model name (lscpu, else /proc/cpuinfo)."""
    import subprocess
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


if __name__ == "__main__":
    main()
