"""Shared helpers of the test suite (not collected as tests)."""
from __future__ import annotations

import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def tiny_qwen3_layer(li: int) -> tuple[dict, dict]:
    """(layer dict in colizig_amd.synth.make_layer layout, golden vectors) of
    the tiny-qwen3 fixture layer `li`."""
    z = np.load(os.path.join(GOLDEN, "tiny_qwen3_moe.npz"))
    p = f"l{li}."
    experts = []
    for e in range(4):
        experts.append(dict(
            gate_w=z[p + f"e{e}.gate_proj.w"], gate_s=z[p + f"e{e}.gate_proj.s"],
            up_w=z[p + f"e{e}.up_proj.w"], up_s=z[p + f"e{e}.up_proj.s"],
            down_w=z[p + f"e{e}.down_proj.w"], down_s=z[p + f"e{e}.down_proj.s"]))
    layer = dict(dims=dict(hidden=32, experts=4, topk=2, inter=16, shared_inter=0, norm_topk=1),
                 router=z[p + "router"], experts=experts, shared=None)
    gold = dict(x=z[p + "x"], out=z[p + "out_f64"], idx=z[p + "idx_f64"])
    return layer, gold


def e4m3_f64(b) -> np.ndarray:
    """Closed-form OCP E4M3 decode in float64 (bias 7, subnormal m/8*2^-6,
    0x7F/0xFF NaN)."""
    b = np.asarray(b).astype(np.int64)
    s = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 15
    m = b & 7
    v = np.where(e == 0, (m / 8.0) * 2.0 ** -6, (1 + m / 8.0) * 2.0 ** (e - 7.0))
    return s * np.where((e == 15) & (m == 7), np.nan, v)


def deq_f64(w, s) -> np.ndarray:
    rows, cols = w.shape
    sc = np.repeat(np.repeat(np.asarray(s, np.float64), 128, 0), 128, 1)[:rows, :cols]
    return e4m3_f64(w) * sc


def moe_f64(layer: dict, x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Independent float64 MoE: exp in f64, top-k by stable sort (lowest index
    on ties), SwiGLU experts, gate-weighted combine, shared expert."""
    d = layer["dims"]
    E, K = d["experts"], d["topk"]
    cache = {}

    def mat(e, k):
        key = (e, k)
        if key not in cache:
            ex = layer["experts"][e]
            cache[key] = deq_f64(ex[k + "_w"], ex[k + "_s"])
        return cache[key]

    def native(m):  # NativeMatrix rows: f32, or BF16 bits (uint16) widened exactly
        m = np.asarray(m)
        if m.dtype == np.uint16:
            return (m.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        return m.astype(np.float64)

    x = np.asarray(x, np.float64).reshape(-1, d["hidden"])
    out = np.zeros_like(x)
    idx = np.zeros((x.shape[0], K), np.int64)
    R = native(layer["router"])
    for s in range(x.shape[0]):
        lg = R @ x[s]
        v = np.exp(lg - lg.max())
        order = sorted(range(E), key=lambda e: (-v[e], e))[:K]
        den = v[order].sum() if d["norm_topk"] else v.sum()
        for z, e in enumerate(order):
            g = mat(e, "gate") @ x[s]
            u = mat(e, "up") @ x[s]
            h = g / (1 + np.exp(-g)) * u
            out[s] += (v[e] / den) * (mat(e, "down") @ h)
        if d["shared_inter"]:
            sh = layer["shared"]
            if "native" in sh:
                wg, wu, wd = native(sh["gate"]), native(sh["up"]), native(sh["down"])
            else:
                wg, wu = deq_f64(sh["gate_w"], sh["gate_s"]), deq_f64(sh["up_w"], sh["up_s"])
                wd = deq_f64(sh["down_w"], sh["down_s"])
            g = wg @ x[s]
            u = wu @ x[s]
            h = g / (1 + np.exp(-g)) * u
            sg = 1 / (1 + np.exp(-(x[s] @ np.asarray(sh["sh_gate"], np.float64))))
            out[s] += sg * (wd @ h)
        idx[s] = order
    return out, idx


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def f32_bits(a) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32).view(np.uint32)
