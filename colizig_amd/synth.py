"""Seeded synthetic MoE layers (a workload generator, not reference code).

Weights are drawn N(0, std) and quantised per 128x128 block to OCP E4M3
(e4m3fn) with scale = amax/448 (1 for an all-zero block), round to nearest
even - the block-FP8 format the reference's checkpoints use (fp8.zig:1-6).
The GPU-side generator is colizig_hip_layer_synth; this one serves small
host-built layers.
"""
from __future__ import annotations

import numpy as np

BLOCK = 128


def nblk(x: int) -> int:
    """fp8.zig:19-21"""
    return (x + BLOCK - 1) // BLOCK


def e4m3_positive_values() -> np.ndarray:
    """Values of the 127 finite non-negative E4M3 codes 0x00..0x7E (closed form:
    bias 7, subnormal m/8 * 2^-6)."""
    codes = np.arange(127)
    e = (codes >> 3) & 15
    m = codes & 7
    sub = (m / 8.0) * 2.0 ** -6
    nor = (1.0 + m / 8.0) * 2.0 ** (e.astype(np.float64) - 7)
    return np.where(e == 0, sub, nor)


_POS = e4m3_positive_values()


def quantize_e4m3(q: np.ndarray) -> np.ndarray:
    """f32 -> E4M3 bytes, round to nearest even, saturating at +-448."""
    a = np.minimum(np.abs(q.astype(np.float64)), 448.0)
    hi = np.clip(np.searchsorted(_POS, a, side="left"), 0, 126)
    lo = np.maximum(hi - 1, 0)
    d_lo = a - _POS[lo]
    d_hi = _POS[hi] - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & ((hi & 1) == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    code = np.where(a == 0, 0, code).astype(np.uint8)
    sign = np.where(q < 0, 0x80, 0).astype(np.uint8)
    return np.where(code == 0, 0, code | sign).astype(np.uint8)


def block_quantize(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """[rows, cols] f32 -> (E4M3 bytes [rows, cols], scales [nblk(rows), nblk(cols)])."""
    rows, cols = w.shape
    nr, nc = nblk(rows), nblk(cols)
    scales = np.ones((nr, nc), dtype=np.float32)
    out = np.empty((rows, cols), dtype=np.uint8)
    for br in range(nr):
        for bc in range(nc):
            blk = w[br * BLOCK:(br + 1) * BLOCK, bc * BLOCK:(bc + 1) * BLOCK].astype(np.float32)
            amax = float(np.max(np.abs(blk))) if blk.size else 0.0
            s = np.float32(amax / 448.0) if amax > 0 else np.float32(1.0)
            scales[br, bc] = s
            out[br * BLOCK:(br + 1) * BLOCK, bc * BLOCK:(bc + 1) * BLOCK] = quantize_e4m3(blk / s)
    return out, scales


def make_layer(hidden: int, experts: int, topk: int, inter: int, shared_inter: int = 0, norm_topk: bool = True,
               seed: int = 0, std_w: float = 0.02, std_router: float = 0.02) -> dict:
    """One synthetic MoE layer as host arrays:
    router [E,H] f32; experts: list of dicts gate_w/gate_s/up_w/up_s/down_w/down_s;
    shared (or None) likewise plus sh_gate [H] f32."""
    rng = np.random.default_rng(seed)
    H, E, I, SI = hidden, experts, inter, shared_inter

    def mat(rows, cols):
        return block_quantize(rng.normal(0.0, std_w, size=(rows, cols)).astype(np.float32))

    router = rng.normal(0.0, std_router, size=(E, H)).astype(np.float32)
    ex = []
    for _ in range(E):
        gw, gs = mat(I, H)
        uw, us = mat(I, H)
        dw, ds = mat(H, I)
        ex.append(dict(gate_w=gw, gate_s=gs, up_w=uw, up_s=us, down_w=dw, down_s=ds))
    shared = None
    if SI:
        gw, gs = mat(SI, H)
        uw, us = mat(SI, H)
        dw, ds = mat(H, SI)
        shared = dict(gate_w=gw, gate_s=gs, up_w=uw, up_s=us, down_w=dw, down_s=ds,
                      sh_gate=rng.normal(0.0, std_router, size=(H,)).astype(np.float32))
    return dict(dims=dict(hidden=H, experts=E, topk=topk, inter=I, shared_inter=SI, norm_topk=int(norm_topk)),
                router=router, experts=ex, shared=shared)


def hidden_states(S: int, hidden: int, seed: int) -> np.ndarray:
    """x ~ N(0,1) f32 [S, hidden]"""
    return np.random.default_rng(seed).normal(0.0, 1.0, size=(S, hidden)).astype(np.float32)


def zipf_router_bias(E: int, s: float, seed: int) -> np.ndarray:
    """Per-expert router bias that makes expert popularity Zipf(s): p_e is
    proportional to rank^-s over a seeded permutation of the experts, and
    b_e = ln(p_e) - mean(ln p).  Added to the logits, it multiplies each
    expert's softmax weight by p_e (up to a common factor)."""
    rng = np.random.default_rng(seed)
    ranks = np.empty(E, np.float64)
    ranks[rng.permutation(E)] = np.arange(1, E + 1, dtype=np.float64)
    lp = -s * np.log(ranks)
    return (lp - lp.mean()).astype(np.float32)


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round f32 values to BF16 (nearest, ties to even) as uint16 bits."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def with_native(host: dict, seed: int, router_bf16: bool = True, shared: str | None = None,
                std_w: float = 0.02) -> dict:
    """A make_layer host with NativeMatrix weights (tensors.zig:65-120): the
    router rounded to BF16 bits, and/or (shared = "f32" or "bf16") a shared
    expert of f32 or BF16 rows drawn N(0, std_w) with an f32 sh_gate."""
    out = dict(host)
    if router_bf16:
        out["router"] = f32_to_bf16_bits(host["router"])
    if shared:
        d = host["dims"]
        H, SI = d["hidden"], d["shared_inter"]
        assert SI, "the dims have no shared expert"
        rng = np.random.default_rng(seed)
        mats = [rng.normal(0.0, std_w, size=s).astype(np.float32) for s in ((SI, H), (SI, H), (H, SI))]
        if shared == "bf16":
            mats = [f32_to_bf16_bits(m) for m in mats]
        sg = host["shared"]["sh_gate"] if host.get("shared") else rng.normal(0.0, 0.02, size=(H,)).astype(np.float32)
        out["shared"] = dict(native=shared, gate=mats[0], up=mats[1], down=mats[2], sh_gate=sg)
    return out
