"""ctypes wrapper of oracle/libczoracle.so (the C restatement in cz_oracle.c).

TEST INFRASTRUCTURE ONLY: what the HIP library's results are compared against,
and the timed CPU baseline.  Build with `make -C oracle` (or oracle.oracle.build()).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# CZ_ORACLE_LIB: another build of the same sources (the sanitizer build of
# tests/sanitize) in place of the default one
LIB = os.environ.get("CZ_ORACLE_LIB") or os.path.join(HERE, "libczoracle.so")

vp = ctypes.c_void_p
F32FN = ctypes.CFUNCTYPE(ctypes.c_float, ctypes.c_float)


class CDims(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("hidden", "experts", "topk", "inter", "shared_inter", "norm_topk")]


class CMat(ctypes.Structure):
    _fields_ = [("w", vp), ("s", vp), ("rows", ctypes.c_uint32), ("cols", ctypes.c_uint32)]


class CExpert(ctypes.Structure):
    _fields_ = [("gate", CMat), ("up", CMat), ("down", CMat)]


class CLayer(ctypes.Structure):
    _fields_ = [("d", CDims), ("router", vp), ("experts", ctypes.POINTER(CExpert)),
                ("sh_gate_proj", CMat), ("sh_up_proj", CMat), ("sh_down_proj", CMat), ("sh_gate", vp),
                ("router_bias", vp), ("sh_native_gate", vp), ("sh_native_up", vp), ("sh_native_down", vp)]


def widen_bf16(bits: np.ndarray) -> np.ndarray:
    """BF16 bit patterns -> f32, exactly (bf16 is the top half of an f32)."""
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def native_f32(m: np.ndarray) -> np.ndarray:
    """A NativeMatrix's values as f32: BF16 bits (uint16) widened, f32 as is."""
    return widen_bf16(m) if m.dtype == np.uint16 else np.ascontiguousarray(m, dtype=np.float32)


class CCacheStats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in ("hits", "misses", "loads", "evictions", "prefetch_hits",
                                                 "prefetch_wasted")]


POOL_STAT_NAMES = ("hits", "misses", "loads", "evictions", "prefetch_issued", "prefetch_hits", "prefetch_wasted")


class CPoolStats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in POOL_STAT_NAMES]


_SIGS = {
    "czo_nblk": (ctypes.c_size_t, [ctypes.c_size_t]),
    "czo_e4m3_decode": (ctypes.c_float, [ctypes.c_uint8]),
    "czo_e4m3_lut": (ctypes.POINTER(ctypes.c_float), []),
    "czo_decode_lane": (None, [vp, ctypes.c_float, vp]),
    "czo_dequant_row": (None, [vp, vp, vp, ctypes.c_size_t]),
    "czo_dequant_matrix": (None, [vp, vp, vp, ctypes.c_size_t, ctypes.c_size_t]),
    "czo_dot_fp8_row": (ctypes.c_float, [vp, vp, vp, ctypes.c_size_t]),
    "czo_dot_fp8_row_scalar": (ctypes.c_float, [vp, vp, vp, ctypes.c_size_t]),
    "czo_matmul_fp8": (None, [vp, vp, vp, vp, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t]),
    "czo_dot_f32": (ctypes.c_float, [vp, vp, ctypes.c_size_t]),
    "czo_dot_f32_scalar": (ctypes.c_float, [vp, vp, ctypes.c_size_t]),
    "czo_matmul_f32": (None, [vp, vp, vp, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t]),
    "czo_expf": (ctypes.c_float, [ctypes.c_float]),
    "czo_expf_array": (None, [vp, vp, ctypes.c_size_t]),
    "czo_sigmoid": (ctypes.c_float, [ctypes.c_float]),
    "czo_silu": (ctypes.c_float, [ctypes.c_float]),
    "czo_route": (None, [ctypes.POINTER(CLayer), vp, vp, vp, vp]),
    "czo_router_logits": (None, [ctypes.POINTER(CLayer), vp, vp]),
    "czo_moe_forward": (ctypes.c_int, [ctypes.POINTER(CLayer), vp, ctypes.c_size_t, vp, vp, vp]),
    "czo_moe_forward_dense_each": (ctypes.c_int, [ctypes.POINTER(CLayer), vp, ctypes.c_size_t, vp, vp, vp]),
    "czo_parallel_enable": (None, [ctypes.c_uint32]),
    "czo_parallel_disable": (None, []),
    "czo_parallel_max_tasks": (ctypes.c_uint32, []),
    "czo_chunk_bounds": (ctypes.c_uint32, [ctypes.c_size_t, ctypes.c_size_t, vp, ctypes.c_uint32]),
    "czo_cache_replay": (ctypes.c_uint32, [ctypes.c_uint32, vp, ctypes.c_size_t, vp, ctypes.POINTER(CCacheStats)]),
    "czo_pool_replay": (ctypes.c_int64, [ctypes.c_uint32, vp, ctypes.c_size_t, vp, ctypes.POINTER(CPoolStats)]),
    "czo_chain_layer": (ctypes.c_int, [ctypes.POINTER(CLayer), vp, ctypes.c_size_t, ctypes.c_float, vp, vp, vp]),
    "czo_rms_unit": (None, [vp, vp, ctypes.c_size_t, ctypes.c_float]),
    "czo_exp_audit": (None, [vp, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32, vp]),
    "czo_f32fn_compare": (ctypes.c_uint64, [vp, vp, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32, vp]),
}

_lib = None


def build() -> None:
    if os.environ.get("CZ_ORACLE_LIB"):
        return  # another build of the sources, made by its own recipe
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        l = ctypes.CDLL(LIB)
        for n, (r, a) in _SIGS.items():
            f = getattr(l, n)
            f.restype = r
            f.argtypes = a
        _lib = l
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(vp)


def _mat(w: np.ndarray, s: np.ndarray) -> CMat:
    return CMat(_p(w), _p(s), w.shape[0], w.shape[1])


class OracleLayer:
    """A host-built layer (colizig_amd.synth.make_layer layout) bound for the oracle.
    Keeps references to every array the C struct points at."""

    def __init__(self, host: dict):
        d = host["dims"]
        self.host = host
        self._keep = []
        # an f32 router, or BF16 bits: dotBf16 is dotF32 on the widened values (matmul.zig:60-110)
        self.router = native_f32(np.asarray(host["router"]))
        exs = (CExpert * d["experts"])()
        for e, ex in enumerate(host["experts"]):
            arr = {k: np.ascontiguousarray(v) for k, v in ex.items()}
            self._keep.append(arr)
            exs[e] = CExpert(_mat(arr["gate_w"], arr["gate_s"]), _mat(arr["up_w"], arr["up_s"]),
                             _mat(arr["down_w"], arr["down_s"]))
        self._exs = exs
        L = CLayer()
        L.d = CDims(d["hidden"], d["experts"], d["topk"], d["inter"], d["shared_inter"], d["norm_topk"])
        L.router = _p(self.router)
        L.experts = exs
        sh = host.get("shared")
        if sh is not None and "native" in sh:  # NativeMatrix rows (f32 or BF16 bits)
            s = {k: native_f32(np.asarray(sh[k])) for k in ("gate", "up", "down")}
            s["sh_gate"] = np.ascontiguousarray(sh["sh_gate"], dtype=np.float32)
            self._keep.append(s)
            L.sh_native_gate = _p(s["gate"])
            L.sh_native_up = _p(s["up"])
            L.sh_native_down = _p(s["down"])
            L.sh_gate = _p(s["sh_gate"])
        elif sh is not None:
            s = {k: np.ascontiguousarray(v) for k, v in sh.items()}
            self._keep.append(s)
            L.sh_gate_proj = _mat(s["gate_w"], s["gate_s"])
            L.sh_up_proj = _mat(s["up_w"], s["up_s"])
            L.sh_down_proj = _mat(s["down_w"], s["down_s"])
            L.sh_gate = _p(s["sh_gate"])
        if host.get("router_bias") is not None:
            self.router_bias = np.ascontiguousarray(host["router_bias"], dtype=np.float32)
            L.router_bias = _p(self.router_bias)
        self.c = L
        self.d = d

    def forward(self, x: np.ndarray, dense_each: bool = False):
        """moe.forward (moe.zig:409-426) -> (out [S,H], idx [S,K], gates [S,K])"""
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, self.d["hidden"])
        S = x.shape[0]
        out = np.empty_like(x)
        idx = np.empty((S, self.d["topk"]), np.uint32)
        gates = np.empty((S, self.d["topk"]), np.float32)
        fn = lib().czo_moe_forward_dense_each if dense_each else lib().czo_moe_forward
        rc = fn(ctypes.byref(self.c), _p(x), S, _p(out), _p(idx), _p(gates))
        if rc != 0:
            raise MemoryError("oracle forward failed")
        return out, idx, gates

    def route(self, xs: np.ndarray):
        """route (moe.zig:435-463) -> (idx [K], gates [K], v [E] post-exp values)"""
        xs = np.ascontiguousarray(xs, dtype=np.float32)
        K, E = self.d["topk"], self.d["experts"]
        idx = np.empty(K, np.uint32)
        gates = np.empty(K, np.float32)
        v = np.empty(E, np.float32)
        lib().czo_route(ctypes.byref(self.c), _p(xs), _p(idx), _p(gates), _p(v))
        return idx, gates, v

    def router_logits(self, xs: np.ndarray) -> np.ndarray:
        xs = np.ascontiguousarray(xs, dtype=np.float32)
        out = np.empty(self.d["experts"], np.float32)
        lib().czo_router_logits(ctypes.byref(self.c), _p(xs), _p(out))
        return out

    def chain(self, x: np.ndarray, eps: float):
        """x <- x + moe(rms(x)) in place; returns (xn, idx, gates)"""
        S = x.shape[0]
        xn = np.empty_like(x)
        idx = np.empty((S, self.d["topk"]), np.uint32)
        gates = np.empty((S, self.d["topk"]), np.float32)
        rc = lib().czo_chain_layer(ctypes.byref(self.c), _p(x), S, eps, _p(xn), _p(idx), _p(gates))
        if rc != 0:
            raise MemoryError("oracle chain failed")
        return xn, idx, gates


def matmul_fp8(x, w, s, S, I, O):
    y = np.empty((S, O), np.float32)
    lib().czo_matmul_fp8(_p(y), _p(np.ascontiguousarray(x, np.float32)), _p(np.ascontiguousarray(w, np.uint8)),
                         _p(np.ascontiguousarray(s, np.float32)), S, I, O)
    return y


def matmul_f32(x, w, S, I, O):
    """matmul.zig:21-33 with dotF32 (matmul.zig:60-82): y[S,O] = x[S,I] . w[O,I]^T."""
    y = np.empty((S, O), np.float32)
    lib().czo_matmul_f32(_p(y), _p(np.ascontiguousarray(x, np.float32)), _p(np.ascontiguousarray(w, np.float32)),
                         S, I, O)
    return y


def matmul_bf16(x, w_bits, S, I, O):
    """dotBf16 rows (matmul.zig:84-110): the dotF32 loop with each BF16 weight
    widened exactly (bits << 16), so it is matmul_f32 on the widened matrix."""
    w = (np.ascontiguousarray(w_bits, np.uint16).astype(np.uint32) << 16).view(np.float32)
    return matmul_f32(x, w, S, I, O)


def rms_unit(x, eps: float) -> np.ndarray:
    """rmsnorm.zig:32-40 `rms` with a unit weight, row by row."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    rows = x.reshape(-1, x.shape[-1])
    o = out.reshape(-1, x.shape[-1])
    for r in range(rows.shape[0]):
        lib().czo_rms_unit(_p(o[r]), _p(rows[r]), rows.shape[1], eps)
    return out


def dequant_matrix(w, s):
    w = np.ascontiguousarray(w, np.uint8)
    out = np.empty(w.shape, np.float32)
    lib().czo_dequant_matrix(_p(out), _p(w), _p(np.ascontiguousarray(s, np.float32)), w.shape[0], w.shape[1])
    return out


def lut() -> np.ndarray:
    p = lib().czo_e4m3_lut()
    return np.ctypeslib.as_array(p, shape=(256,)).copy()


def expf(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.empty_like(x)
    lib().czo_expf_array(_p(x), _p(out), x.size)
    return out


def fn_ptr(name: str) -> int:
    return ctypes.cast(getattr(lib(), name), vp).value


def pool_replay(nslots: int, ops: np.ndarray):
    """czo_pool_replay over an [n, 4] uint32 op log: (resident at the end or
    -1, per-op results [n] uint32, stats dict)."""
    ops = np.ascontiguousarray(ops, np.uint32).reshape(-1, 4)
    res = np.zeros(len(ops), np.uint32)
    st = CPoolStats()
    r = lib().czo_pool_replay(nslots, ops.ctypes.data_as(ctypes.c_void_p), len(ops),
                              res.ctypes.data_as(ctypes.c_void_p), ctypes.byref(st))
    return int(r), res, {n: int(getattr(st, n)) for n in POOL_STAT_NAMES}
