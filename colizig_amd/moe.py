"""Host-side mirror of colizig's MoE interface (src/qwen38/moe.zig,
src/ops/fp8.zig, src/backend/gpu.zig) over libcolizig_hip.so.

Names and argument meaning follow the reference: `Dims`, `Fp8Matrix`
(with `expert_key`), `Layer.load` -> HBM registration, `forward(x, S)`,
`matmul_fp8`.  Errors are the library's negative return codes, raised as
`GpuBackendError` - the point where the reference's engine would fall back to
its CPU path (fp8.zig:182-187).  Nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from ._lib import Dims

BLOCK = 128


def nblk(x: int) -> int:
    """fp8.zig:19-21"""
    return (x + BLOCK - 1) // BLOCK


class GpuBackendError(RuntimeError):
    def __init__(self, what: str, rc: int):
        super().__init__(f"{what} failed rc={rc}: {_lib.last_error()}")
        self.rc = rc


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _check(what: str, rc: int) -> None:
    if rc != 0:
        raise GpuBackendError(what, rc)


def init() -> str:
    """colizig_cuda_init + device name (gpu.zig:72-109); raises when no GPU."""
    lib = _lib.hip()
    _check("colizig_cuda_init", lib.colizig_cuda_init())
    return lib.colizig_cuda_device_name().decode()


def shutdown() -> None:
    _lib.hip().colizig_cuda_shutdown()


def set_vram_budget(nbytes: int) -> None:
    """gpu.zig:156-158"""
    _lib.hip().colizig_cuda_set_vram_budget(nbytes)


def stats() -> dict:
    """colizig_cuda_stats (gpu.zig:160-170)"""
    v = [ctypes.c_uint64() for _ in range(4)]
    _lib.hip().colizig_cuda_stats(*[ctypes.byref(x) for x in v])
    return dict(hits=v[0].value, misses=v[1].value, uploaded_mib=v[2].value, resident=v[3].value)


def matmul_fp8(x: np.ndarray, w: np.ndarray, scales: np.ndarray, S: int, I: int, O: int, key: int = 0) -> np.ndarray:
    """fp8.matmulFp8Keyed's GPU leg (fp8.zig:165-188): y[S,O] = x[S,I] @ dequant(w[O,I])^T."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    assert x.size == S * I and w.size == O * I and scales.size == nblk(O) * nblk(I)
    y = np.empty((S, O), dtype=np.float32)
    _check("colizig_cuda_matmul_fp8", _lib.hip().colizig_cuda_matmul_fp8(_p(y), _p(x), _p(w), _p(scales), S, I, O,
                                                                          key))
    return y


def matrix_load(key: int, w: np.ndarray, scales: np.ndarray) -> None:
    """Puts an FP8 matrix w[O,I] (+ block scales) under `key` in the HBM cache
    for matmul_fp8_dev (the keyed cache of fp8.zig:182's GPU leg)."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    O, I = w.shape
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    assert scales.size == nblk(O) * nblk(I)
    _check("colizig_hip_matrix_load", _lib.hip().colizig_hip_matrix_load(key, _p(w), _p(scales), I, O))


def matmul_fp8_dev(y_ptr: int, x_ptr: int, S: int, I: int, O: int, key: int, stream=None) -> None:
    """y[S,O] = x[S,I] @ dequant(W_key)^T on device pointers (asynchronous)."""
    _check("colizig_hip_matmul_fp8_dev", _lib.hip().colizig_hip_matmul_fp8_dev(y_ptr, x_ptr, S, I, O, key, stream))


def matmul_fp8_dev_multi(y_ptrs, x_ptr: int, S: int, I: int, Os, keys, stream=None) -> None:
    """Several keyed FP8 matrices of row width I on the same input rows, one
    launch: y_m[S,O_m] = x[S,I] @ dequant(W_keys[m])^T (asynchronous; the
    bits of matmul_fp8_dev of each key)."""
    n = len(keys)
    ys = (ctypes.c_void_p * n)(*y_ptrs)
    ks = (ctypes.c_uint64 * n)(*keys)
    os_ = (ctypes.c_int * n)(*Os)
    _check("colizig_hip_matmul_fp8_dev_multi",
           _lib.hip().colizig_hip_matmul_fp8_dev_multi(n, ys, ks, os_, x_ptr, S, I, stream))


def matrix_load_bf16(key: int, w_bits: np.ndarray) -> None:
    """Puts BF16 rows w[O,I] (uint16 bits) under `key` in the HBM cache."""
    w_bits = np.ascontiguousarray(w_bits, dtype=np.uint16)
    O, I = w_bits.shape
    _check("colizig_hip_matrix_load_bf16", _lib.hip().colizig_hip_matrix_load_bf16(key, _p(w_bits), I, O))


def matmul_bf16_dev(y_ptr: int, x_ptr: int, S: int, I: int, O: int, key: int, stream=None) -> None:
    """y[S,O] = dotBf16 rows (matmul.zig:84-110) on device pointers (asynchronous)."""
    _check("colizig_hip_matmul_bf16_dev", _lib.hip().colizig_hip_matmul_bf16_dev(y_ptr, x_ptr, S, I, O, key, stream))


def dequant_fp8(w: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """GPU dequantisation e4m3(w) * scale (fp8.zig:123-130 semantics)."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    rows, cols = w.shape
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    out = np.empty((rows, cols), dtype=np.float32)
    _check("colizig_hip_dequant_fp8", _lib.hip().colizig_hip_dequant_fp8(_p(out), _p(w), _p(scales), rows, cols))
    return out


@dataclass
class Fp8Matrix:
    """moe.zig:50-100"""

    data: np.ndarray    # [rows, cols] uint8 E4M3
    scales: np.ndarray  # [nblk(rows), nblk(cols)] f32
    key: int = 0

    @property
    def rows(self) -> int:
        return self.data.shape[0]

    @property
    def cols(self) -> int:
        return self.data.shape[1]

    def byte_len(self) -> int:
        """moe.zig:88-90"""
        return self.data.size + self.scales.size * 4

    def matmul(self, x: np.ndarray, S: int) -> np.ndarray:
        """moe.zig:93-95: y[S, rows] = x[S, cols] @ dequant(self)^T"""
        return matmul_fp8(x, self.data, self.scales, S, self.cols, self.rows, self.key)

    @staticmethod
    def expert_key(layer: int, expert: int, role: int) -> int:
        """moe.zig:97-99: 1 + ((layer*512 + expert)*4 + role)"""
        return 1 + (layer * 512 + expert) * 4 + role

    @staticmethod
    def attn_key(layer: int, role: int) -> int:
        """attn.zig:47-50 attnKey: expert slot 1020 + role (0..3 = q/k/v/o)."""
        return Fp8Matrix.expert_key(layer, 1020 + role, 0)


def dims(hidden: int, experts: int, topk: int, inter: int, shared_inter: int = 0, norm_topk: bool = True) -> Dims:
    return Dims(hidden, experts, topk, inter, shared_inter, int(norm_topk))


@dataclass
class Layer:
    """A registered MoE layer (moe.zig:297-338 Layer + its resident experts)."""

    layer: int
    d: Dims
    registered: bool = field(default=False)

    @staticmethod
    def load(layer: int, d: Dims, router: np.ndarray) -> "Layer":
        """Layer.load (moe.zig:306-328): router weights into HBM."""
        router = np.ascontiguousarray(router, dtype=np.float32)
        assert router.shape == (d.experts, d.hidden)
        _check("colizig_hip_layer_init", _lib.hip().colizig_hip_layer_init(layer, ctypes.byref(d), _p(router)))
        return Layer(layer, d, True)

    def load_expert(self, expert: int, gate_w, gate_s, up_w, up_s, down_w, down_s) -> None:
        """loadExpert (moe.zig:251-292) into the expert's HBM slot."""
        H, I = self.d.hidden, self.d.inter
        arrs = [np.ascontiguousarray(a, dtype=t) for a, t in
                ((gate_w, np.uint8), (gate_s, np.float32), (up_w, np.uint8), (up_s, np.float32),
                 (down_w, np.uint8), (down_s, np.float32))]
        assert arrs[0].shape == (I, H) and arrs[2].shape == (I, H) and arrs[4].shape == (H, I)
        _check("colizig_hip_expert_load",
               _lib.hip().colizig_hip_expert_load(self.layer, expert, *[_p(a) for a in arrs]))

    def set_shared(self, gate_w, gate_s, up_w, up_s, down_w, down_s, sh_gate) -> None:
        arrs = [np.ascontiguousarray(a, dtype=t) for a, t in
                ((gate_w, np.uint8), (gate_s, np.float32), (up_w, np.uint8), (up_s, np.float32),
                 (down_w, np.uint8), (down_s, np.float32), (sh_gate, np.float32))]
        _check("colizig_hip_layer_set_shared",
               _lib.hip().colizig_hip_layer_set_shared(self.layer, *[_p(a) for a in arrs]))

    def set_router_bf16(self, bits: np.ndarray) -> None:
        """A BF16 router (NativeMatrix bf16, tensors.zig:65-120) as raw bits
        [E][H]; logits in dotBf16's order (matmul.zig:84-110)."""
        b = np.ascontiguousarray(bits, dtype=np.uint16)
        assert b.shape == (self.d.experts, self.d.hidden)
        _check("colizig_hip_layer_set_router_bf16", _lib.hip().colizig_hip_layer_set_router_bf16(self.layer, _p(b)))

    def set_shared_native(self, gate: np.ndarray, up: np.ndarray, down: np.ndarray, sh_gate: np.ndarray) -> None:
        """A NativeMatrix shared expert (moe.zig:300-303, 316-325): gate, up
        [SI][H] and down [H][SI] as f32 or BF16 bits (uint16), sh_gate [H]."""
        H, SI = self.d.hidden, self.d.shared_inter
        bf16 = np.asarray(gate).dtype == np.uint16
        t = np.uint16 if bf16 else np.float32
        g, u, dn = (np.ascontiguousarray(m, dtype=t) for m in (gate, up, down))
        assert g.shape == (SI, H) and u.shape == (SI, H) and dn.shape == (H, SI)
        sg = np.ascontiguousarray(sh_gate, dtype=np.float32)
        _check("colizig_hip_layer_set_shared_native", _lib.hip().colizig_hip_layer_set_shared_native(
            self.layer, 1 if bf16 else 0, _p(g), _p(u), _p(dn), _p(sg)))

    def set_router_bias(self, bias: np.ndarray | None) -> None:
        """Optional per-expert logit bias (workload shaping; None clears it)."""
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        assert b is None or b.shape == (self.d.experts,)
        _check("colizig_hip_layer_set_router_bias", _lib.hip().colizig_hip_layer_set_router_bias(self.layer, _p(b)))

    def synth(self, seed: int, std_w: float = 0.02, std_router: float = 0.02) -> None:
        _check("colizig_hip_layer_synth", _lib.hip().colizig_hip_layer_synth(self.layer, seed, std_w, std_router))

    def forward(self, x: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        """moe.forward (moe.zig:409-426): returns (out [S,H], idx [S,K], gates [S,K])."""
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, self.d.hidden)
        S = x.shape[0]
        out = np.empty_like(x)
        idx = np.empty((S, self.d.topk), dtype=np.uint32)
        gates = np.empty((S, self.d.topk), dtype=np.float32)
        _check("colizig_hip_moe_forward",
               _lib.hip().colizig_hip_moe_forward(self.layer, _p(x), S, _p(out), _p(idx), _p(gates)))
        return out, idx, gates

    def read_expert(self, expert: int) -> dict:
        H, I = self.d.hidden, self.d.inter
        r = dict(gate_w=np.empty((I, H), np.uint8), gate_s=np.empty((nblk(I), nblk(H)), np.float32),
                 up_w=np.empty((I, H), np.uint8), up_s=np.empty((nblk(I), nblk(H)), np.float32),
                 down_w=np.empty((H, I), np.uint8), down_s=np.empty((nblk(H), nblk(I)), np.float32))
        _check("colizig_hip_expert_read", _lib.hip().colizig_hip_expert_read(
            self.layer, expert, _p(r["gate_w"]), _p(r["gate_s"]), _p(r["up_w"]), _p(r["up_s"]),
            _p(r["down_w"]), _p(r["down_s"])))
        return r

    def read_router(self) -> np.ndarray:
        r = np.empty((self.d.experts, self.d.hidden), np.float32)
        _check("colizig_hip_router_read", _lib.hip().colizig_hip_router_read(self.layer, _p(r)))
        return r

    def read_shared(self) -> dict | None:
        if not self.d.shared_inter:
            return None
        H, SI = self.d.hidden, self.d.shared_inter
        r = dict(gate_w=np.empty((SI, H), np.uint8), gate_s=np.empty((nblk(SI), nblk(H)), np.float32),
                 up_w=np.empty((SI, H), np.uint8), up_s=np.empty((nblk(SI), nblk(H)), np.float32),
                 down_w=np.empty((H, SI), np.uint8), down_s=np.empty((nblk(H), nblk(SI)), np.float32),
                 sh_gate=np.empty((H,), np.float32))
        _check("colizig_hip_shared_read", _lib.hip().colizig_hip_shared_read(
            self.layer, *[_p(r[k]) for k in ("gate_w", "gate_s", "up_w", "up_s", "down_w", "down_s", "sh_gate")]))
        return r


def register_layer(layer: int, host: dict) -> Layer:
    """Registers a host-built layer (colizig_amd.synth.make_layer layout)."""
    d = Dims(**host["dims"])
    router = np.asarray(host["router"])
    bf16_router = router.dtype == np.uint16  # BF16 bits: a NativeMatrix bf16 router
    L = Layer.load(layer, d, np.zeros((d.experts, d.hidden), np.float32) if bf16_router else router)
    if bf16_router:
        L.set_router_bf16(router)
    for e, ex in enumerate(host["experts"]):
        L.load_expert(e, ex["gate_w"], ex["gate_s"], ex["up_w"], ex["up_s"], ex["down_w"], ex["down_s"])
    if host.get("shared") is not None:
        s = host["shared"]
        if "native" in s:
            L.set_shared_native(s["gate"], s["up"], s["down"], s["sh_gate"])
        else:
            L.set_shared(s["gate_w"], s["gate_s"], s["up_w"], s["up_s"], s["down_w"], s["down_s"], s["sh_gate"])
    if host.get("router_bias") is not None:
        L.set_router_bias(host["router_bias"])
    return L


class DeviceBuffer:
    """Device allocation through the library (no GPU framework needed)."""

    def __init__(self, nbytes: int):
        self.nbytes = nbytes
        self.ptr = _lib.hip().colizig_hip_malloc(nbytes)
        if not self.ptr:
            raise GpuBackendError("colizig_hip_malloc", -2)

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        _check("colizig_hip_memcpy_htod", _lib.hip().colizig_hip_memcpy_htod(self.ptr, _p(a), a.nbytes))

    def download(self, a: np.ndarray) -> np.ndarray:
        assert a.flags.c_contiguous and a.nbytes <= self.nbytes
        _check("colizig_hip_memcpy_dtoh", _lib.hip().colizig_hip_memcpy_dtoh(_p(a), self.ptr, a.nbytes))
        return a

    def free(self) -> None:
        if self.ptr:
            _lib.hip().colizig_hip_free(self.ptr)
            self.ptr = None


class HostBuffer:
    """Pinned host memory through the library, viewed as a numpy array."""

    def __init__(self, nbytes: int):
        self.nbytes = nbytes
        self.ptr = _lib.hip().colizig_hip_host_alloc(nbytes)
        if not self.ptr:
            raise GpuBackendError("colizig_hip_host_alloc", -2)
        self.array = np.ctypeslib.as_array((ctypes.c_uint8 * nbytes).from_address(self.ptr))

    def view(self, dtype) -> np.ndarray:
        return self.array.view(dtype)

    def free(self) -> None:
        if self.ptr:
            _lib.hip().colizig_hip_host_free(self.ptr)
            self.ptr = None


STREAM_STAT_NAMES = ("hits", "misses", "loads", "evictions", "prefetch_issued", "prefetch_hits",
                     "prefetch_wasted", "bytes_h2d", "slots", "resident", "next_predicted", "next_correct",
                     "last_predicted", "last_correct", "sched_submitted", "sched_deduped", "sched_upgraded",
                     "sched_rejected_full", "sched_serviced_high", "sched_serviced_medium", "sched_serviced_low",
                     "sched_cancelled", "sched_queue_peak", "tok_predicted", "tok_correct", "spec_layers",
                     "spec_stops")


def stream_pool_init(d: Dims, cap_bytes: int) -> None:
    _check("colizig_hip_stream_pool_init", _lib.hip().colizig_hip_stream_pool_init(ctypes.byref(d), cap_bytes))


def stream_stats() -> dict:
    v = (ctypes.c_uint64 * len(STREAM_STAT_NAMES))()
    _check("colizig_hip_stream_stats", _lib.hip().colizig_hip_stream_stats(v, len(STREAM_STAT_NAMES)))
    return dict(zip(STREAM_STAT_NAMES, (int(x) for x in v)))


def host_expert_slab(d: Dims, experts: list) -> tuple[HostBuffer, HostBuffer]:
    """Pinned host slabs of a layer's experts in the HBM slab layout
    (expert e: gate | up | down bytes; its scales likewise)."""
    H, I, E = d.hidden, d.inter, d.experts
    mat, nsc = I * H, nblk(I) * nblk(H)
    wb = HostBuffer(E * 3 * mat)
    sb = HostBuffer(E * 3 * nsc * 4)
    w = wb.view(np.uint8).reshape(E, 3, mat)
    sc = sb.view(np.float32).reshape(E, 3, nsc)
    for e, ex in enumerate(experts):
        for r, k in enumerate(("gate", "up", "down")):
            w[e, r] = np.ascontiguousarray(ex[k + "_w"], np.uint8).ravel()
            sc[e, r] = np.ascontiguousarray(ex[k + "_s"], np.float32).ravel()
    return wb, sb


def stream_layer_from_host(layer: int, wb: HostBuffer, sb: HostBuffer) -> None:
    _check("colizig_hip_layer_stream_from_host",
           _lib.hip().colizig_hip_layer_stream_from_host(layer, wb.ptr, sb.ptr))


def packed_expert_bytes(d: Dims) -> int:
    """Bytes of one expert in a packed host slab: weights, then scales."""
    return 3 * d.inter * d.hidden + 12 * nblk(d.inter) * nblk(d.hidden)


def host_expert_slab_packed(d: Dims, ew: np.ndarray, es: np.ndarray) -> HostBuffer:
    """One pinned slab of E experts, expert e: its gate | up | down bytes
    (ew[e], 3*I*H bytes) then their scales (es[e], f32)."""
    E, P = d.experts, packed_expert_bytes(d)
    w_slot = 3 * d.inter * d.hidden
    hb = HostBuffer(E * P)
    a = hb.view(np.uint8).reshape(E, P)
    a[:, :w_slot] = np.ascontiguousarray(ew, np.uint8).reshape(E, w_slot)
    a[:, w_slot:] = np.ascontiguousarray(es, np.float32).reshape(E, -1).view(np.uint8)
    return hb


def stream_layer_from_host_packed(layer: int, hb: HostBuffer) -> None:
    _check("colizig_hip_layer_stream_from_host_packed",
           _lib.hip().colizig_hip_layer_stream_from_host_packed(layer, hb.ptr))


def plan_hbm(d: Dims, layers: int, hbm_budget: int = 0, max_tokens: int = 1) -> dict:
    """budget.plan (src/runtime/budget.zig:184-264) for one GPU's HBM: the
    resident bytes, and whether every expert stays resident or how many
    expert slots the streaming pool gets (hbm_budget 0: the device's free
    memory less an eighth; needs init)."""
    p = _lib.HbmPlan()
    _check("colizig_hip_plan_hbm", _lib.hip().colizig_hip_plan_hbm(ctypes.byref(d), layers, hbm_budget, max_tokens,
                                                                     ctypes.byref(p)))
    out = {name: getattr(p, name) for name, _ in _lib.HbmPlan._fields_}
    out["reason"] = p.reason.decode()
    return out


def stream_pool_free() -> None:
    _check("colizig_hip_stream_pool_free", _lib.hip().colizig_hip_stream_pool_free())


def stream_log_read() -> np.ndarray:
    """The pool's op log as an [n, 4] uint32 array (op, layer, expert, result)."""
    hip = _lib.hip()
    n = int(hip.colizig_hip_stream_log_read(None, 0))
    out = np.zeros((n, 4), np.uint32)
    if n:
        hip.colizig_hip_stream_log_read(out.ctypes.data_as(ctypes.c_void_p), n)
    return out
