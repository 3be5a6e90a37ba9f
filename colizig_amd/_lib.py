"""ctypes bindings of libcolizig_hip.so (declarations in include/colizig_hip.h).

The library must be built (colizig_amd.build); loading fails loudly when it is
missing - there is no CPU fallback inside this package.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
HIP_LIB = os.path.join(HERE, "libcolizig_hip.so")
LOADER_LIB = os.path.join(HERE, "libcolizig_gpu.so")

c_f32p = ctypes.POINTER(ctypes.c_float)
c_u8p = ctypes.POINTER(ctypes.c_uint8)
c_u32p = ctypes.POINTER(ctypes.c_uint32)
c_u64p = ctypes.POINTER(ctypes.c_uint64)
vp = ctypes.c_void_p


class Dims(ctypes.Structure):
    """`colizig_dims` - src/qwen38/moe.zig:23-46 `Dims`."""

    _fields_ = [
        ("hidden", ctypes.c_uint32),
        ("experts", ctypes.c_uint32),
        ("topk", ctypes.c_uint32),
        ("inter", ctypes.c_uint32),
        ("shared_inter", ctypes.c_uint32),
        ("norm_topk", ctypes.c_uint32),
    ]

    def has_shared(self) -> bool:
        """moe.zig:32-34"""
        return self.shared_inter != 0


class HbmPlan(ctypes.Structure):
    """`colizig_hbm_plan` - budget.plan's Plan (src/runtime/budget.zig:66-90) for HBM."""

    _fields_ = [
        ("hbm_budget", ctypes.c_uint64),
        ("per_expert_bytes", ctypes.c_uint64),
        ("per_layer_fixed", ctypes.c_uint64),
        ("scratch", ctypes.c_uint64),
        ("fixed_resident", ctypes.c_uint64),
        ("expert_bytes", ctypes.c_uint64),
        ("total", ctypes.c_uint64),
        ("all_resident", ctypes.c_uint32),
        ("pool_slots", ctypes.c_uint32),
        ("expert_cap", ctypes.c_uint32),
        ("ladder_cap", ctypes.c_uint32),
        ("fits", ctypes.c_uint32),
        ("reason", ctypes.c_char * 128),
    ]


# name -> (restype, argtypes)
SIGNATURES = {
    # the existing backend ABI (src/backend/gpu.zig:20-34)
    "colizig_cuda_init": (ctypes.c_int, []),
    "colizig_cuda_device_name": (ctypes.c_char_p, []),
    "colizig_cuda_set_vram_budget": (None, [ctypes.c_uint64]),
    "colizig_cuda_stats": (None, [c_u64p, c_u64p, c_u64p, c_u64p]),
    "colizig_cuda_shutdown": (None, []),
    "colizig_cuda_matmul_fp8": (ctypes.c_int, [vp, vp, vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_uint64]),
    "colizig_hip_matrix_load": (ctypes.c_int, [ctypes.c_uint64, vp, vp, ctypes.c_int, ctypes.c_int]),
    "colizig_hip_matmul_fp8_dev": (ctypes.c_int, [vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_uint64, vp]),
    "colizig_hip_matmul_fp8_dev_multi": (ctypes.c_int, [ctypes.c_int, vp, vp, vp, vp, ctypes.c_int, ctypes.c_int, vp]),
    "colizig_hip_stream_usage": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, vp]),
    "colizig_hip_usage_read": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, vp]),
    "colizig_hip_usage_reset": (ctypes.c_int, []),
    "colizig_hip_stream_warm": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, vp]),
    "colizig_hip_stream_evict_all": (ctypes.c_int, []),
    "colizig_hip_matrix_load_bf16": (ctypes.c_int, [ctypes.c_uint64, vp, ctypes.c_int, ctypes.c_int]),
    "colizig_hip_matmul_bf16_dev": (ctypes.c_int, [vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_uint64, vp]),
    # extensions
    "colizig_hip_dequant_fp8": (ctypes.c_int, [vp, vp, vp, ctypes.c_int, ctypes.c_int]),
    "colizig_hip_layer_init": (ctypes.c_int, [ctypes.c_uint32, ctypes.POINTER(Dims), vp]),
    "colizig_hip_expert_load": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_uint32, vp, vp, vp, vp, vp, vp]),
    "colizig_hip_layer_set_shared": (ctypes.c_int, [ctypes.c_uint32, vp, vp, vp, vp, vp, vp, vp]),
    "colizig_hip_layer_set_router_bias": (ctypes.c_int, [ctypes.c_uint32, vp]),
    "colizig_hip_moe_forward": (ctypes.c_int, [ctypes.c_uint32, vp, ctypes.c_int, vp, vp, vp]),
    "colizig_hip_moe_forward_dev": (ctypes.c_int, [ctypes.c_uint32, vp, ctypes.c_int, vp, vp, vp, vp]),
    "colizig_hip_moe_forward_dev_noalloc": (ctypes.c_int, [ctypes.c_uint32, vp, ctypes.c_int, vp, vp, vp, vp]),
    "colizig_hip_chain_decode": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_uint32, vp, ctypes.c_int,
                                                ctypes.c_float, vp, vp, vp, vp]),
    "colizig_hip_chain_graph_create": (ctypes.c_int64, [ctypes.c_uint32, ctypes.c_uint32, vp, ctypes.c_int,
                                                        ctypes.c_float]),
    "colizig_hip_graph_launch": (ctypes.c_int, [ctypes.c_int64, vp]),
    "colizig_hip_graph_destroy": (None, [ctypes.c_int64]),
    "colizig_hip_chain_kernel_times": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_uint32, vp, ctypes.c_int,
                                                      ctypes.c_float, ctypes.c_int, vp]),
    "colizig_hip_expert_slab_read": (ctypes.c_int, [ctypes.c_uint32, vp, vp]),
    "colizig_hip_set_fused_decode": (ctypes.c_int, [ctypes.c_int]),
    "colizig_hip_set_fused_predict": (ctypes.c_int, [ctypes.c_int]),
    "colizig_hip_fused_predict_stats": (ctypes.c_int, [ctypes.c_void_p]),
    "colizig_hip_fused_placement": (ctypes.c_int, []),
    "colizig_hip_set_fused_fault": (ctypes.c_int, [ctypes.c_int]),
    "colizig_hip_fused_decode_active": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int]),
    "colizig_hip_chain_fused_times": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_uint32, vp, ctypes.c_float,
                                                     ctypes.c_int, vp]),
    "colizig_hip_layer_synth": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float, ctypes.c_float]),
    "colizig_hip_expert_read": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_uint32, vp, vp, vp, vp, vp, vp]),
    "colizig_hip_router_read": (ctypes.c_int, [ctypes.c_uint32, vp]),
    "colizig_hip_shared_read": (ctypes.c_int, [ctypes.c_uint32, vp, vp, vp, vp, vp, vp, vp]),
    "colizig_hip_stream_pool_init": (ctypes.c_int, [ctypes.POINTER(Dims), ctypes.c_uint64]),
    "colizig_hip_layer_stream_from_host": (ctypes.c_int, [ctypes.c_uint32, vp, vp]),
    "colizig_hip_stream_decode": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_uint32, vp, ctypes.c_int, ctypes.c_float]),
    "colizig_hip_stream_stats": (ctypes.c_int, [c_u64p, ctypes.c_int]),
    "colizig_hip_stream_stats_reset": (ctypes.c_int, []),
    "colizig_hip_stream_pool_free": (ctypes.c_int, []),
    "colizig_hip_set_prefill_fp8": (ctypes.c_int, [ctypes.c_int]),
    "colizig_hip_work_bytes": (ctypes.c_int, [c_u64p]),
    "colizig_hip_layer_set_router_bf16": (ctypes.c_int, [ctypes.c_uint32, vp]),
    "colizig_hip_layer_set_shared_native": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_int, vp, vp, vp, vp]),
    "colizig_hip_plan_hbm": (ctypes.c_int, [ctypes.POINTER(Dims), ctypes.c_uint32, ctypes.c_uint64, ctypes.c_uint32,
                                            ctypes.POINTER(HbmPlan)]),
    "colizig_hip_layer_stream_from_host_packed": (ctypes.c_int, [ctypes.c_uint32, vp]),
    "colizig_hip_stream_set_predict": (ctypes.c_int, [ctypes.c_int]),
    "colizig_hip_stream_log": (ctypes.c_int, [ctypes.c_int]),
    "colizig_hip_stream_log_read": (ctypes.c_int64, [vp, ctypes.c_uint64]),
    "colizig_hip_sched_create": (ctypes.c_int64, [ctypes.c_uint32]),
    "colizig_hip_sched_destroy": (None, [ctypes.c_int64]),
    "colizig_hip_sched_submit": (ctypes.c_int, [ctypes.c_int64, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int]),
    "colizig_hip_sched_next": (ctypes.c_int, [ctypes.c_int64, c_u32p, c_u32p]),
    "colizig_hip_sched_cancel": (ctypes.c_int, [ctypes.c_int64, ctypes.c_uint32, ctypes.c_uint32]),
    "colizig_hip_sched_has": (ctypes.c_int, [ctypes.c_int64, ctypes.c_uint32, ctypes.c_uint32]),
    "colizig_hip_sched_stats": (ctypes.c_int, [ctypes.c_int64, c_u64p, ctypes.c_int]),
    "colizig_hip_predictor_create": (ctypes.c_int64, [ctypes.c_uint32]),
    "colizig_hip_predictor_destroy": (None, [ctypes.c_int64]),
    "colizig_hip_predictor_record": (ctypes.c_int, [ctypes.c_int64, ctypes.c_uint32, vp, ctypes.c_uint32]),
    "colizig_hip_predictor_predict": (ctypes.c_int, [ctypes.c_int64, ctypes.c_uint32, vp, ctypes.c_uint32]),
    "colizig_hip_predictor_stats": (ctypes.c_int, [ctypes.c_int64, c_u64p, c_u64p]),
    "colizig_hip_predictor_predict_scored": (ctypes.c_int, [ctypes.c_int64, ctypes.c_uint32, vp, ctypes.c_uint32]),
    "colizig_hip_host_alloc": (vp, [ctypes.c_uint64]),
    "colizig_hip_host_free": (None, [vp]),
    "colizig_hip_expf_dev": (ctypes.c_int, [vp, vp, ctypes.c_int]),
    "colizig_hip_expf_host": (ctypes.c_float, [ctypes.c_float]),
    "colizig_hip_malloc": (vp, [ctypes.c_uint64]),
    "colizig_hip_free": (None, [vp]),
    "colizig_hip_memcpy_htod": (ctypes.c_int, [vp, vp, ctypes.c_uint64]),
    "colizig_hip_memcpy_dtoh": (ctypes.c_int, [vp, vp, ctypes.c_uint64]),
    "colizig_hip_memset": (ctypes.c_int, [vp, ctypes.c_int, ctypes.c_uint64]),
    "colizig_hip_stream": (vp, []),
    "colizig_hip_sync": (ctypes.c_int, []),
    "colizig_hip_event_create": (ctypes.c_int64, []),
    "colizig_hip_event_record": (ctypes.c_int, [ctypes.c_int64, vp]),
    "colizig_hip_event_elapsed_ms": (ctypes.c_float, [ctypes.c_int64, ctypes.c_int64]),
    "colizig_hip_event_destroy": (None, [ctypes.c_int64]),
    "colizig_hip_last_error": (ctypes.c_char_p, []),
}

LOADER_SIGNATURES = {
    "czgpu_init": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]),
    "czgpu_deinit": (None, []),
    "czgpu_available": (ctypes.c_int, []),
    "czgpu_has_moe": (ctypes.c_int, []),
    "czgpu_device_name": (ctypes.c_char_p, []),
    "czgpu_set_vram_budget": (None, [ctypes.c_uint64]),
    "czgpu_stats_line": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_size_t]),
    "czgpu_matmul_fp8": (ctypes.c_int, [vp, vp, vp, vp, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t,
                                        ctypes.c_uint64]),
    "czgpu_moe_forward": (ctypes.c_int, [ctypes.c_uint32, vp, ctypes.c_size_t, vp, vp, vp]),
}

_hip = None
_loader = None


def _bind(lib, sigs):
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def hip() -> ctypes.CDLL:
    """The HIP library (raises if it has not been built)."""
    global _hip
    if _hip is None:
        if not os.path.exists(HIP_LIB):
            raise RuntimeError(f"{HIP_LIB} is missing: build it with `python -m colizig_amd.build`")
        _hip = _bind(ctypes.CDLL(HIP_LIB, mode=ctypes.RTLD_GLOBAL), SIGNATURES)
    return _hip


def loader() -> ctypes.CDLL:
    """The host loader library (gpu.zig counterpart)."""
    global _loader
    if _loader is None:
        if not os.path.exists(LOADER_LIB):
            raise RuntimeError(f"{LOADER_LIB} is missing: build it with `python -m colizig_amd.build`")
        _loader = _bind(ctypes.CDLL(LOADER_LIB), LOADER_SIGNATURES)
    return _loader


def last_error() -> str:
    msg = hip().colizig_hip_last_error()
    return msg.decode() if msg else ""
