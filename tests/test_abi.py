"""C-ABI checks that need no GPU: the libraries load, export every symbol
include/colizig_hip.h declares, and take the reference's error paths when no
device answers (gpu.zig:72-109, colizig_cuda.cu:171-187, 228-232)."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from colizig_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "colizig_hip.h")


def header_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(colizig_(?:cuda|hip)_\w+)\s*\(", text)))


def has_device() -> bool:
    return _lib.hip().colizig_cuda_init() == 0


def test_header_declares_reference_abi():
    fns = header_functions()
    for name in ("colizig_cuda_init", "colizig_cuda_device_name", "colizig_cuda_set_vram_budget",
                 "colizig_cuda_stats", "colizig_cuda_shutdown", "colizig_cuda_matmul_fp8"):
        assert name in fns


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.HIP_LIB)
    missing = [n for n in header_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # and the bindings describe exactly the declared set
    assert sorted(_lib.SIGNATURES) == header_functions()


def test_exported_symbols_are_c_abi():
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.HIP_LIB], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (colizig_\w+)", out))
    assert set(header_functions()) <= exported


def test_loader_exports():
    lib = ctypes.CDLL(_lib.LOADER_LIB)
    for n in _lib.LOADER_SIGNATURES:
        assert hasattr(lib, n), n


def test_no_device_error_paths():
    if has_device():
        pytest.skip("a GPU is present")
    h = _lib.hip()
    assert h.colizig_cuda_init() == -1
    assert h.colizig_cuda_device_name() == b""
    x = np.zeros(4, np.float32)
    y = np.zeros(4, np.float32)
    w = np.zeros(16, np.uint8)
    s = np.ones(1, np.float32)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    assert h.colizig_cuda_matmul_fp8(p(y), p(x), p(w), p(s), 1, 4, 4, 0) == -1
    assert h.colizig_hip_moe_forward(0, p(x), 1, p(y), None, None) == -1
    assert h.colizig_hip_dequant_fp8(p(y), p(w), p(s), 2, 2) == -1
    assert h.colizig_hip_layer_synth(0, 1, 0.02, 0.02) == -1
    h.colizig_cuda_set_vram_budget(1 << 30)  # no-op before init
    h.colizig_cuda_stats(None, None, None, None)  # NULL-tolerant
    v = [ctypes.c_uint64(7) for _ in range(4)]
    h.colizig_cuda_stats(*[ctypes.byref(a) for a in v])
    assert [a.value for a in v] == [0, 0, 0, 0]
    h.colizig_cuda_shutdown()  # safe when not initialised
    assert h.colizig_hip_malloc(1024) is None
    # the multi-matrix GEMV and the prediction counters refuse before init
    ys = (ctypes.c_void_p * 1)(p(y).value)
    ks = (ctypes.c_uint64 * 1)(1)
    os_ = (ctypes.c_int * 1)(4)
    assert h.colizig_hip_matmul_fp8_dev_multi(1, ys, ks, os_, p(x), 1, 4, None) == -1
    st = np.zeros(2, np.uint64)
    assert h.colizig_hip_fused_predict_stats(p(st)) == -1
    assert h.colizig_hip_fused_placement() == -1


def test_host_side_switches():
    """Mode switches that are host state only: each returns the previous
    setting and refuses a value outside its range (no device needed)."""
    h = _lib.hip()
    prev = h.colizig_hip_set_fused_predict(0)
    assert prev in (0, 1, 2, 3)
    try:
        assert h.colizig_hip_set_fused_predict(3) == 0
        assert h.colizig_hip_set_fused_predict(4) == -1
        assert h.colizig_hip_set_fused_predict(-1) == -1
        assert h.colizig_hip_set_fused_predict(1) == 3
    finally:
        h.colizig_hip_set_fused_predict(prev)
    p8 = h.colizig_hip_set_prefill_fp8(0)
    try:
        assert h.colizig_hip_set_prefill_fp8(1) == 0
        assert h.colizig_hip_set_prefill_fp8(0) == 1
    finally:
        h.colizig_hip_set_prefill_fp8(p8)
    ff = h.colizig_hip_set_fused_fault(2)
    try:
        assert h.colizig_hip_set_fused_fault(-7) == 2
        assert h.colizig_hip_set_fused_fault(-1) == -1  # any negative position is "off"
    finally:
        h.colizig_hip_set_fused_fault(ff)
    fd = h.colizig_hip_set_fused_decode(0)
    try:
        assert h.colizig_hip_set_fused_decode(1) == 0
    finally:
        h.colizig_hip_set_fused_decode(fd)


def test_loader_falls_back_without_device():
    """gpu.zig:91-96: init rc != 0 -> one line, backend unavailable."""
    if has_device():
        pytest.skip("a GPU is present")
    ld = _lib.loader()
    err = ctypes.create_string_buffer(256)
    assert ld.czgpu_init(_lib.HIP_LIB.encode(), err, 256) == 0
    assert b"no usable GPU device (colizig_cuda_init rc=-1) - using CPU" in err.value
    assert ld.czgpu_available() == 0
    x = np.zeros(4, np.float32)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    assert ld.czgpu_matmul_fp8(p(x), p(x), p(x), p(x), 1, 1, 1, 0) == 0  # false -> CPU path
    ld.czgpu_set_vram_budget(1 << 30)  # no-op when unavailable
    ld.czgpu_deinit()


def test_loader_missing_library():
    """gpu.zig:79-82"""
    ld = _lib.loader()
    err = ctypes.create_string_buffer(256)
    assert ld.czgpu_init(b"/nonexistent/libcolizig_hip.so", err, 256) == 0
    assert b"not found - using CPU" in err.value
    assert ld.czgpu_available() == 0


def test_loader_missing_symbol(tmp_path):
    """gpu.zig:84-89, 111-114: any missing symbol -> that name, CPU."""
    src = tmp_path / "stub.c"
    src.write_text("int colizig_cuda_init(void){return 0;}\n"
                   "const char* colizig_cuda_device_name(void){return \"stub\";}\n"
                   "void colizig_cuda_shutdown(void){}\n")
    so = tmp_path / "libstub.so"
    subprocess.run(["gcc", "-shared", "-fPIC", "-o", str(so), str(src)], check=True)
    ld = _lib.loader()
    err = ctypes.create_string_buffer(256)
    assert ld.czgpu_init(str(so).encode(), err, 256) == 0
    assert b"colizig_cuda_matmul_fp8 missing" in err.value
    assert ld.czgpu_available() == 0


def test_host_expf_matches_oracle_bitwise(oracle_lib):
    """The library's f32 exp (the one the router runs on the GPU), evaluated on
    the host, equals the oracle's bit for bit on 2^24 inputs around the
    router's operating range and on a sparse sweep of all patterns."""
    a = ctypes.cast(_lib.hip().colizig_hip_expf_host, ctypes.c_void_p).value
    b = oracle_lib.fn_ptr("czo_expf")
    first = ctypes.c_uint32()
    f = oracle_lib.lib().czo_f32fn_compare
    lo = int(np.array([-16.0], np.float32).view(np.uint32)[0])
    assert f(a, b, 0x80000000, 0x80000000 + (1 << 22), 8, ctypes.byref(first)) == 0
    assert f(a, b, lo - (1 << 22), lo + (1 << 22), 8, ctypes.byref(first)) == 0
    assert f(a, b, 0x3F800000 - (1 << 21), 0x3F800000 + (1 << 21), 8, ctypes.byref(first)) == 0
    for start in range(0, 1 << 32, 1 << 27):
        assert f(a, b, start, start + 4096, 8, ctypes.byref(first)) == 0, hex(first.value)
