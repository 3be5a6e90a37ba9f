"""The host code under AddressSanitizer and UndefinedBehaviorSanitizer (the
reference's counterpart is its Debug build's safety checks, README.md:161),
on the CPU: tests/sanitize/Makefile builds the scheduler, predictor, HBM
plan and engine-side loader into a checking program (host_check.cpp, run
against host-only stub backends), and the oracle into a sanitized library
whose own test suite then runs against it in a child process.  Any
sanitizer finding aborts the child, failing the test."""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SAN = os.path.join(HERE, "sanitize")
B = os.path.join(SAN, "_build")
SAN_ENV = {"ASAN_OPTIONS": "abort_on_error=1:detect_leaks=0",
           "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"}


def _build() -> None:
    subprocess.run(["make", "-s", "-C", SAN], check=True)


def test_host_code_under_sanitizers():
    _build()
    env = dict(os.environ, **SAN_ENV)
    env["ASAN_OPTIONS"] = env["ASAN_OPTIONS"].replace("detect_leaks=0", "detect_leaks=1")
    r = subprocess.run([os.path.join(B, "host_check")] + [os.path.join(B, f"stub_{k}.so") for k in
                                                          ("ok", "fail", "missing")],
                       capture_output=True, text=True, timeout=600, env=env)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "host_check: ok" in r.stdout
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr


def _runtime(name: str) -> str:
    path = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    assert os.path.isabs(path) and os.path.exists(path), f"{name} not found"
    return path


def test_oracle_suite_under_sanitizers():
    """tests/test_oracle.py (all of it but the torch comparison, whose ROCm
    libraries are not built for the sanitizer runtime) against the sanitized
    oracle library."""
    _build()
    env = dict(os.environ, **SAN_ENV)
    env["LD_PRELOAD"] = " ".join([_runtime("libasan.so"), _runtime("libubsan.so")])
    env["CZ_ORACLE_LIB"] = os.path.join(B, "libczoracle.so")
    r = subprocess.run([sys.executable, "-m", "pytest", os.path.join(HERE, "test_oracle.py"), "-q", "-x",
                        "-m", "not gpu", "-k", "not torch", "-p", "no:cacheprovider"],
                       capture_output=True, text=True, timeout=900, env=env, cwd=ROOT)
    tail = r.stdout[-3000:] + r.stderr[-3000:]
    assert r.returncode == 0, tail
    assert " passed" in r.stdout and "failed" not in r.stdout, tail
    assert "runtime error" not in r.stderr and "ERROR: AddressSanitizer" not in r.stderr, tail
