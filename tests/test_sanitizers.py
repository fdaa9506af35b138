"""CPU code under AddressSanitizer and UndefinedBehaviorSanitizer.

`make -C oracle sanitize` builds the oracle (oracle/aq_oracle.c) and the
reference harness (oracle/ref_harness.cpp with the reference's ggml and
engine sources) instrumented with ASan + UBSan, at their regular
optimisation and ISA; `make -C tests/cpp .../adapter_parity_asan` builds the
C++ adapter program the same way.  These tests run the oracle's pinning
tests against those builds in a child process (libasan preloaded, leak
detection off: the Python interpreter itself is not instrumented) and fail
on any sanitizer report.  They run where the builds exist (this container;
the GPU box does not receive them).
"""

import os
import pathlib
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
ASAN = ROOT / "oracle" / "_asan"
REPORTS = ("ERROR: AddressSanitizer", "runtime error:", "ERROR: LeakSanitizer")


def _preload():
    """libasan, then libstdc++ (loaded before the instrumented libraries, so
    that the sanitizer's C++ exception interceptor finds __cxa_throw)."""
    libs = []
    for name in ("libasan.so", "libstdc++.so"):
        r = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True)
        p = r.stdout.strip()
        if r.returncode != 0 or not os.path.isabs(p):
            pytest.skip(f"{name} not found")
        libs.append(p)
    return " ".join(libs)


def _env():
    if not (ASAN / "liboracle.so").exists():
        pytest.skip("sanitizer builds absent (make -C oracle sanitize)")
    env = dict(os.environ)
    env.update(LD_PRELOAD=_preload(), ASAN_OPTIONS="detect_leaks=0:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1", AQ_ORACLE_LIB=str(ASAN / "liboracle.so"), OMP_NUM_THREADS="4")
    if (ASAN / "libaqref-native.so").exists():
        env["AQ_REF_DIR"] = str(ASAN)
    return env


def test_oracle_and_reference_harness_under_sanitizers():
    env = _env()
    sel = ["tests/test_oracle_shapes.py", "tests/test_oracle.py", "-k",
           "not full_shape and not golden and not qwen3 and not 1024 and not fish_mixed and not 750"]
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", *sel], cwd=ROOT, env=env,
                       capture_output=True, text=True, timeout=900)
    out = r.stdout + r.stderr
    assert not any(s in out for s in REPORTS), out[-4000:]
    assert r.returncode == 0, out[-4000:]


def test_adapter_program_under_sanitizers():
    binary = ROOT / "tests" / "cpp" / "adapter_parity_asan"
    if not binary.exists():
        pytest.skip("tests/cpp/adapter_parity_asan not built")
    env = _env()
    env.pop("LD_PRELOAD")   # the program links libasan itself
    r = subprocess.run([str(binary)], capture_output=True, text=True, timeout=300, env=env)
    out = r.stdout + r.stderr
    assert not any(s in out for s in REPORTS), out[-4000:]
    assert r.returncode in (0, 77), out[-4000:]
