"""The C++ host interface (include/aq_mi355x.hpp) over the C ABI.

tests/cpp/adapter_parity drives aq::engine::runtime::VectorQuantizer,
aq::EuclideanRvq and aq::DacRvq like audio.cpp's call sites would and checks
each result bit for bit against the oracle.  tests/cpp/ref_adapter_parity is
the binding a maintainer adds to the reference's host_ops.cpp, compiled
against the reference's own header (include/engine/framework/runtime/
host_ops.h) where the reference tree is present, and called through the
reference's engine::runtime::VectorQuantizer type.  Without a GPU both must
report that (exit 77) rather than compute anything.
"""

import pathlib
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
BIN = ROOT / "tests" / "cpp" / "adapter_parity"
REF_BIN = ROOT / "tests" / "cpp" / "ref_adapter_parity"


def _binary(path=BIN):
    if not path.exists():
        pytest.skip(f"{path.relative_to(ROOT)} not built (run __graft_entry__.build())")
    return str(path)


def test_header_compiles_standalone(tmp_path):
    src = tmp_path / "inc.cpp"
    src.write_text('#include "aq_mi355x.hpp"\nint main() { return 0; }\n')
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__",
                        "-I/opt/rocm/include", f"-I{ROOT / 'include'}", str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_adapter_without_gpu_reports_it():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    r = subprocess.run([_binary()], capture_output=True, text=True, timeout=120)
    assert r.returncode == 77, r.stdout + r.stderr
    assert "no GPU" in r.stdout


@pytest.mark.gpu
def test_adapter_parity_on_gpu():
    print("[gpu] C++ adapter parity", flush=True)
    r = subprocess.run([_binary()], capture_output=True, text=True, timeout=300)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FAIL" not in r.stdout


def test_reference_header_binding_builds_here():
    """Where the reference tree is present, build() compiles the binding
    against the reference's own VectorQuantizer declaration."""
    if not pathlib.Path("/root/reference/include/engine/framework/runtime/host_ops.h").exists():
        pytest.skip("no reference tree here")
    assert REF_BIN.exists()


def test_reference_header_binding_without_gpu_reports_it():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    r = subprocess.run([_binary(REF_BIN)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 77, r.stdout + r.stderr
    assert "no GPU" in r.stdout


@pytest.mark.gpu
def test_reference_header_binding_parity_on_gpu():
    print("[gpu] reference-header VectorQuantizer binding parity", flush=True)
    r = subprocess.run([_binary(REF_BIN)], capture_output=True, text=True, timeout=300)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FAIL" not in r.stdout
