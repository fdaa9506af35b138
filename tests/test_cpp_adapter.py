"""The C++ host interface (include/aq_mi355x.hpp) over the C ABI.

tests/cpp/adapter_parity drives aq::engine::runtime::VectorQuantizer,
aq::EuclideanRvq and aq::DacRvq like audio.cpp's call sites would and checks
each result bit for bit against the oracle.  Without a GPU it must report
that (exit 77) rather than compute anything.
"""

import pathlib
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
BIN = ROOT / "tests" / "cpp" / "adapter_parity"


def _binary():
    if not BIN.exists():
        pytest.skip("tests/cpp/adapter_parity not built (run __graft_entry__.build())")
    return str(BIN)


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
