"""CPU checks of the C ABI: the library loads (no GPU needed to dlopen) and
exports every entry point include/aq_mi355x.h declares."""

import re

import pytest

from conftest import ROOT


def declared_symbols():
    text = (ROOT / "include" / "aq_mi355x.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+char\s*\*\s*|aq_status\s+|int\s+)(aq_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "aq_dac_encode" in syms and "aq_ctx_create" in syms


def test_library_exports_every_declared_symbol():
    import aqmi

    if not aqmi.LIB_PATH.exists():
        pytest.fail("libaq_mi355x.so is not built: run python audio.cpp_amd/build.py")
    lib = aqmi.load_library()
    for name in declared_symbols():
        assert hasattr(lib, name), f"{name} declared in aq_mi355x.h but not exported"
    assert lib.aq_abi_version() == 1


def test_binding_lists_every_declared_symbol():
    import aqmi

    assert set(declared_symbols()) == set(aqmi.EXPORTED)


def test_context_without_gpu_fails_loudly():
    import torch

    import aqmi

    if torch.cuda.is_available():
        pytest.skip("GPU present")
    with pytest.raises(RuntimeError):
        aqmi.Context(0)
