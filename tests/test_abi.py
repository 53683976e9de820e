"""CPU-side checks of the drop-in boundary: the HIP library is built, loads,
and exports every entry point include/rusticide_hip.h declares."""

import ctypes
import os
import re

import pytest

import rusticide_amd as R

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rusticide_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rh_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    syms = declared_symbols()
    for s in ("rh_init", "rh_matrix_load", "rh_matmul_batch", "rh_matmul_batch_device",
              "rh_matvec_batch", "rh_quantize", "rh_ternary_dot_i32", "rh_last_error"):
        assert s in syms


def test_library_loads_and_exports_every_declared_symbol():
    if not os.path.exists(R.library_path()):
        pytest.fail("librusticide_hip.so is not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(R.library_path())
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_adapter_name_needs_no_device():
    assert R.lib().rh_adapter_name() == b"hip-gfx950"


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(R, "_LIB", str(tmp_path / "absent.so"))
    monkeypatch.setattr(R, "_lib", None)
    with pytest.raises(R.RusticideError):
        R.lib()
