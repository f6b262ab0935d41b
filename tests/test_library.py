"""CPU checks of the product boundary: the C-ABI library builds for gfx950,
loads, and exports every entry point include/sandyrt_hip.h declares (no
compute calls -- there is no GPU here)."""
import ctypes
import os
import re

from sandyrt_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "sandyrt_hip.h")).read()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(sandy_hip_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "sandy_hip_paged_attention" in syms and "sandy_hip_norm" in syms
    assert len(syms) >= 15


def test_library_exports_every_declared_symbol():
    assert os.path.exists(_lib.LIB_PATH), "run sandyrt_amd.build.build() first"
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, f"not exported: {missing}"
    assert set(_lib.exported_symbols()) == set(declared_symbols())


def test_version_string():
    assert _lib.lib().sandy_hip_version().decode().startswith("sandyrt-hip")


def test_code_object_targets_gfx950():
    data = open(_lib.LIB_PATH, "rb").read()
    assert b"gfx950" in data
