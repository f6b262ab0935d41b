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


def test_paged_operand_checks_on_the_host():
    """sandy_hip_paged_to_dense / _stage reject descriptors the reference's
    pack_tensor_arg rejects (CudaKernelUtils.cuh:290-374) before any device
    work, so these run without a GPU."""
    import pytest

    def pt(**kw):
        s = _lib.SandyPagedTensor()
        s.pages, s.dtype, s.rank = 0x1000, _lib.F32, 3
        for i, d in enumerate([2, 3, 4]):
            s.dims[i] = d
        s.grow_dim, s.page_size, s.page_count = 1, 2, 2
        for k, v in kw.items():
            setattr(s, k, v)
        return ctypes.pointer(s)

    dst = _lib.SandyTensor()
    dst.rank, dst.dtype = 3, _lib.F32
    for i, (d, st) in enumerate([(2, 12), (3, 4), (4, 1)]):
        dst.dims[i], dst.strides[i] = d, st
    dst.data = 0x2000
    cases = [
        (pt(page_size=3), "page_size must be a power of two"),
        (pt(page_size=0), "page_size must be > 0"),
        (pt(grow_dim=3), "grow_dim out of range"),
        (pt(page_count=-1), "page_count must be >= 0"),
        (pt(pages=None), "page table is null"),
        (pt(dtype=_lib.U8), "unsupported dtype"),
    ]
    for p, msg in cases:
        with pytest.raises(_lib.SandyError, match=msg):
            _lib.call("sandy_hip_paged_to_dense", p, ctypes.byref(dst), stream=0)
    bad = _lib.SandyTensor.from_buffer_copy(dst)
    bad.dims[2] = 5
    with pytest.raises(_lib.SandyError, match="destination must be a contiguous tensor"):
        _lib.call("sandy_hip_paged_to_dense", pt(), ctypes.byref(bad), stream=0)
    with pytest.raises(_lib.SandyError, match="slot out of range"):
        _lib.call("sandy_hip_paged_stage", pt(), ctypes.c_int32(-1), ctypes.byref(dst), stream=0)
