"""The reference-side binding (sandyrt_amd/reference_binding/
HipKernelDispatch.cpp: KernelIR op -> sandy_hip_* call, the place
CudaDevice::run calls launch_cuda_*, src/device/cuda/CudaDevice.cpp:520-578)
compiles against the reference's own headers and covers every KernelIR
OpKind.  CPU only; skipped where the reference tree is absent."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference/src"
SRC = os.path.join(ROOT, "sandyrt_amd", "reference_binding", "HipKernelDispatch.cpp")
CLANG = "/opt/rocm/lib/llvm/bin/clang++"


def _compiler():
    if not os.path.isdir(REF):
        pytest.skip("reference tree not present")
    return CLANG if os.path.exists(CLANG) else (shutil.which("clang++") or pytest.skip("no clang++"))


def test_dispatch_compiles_against_reference_headers(tmp_path):
    cmd = [_compiler(), "-std=c++20", "-c", "-Werror=switch", "-Werror=return-type", f"-I{REF}/core", f"-I{REF}/ir",
           f"-I{REF}/device", "-I" + os.path.join(ROOT, "include"), SRC, "-o", str(tmp_path / "dispatch.o")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_dispatch_names_every_op_kind():
    header = open(os.path.join(REF if os.path.isdir(REF) else "/nonexistent", "ir", "KernelIR.h")).read() \
        if os.path.isdir(REF) else pytest.skip("reference tree not present")
    kinds = re.search(r"enum class OpKind \{(.*?)\};", header, re.S).group(1)
    kinds = [k.strip() for k in kinds.split(",") if k.strip()]
    body = open(SRC).read()
    missing = [k for k in kinds if f"OpKind::{k}:" not in body]
    assert not missing, missing


def test_dispatch_calls_only_declared_entry_points():
    declared = set(re.findall(r"\b(sandy_hip_\w+)\s*\(", open(os.path.join(ROOT, "include", "sandyrt_hip.h")).read()))
    used = set(re.findall(r"\b(sandy_hip_\w+)\s*\(", open(SRC).read()))
    assert used and used <= declared, used - declared
