"""The reference-side binding (sandyrt_amd/reference_binding/
HipKernelDispatch.cpp: KernelIR op -> sandy_hip_* call, the place
CudaDevice::run calls launch_cuda_*, src/device/cuda/CudaDevice.cpp:520-578)
is compiled with the reference's own src/ir and src/core sources and a
recording stand-in of the C ABI (tests/binding/record_stub.cpp), and
tests/binding/dispatch_driver.cpp runs ops of every KernelIR OpKind through
it.  The tests check the descriptors each entry point receives, the NULL
optionals, the paged-operand handling (staged for the families whose
reference kernels read paged inputs through load_float / load_int,
src/device/cuda/CudaKernelUtils.cuh:82-157, rejected with the reference's
wording elsewhere) and error propagation.  CPU only; skipped where the
reference tree is absent."""
import json
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference/src"
BIND = os.path.join(ROOT, "sandyrt_amd", "reference_binding")
SRC = os.path.join(BIND, "HipKernelDispatch.cpp")
CLANG = "/opt/rocm/lib/llvm/bin/clang++"
STAGED = 0x5000000  # record_stub.cpp: staged slot s answers data = STAGED + s


def _compiler():
    if not os.path.isdir(REF):
        pytest.skip("reference tree not present")
    return CLANG if os.path.exists(CLANG) else (shutil.which("clang++") or pytest.skip("no clang++"))


@pytest.fixture(scope="module")
def cases(tmp_path_factory):
    cxx = _compiler()
    exe = str(tmp_path_factory.mktemp("binding") / "dispatch_driver")
    srcs = [SRC, os.path.join(ROOT, "tests", "binding", "dispatch_driver.cpp"),
            os.path.join(ROOT, "tests", "binding", "record_stub.cpp")]
    srcs += [f"{REF}/ir/{f}" for f in ("KernelIR.cpp", "MidIR.cpp", "HighIR.cpp")]
    srcs += [f"{REF}/core/{f}" for f in sorted(os.listdir(f"{REF}/core")) if f.endswith(".cpp")]
    cmd = [cxx, "-std=c++20", "-O1", "-Werror=switch", "-Werror=return-type", f"-I{REF}/core", f"-I{REF}/ir",
           f"-I{REF}/device", "-I" + os.path.join(ROOT, "include"), "-I" + BIND, *srcs, "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    out = {}
    for line in r.stdout.splitlines():
        c = json.loads(line)
        out[c["case"]] = c
    return out


def _ok(c, calls):
    assert c["ok"], c["error"]
    assert [x["call"] for x in c["calls"]] == calls
    return c["calls"]


def _err(c, msg):
    assert not c["ok"]
    assert c["error"] == msg
    return c["calls"]


def _dense(t, addr, dims, dtype=0, strides=None, offset=0):
    assert int(t["data"], 16) == addr
    assert t["dims"] == dims and t["dtype"] == dtype and t["offset"] == offset
    if strides is None:
        strides, s = [], 1
        for d in reversed(dims):
            strides.insert(0, s)
            s *= d
    assert t["strides"] == strides


def test_every_op_kind_is_run(cases):
    header = open(os.path.join(REF, "ir", "KernelIR.h")).read()
    kinds = re.search(r"enum class OpKind \{(.*?)\};", header, re.S).group(1)
    kinds = [k.strip() for k in kinds.split(",") if k.strip()]
    snake = {k: re.sub(r"(?<!^)(?=[A-Z])", "_", k.replace("Kernel", "").replace("RoPE", "Rope")
                       .replace("MatMul", "Matmul").replace("TopK", "Topk")).lower() for k in kinds}
    prefix = {"rope": "rope", "norm": "rms_norm", "layout_transform": "layout_", "reduction": "reduction_",
              "matmul": "matmul", "moe_matmul": "moe_matmul", "moe_gather": "moe_gather",
              "moe_scatter_sum": "moe_scatter_sum", "attention": "attention_", "topk": "topk",
              "sliding_query_key_score": "sliding_query_key_score"}
    for k, s in snake.items():
        p = prefix.get(s, s)
        assert any(name.startswith(p) for name in cases), (k, p)


def test_boundary_ops_rejected(cases):
    for name in ("input", "tensor_tuple_create", "device_transfer", "paged_append"):
        assert _err(cases[name], "hip device cannot run boundary op") == []
    _err(cases["sliding_query_key_score"], "hip device: sliding_query_key_score is not part of this backend")


def test_layout_transform(cases):
    (c,) = _ok(cases["layout_transpose"], ["sandy_hip_layout_transform"])
    _dense(c["in"], 0x1000, [3, 4], strides=[1, 3], offset=2)
    _dense(c["out"], 0x2000, [3, 4])
    assert c["kind"] == 1  # LayoutTransformKind::Transpose
    # CudaLayoutTransformKernels.cu:65-66
    assert _err(cases["layout_paged"], "hip layout_transform does not support paged tensors") == []


def test_elementwise_descriptors(cases):
    (c,) = _ok(cases["elementwise_dense"], ["sandy_hip_elementwise"])
    assert [(n["id"], n["op"], n["input"], n["constant"], n["operands"]) for n in c["nodes"]] == [
        (0, 0, 0, 0, []), (1, 0, 1, 0, []), (2, 1, 0, 0.5, []), (3, 4, 0, 0, [0, 2]), (4, 2, 0, 0, [3, 1])]
    assert c["result"] == 4 and c["broadcast"] == [0, 1]
    _dense(c["inputs"][0], 0x1000, [2, 3, 4], 2)
    _dense(c["inputs"][1], 0x2000, [4], 2)
    _dense(c["out"], 0x3000, [2, 3, 4], 2)
    _err(cases["elementwise_three_operands"], "hip elementwise scalar node has more than two operands")
    _err(cases["elementwise_arity"], "hip elementwise input arity mismatch")


def test_elementwise_reads_paged_inputs(cases):
    # RunElementwiseReadsPagedTensorF32 (test/engine/CudaDeviceTest.cpp:685-760): [2, T, 4] grows along dim 1
    stage, ew = _ok(cases["elementwise_paged"], ["sandy_hip_paged_stage", "sandy_hip_elementwise"])
    assert stage["slot"] == 0
    assert stage["src"] == {"pages": "1000", "dtype": 0, "dims": [2, 3, 4], "grow_dim": 1, "page_size": 2,
                            "page_count": 2}
    _dense(ew["inputs"][0], STAGED, [2, 3, 4])
    _dense(ew["inputs"][1], 0x2000, [4])
    s0, s1, ew = _ok(cases["elementwise_paged_both"],
                     ["sandy_hip_paged_stage", "sandy_hip_paged_stage", "sandy_hip_elementwise"])
    assert (s0["slot"], s1["slot"]) == (0, 1)
    _dense(ew["inputs"][1], STAGED + 1, [2, 3, 4])


def test_paged_view_rules(cases):
    # pack_tensor_arg (CudaKernelUtils.cuh:303-306) and CudaDevice::run's dense outputs (CudaDevice.cpp:497-503)
    assert _err(cases["elementwise_paged_noncontiguous"], "hip paged tensor view must be contiguous") == []
    assert _err(cases["elementwise_paged_offset"], "hip paged tensor storage offset must be zero") == []
    assert _err(cases["elementwise_paged_output"], "hip device kernel output must be a dense tensor view") == []


def test_errors_come_back_as_result(cases):
    assert len(_err(cases["elementwise_error"], "sandy_hip_elementwise failed in the stub")) == 1
    assert len(_err(cases["softmax_error"], "sandy_hip_softmax failed in the stub")) == 1


def test_reduction(cases):
    (c,) = _ok(cases["reduction_sum"], ["sandy_hip_reduce_sum"])
    _dense(c["x"], 0x1000, [4, 8])
    assert c["axis"] == 1 and c["keep_dims"] == 1
    _, c = _ok(cases["reduction_paged"], ["sandy_hip_paged_stage", "sandy_hip_reduce_sum"])
    _dense(c["x"], STAGED, [4, 8])
    _err(cases["reduction_max"], "hip reduction only supports sum")
    _err(cases["reduction_two_axes"], "hip reduction only supports one axis")


def test_linear_and_matmul(cases):
    (c,) = _ok(cases["linear_bias"], ["sandy_hip_linear"])
    _dense(c["bias"], 0x3000, [16])
    (c,) = _ok(cases["linear_no_bias"], ["sandy_hip_linear"])
    assert c["bias"] is None
    _err(cases["linear_paged"], "hip linear does not support paged tensor operands")
    (c,) = _ok(cases["matmul"], ["sandy_hip_matmul"])
    assert (c["transpose_lhs"], c["transpose_rhs"]) == (0, 1)
    _dense(c["lhs"], 0x1000, [2, 8], 2)
    _dense(c["rhs"], 0x2000, [16, 8], 2)
    (c,) = _ok(cases["matmul_transpose_lhs"], ["sandy_hip_matmul"])
    assert (c["transpose_lhs"], c["transpose_rhs"]) == (1, 0)
    # CudaMatMulKernels.cu:85-86
    _err(cases["matmul_paged"], "hip matmul does not support paged tensor operands")


def test_gather_softmax_topk(cases):
    (c,) = _ok(cases["gather"], ["sandy_hip_gather"])
    _dense(c["ids"], 0x1000, [5], 4)
    st, c = _ok(cases["gather_paged_table"], ["sandy_hip_paged_stage", "sandy_hip_gather"])
    assert st["slot"] == 1 and st["src"]["grow_dim"] == 0 and st["src"]["page_count"] == 7
    _dense(c["table"], STAGED + 1, [100, 8])
    (c,) = _ok(cases["softmax"], ["sandy_hip_softmax"])
    assert c["axis"] == -1
    st, c = _ok(cases["softmax_paged"], ["sandy_hip_paged_stage", "sandy_hip_softmax"])
    assert st["src"]["dtype"] == 2
    _dense(c["x"], STAGED, [2, 5, 8], 2)
    (c,) = _ok(cases["topk"], ["sandy_hip_topk"])
    assert c["k"] == 8 and c["axis"] == -1
    _dense(c["indices"], 0x3000, [512, 8], 4)
    # CudaTopKKernels.cu:51-52
    _err(cases["topk_paged"], "hip topk does not support paged tensor operands")
    _err(cases["topk_arity"], "hip topk output arity mismatch")


def test_norm_and_rope(cases):
    (c,) = _ok(cases["rms_norm"], ["sandy_hip_norm"])
    assert c["kind"] == 0 and c["bias"] is None and c["epsilon"] == 1e-5
    (c,) = _ok(cases["rms_norm_no_weight"], ["sandy_hip_norm"])
    assert c["weight"] is None and c["bias"] is None and c["epsilon"] == 1e-6
    (c,) = _ok(cases["layer_norm"], ["sandy_hip_norm"])
    assert c["kind"] == 1
    _dense(c["bias"], 0x2800, [768])
    st, c = _ok(cases["rms_norm_paged"], ["sandy_hip_paged_stage", "sandy_hip_norm"])
    assert st["src"]["dims"] == [1, 6, 64] and st["src"]["page_size"] == 4
    _dense(c["x"], STAGED, [1, 6, 64], 2)
    _dense(c["weight"], 0x2000, [64], 2)
    (c,) = _ok(cases["rope"], ["sandy_hip_rope"])
    assert c["position_ids"] is None and c["theta"] == 10000 and c["rotary_dim"] == -1 and c["split_half"] == 1
    (c,) = _ok(cases["rope_ids"], ["sandy_hip_rope"])
    _dense(c["position_ids"], 0x1800, [16], 4)
    assert c["theta"] == 500000 and c["rotary_dim"] == 32 and c["split_half"] == 0
    st, c = _ok(cases["rope_paged"], ["sandy_hip_paged_stage", "sandy_hip_rope"])
    _dense(c["x"], STAGED, [1, 8, 16, 64])
    _dense(c["position_ids"], 0x1800, [16], 4)


def test_attention(cases):
    (c,) = _ok(cases["attention_dense"], ["sandy_hip_attention"])
    assert c["position_offsets"] is None and c["window"] == 0 and c["scale"] == 0.125
    (c,) = _ok(cases["attention_paged_decode"], ["sandy_hip_attention_paged_view"])
    assert c["k"] == {"pages": "2000", "dtype": 2, "dims": [32, 4, 4096, 64], "page_size": 16, "page_count": 8192}
    assert c["v"]["pages"] == "3000" and c["window"] == 128 and c["scale"] == -1
    _dense(c["position_offsets"], 0x5000, [32], 4)
    st, c = _ok(cases["attention_paged_q"], ["sandy_hip_paged_stage", "sandy_hip_attention_paged_view"])
    assert st["slot"] == 0
    _dense(c["q"], STAGED, [2, 8, 1, 64], 2)
    _dense(c["position_offsets"], 0x5000, [2], 3)
    st, c = _ok(cases["attention_paged_other_grow"], ["sandy_hip_paged_stage", "sandy_hip_attention"])
    assert st["slot"] == 1 and st["src"]["grow_dim"] == 1
    _dense(c["k"], STAGED + 1, [2, 4, 64, 64])
    _dense(c["v"], 0x3000, [2, 4, 64, 64])
    _err(cases["attention_arity"], "hip attention input arity mismatch")


def test_moe(cases):
    (c,) = _ok(cases["moe_gather"], ["sandy_hip_moe_gather"])
    assert c["num_experts"] == 128 and c["top_k"] == 8
    _dense(c["expert_offsets"], 0x7000, [129], 4)
    # CudaGatherKernels.cu:127-132
    _err(cases["moe_gather_paged_ids"], "hip moe_gather topk_ids cannot be paged")
    (c,) = _ok(cases["moe_matmul"], ["sandy_hip_moe_matmul"])
    assert c["transpose_rhs"] == 1
    _dense(c["weight"], 0x3000, [128, 704, 2816], 2)
    # CudaMatMulKernels.cu:311-312
    _err(cases["moe_matmul_paged"], "hip moe_matmul does not support paged tensor operands")
    (c,) = _ok(cases["moe_scatter_sum"], ["sandy_hip_moe_scatter_sum"])
    _dense(c["out"], 0x4000, [512, 2816], 2)
    # CudaMoeScatterSumKernels.cu:26-31
    _err(cases["moe_scatter_sum_paged_tokens"], "hip moe_scatter_sum token_ids cannot be paged")


def test_dispatch_calls_only_declared_entry_points():
    declared = set(re.findall(r"\b(sandy_hip_\w+)\s*\(", open(os.path.join(ROOT, "include", "sandyrt_hip.h")).read()))
    used = set(re.findall(r"\b(sandy_hip_\w+)\s*\(", open(SRC).read()))
    assert used and used <= declared, used - declared
