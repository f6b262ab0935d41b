"""The reference-side binding executed on the GPU: the reference's own
KernelIR op classes (src/ir/KernelIR.h) run through
sandyrt_amd/reference_binding/HipKernelDispatch.cpp -- the call
CudaDevice::run makes into launch_cuda_* (src/device/cuda/CudaDevice.cpp:
455-578) -- on the built library, with paged operands in the reference's
page-address layout (CudaPagedTensor.cpp:187-226).  tests/binding/
gpu_driver.cpp (built by `make -C oracle binding` where the reference tree
exists; the binary travels with the tree) prints every case's inputs and
outputs, and each output is checked against the CPU oracle on the same
inputs: floating point within the tolerance rule of tests/helpers.py,
indices exactly."""
import json
import os
import subprocess

import numpy as np
import pytest
import torch

from oracle import oracle as O
from sandyrt_amd import ops
from tests.helpers import assert_close, assert_equal

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER = os.path.join(ROOT, "oracle", "_ref", "binding_gpu_driver")
NP = {"bf16": np.uint16, "f32": np.float32, "i32": np.int32, "i64": np.int64}
TORCH = {"bf16": torch.bfloat16, "f32": torch.float32}


@pytest.fixture(scope="module")
def cases():
    if not os.path.exists(DRIVER):
        pytest.skip("binding driver not built (needs the reference tree at build time)")
    r = subprocess.run([DRIVER], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    out = {}
    for line in r.stdout.splitlines():
        c = json.loads(line)
        c["t"] = {k: np.array(v["data"], dtype=NP[v["dtype"]]).reshape(v["shape"]) for k, v in c["tensors"].items()}
        c["dt"] = {k: v["dtype"] for k, v in c["tensors"].items()}
        out[c["case"]] = c
    return out


def _case(cases, name):
    c = cases[name]
    assert c["ok"], c["error"]
    return c["t"], c["dt"]


def _half_x_plus_y(oracle, x, y):
    nodes = O.make_nodes([(0, ops.LOAD, 0, 0.0, []), (1, ops.LOAD, 1, 0.0, []), (2, ops.CONST, 0, 0.5, []),
                          (3, ops.MUL, 0, 0.0, [0, 2]), (4, ops.ADD, 0, 0.0, [3, 1])])
    return oracle.elementwise_dag(nodes, 4, [x, y], [0, 1], x.shape, x.dtype)


@pytest.mark.parametrize("name", ["elementwise_bf16", "elementwise_paged_f32"])
def test_elementwise(cases, oracle, name):
    t, dt = _case(cases, name)
    assert_close(t["out"], _half_x_plus_y(oracle, t["x"], t["y"]), TORCH[dt["out"]], name)


def test_rms_norm(cases, oracle):
    t, _ = _case(cases, "rms_norm_bf16")
    assert_close(t["out"], oracle.rms_norm(t["x"], t["w"], 1e-5), torch.bfloat16, "rms_norm")


def test_rope(cases, oracle):
    t, _ = _case(cases, "rope_bf16")
    assert_close(t["out"], oracle.rope(t["x"], 10000.0, split_half=True), torch.bfloat16, "rope")


def test_softmax(cases, oracle):
    t, _ = _case(cases, "softmax_f32")
    assert_close(t["out"], oracle.softmax(t["x"]), torch.float32, "softmax")


def test_topk(cases, oracle):
    t, _ = _case(cases, "topk_f32")
    values, indices = oracle.topk(t["x"], 8)
    assert_equal(t["values"], values, "topk values")
    assert_equal(t["indices"], indices, "topk indices")


def test_paged_decode_attention(cases, oracle):
    t, _ = _case(cases, "attention_paged_decode_bf16")
    want = oracle.attention(t["q"], t["k"], t["v"], position_offsets=t["pos"])
    assert_close(t["out"], want, torch.bfloat16, "paged decode attention")


def test_moe_chain(cases, oracle):
    g, _ = _case(cases, "moe_gather_bf16")
    px, pw, tok, off = oracle.moe_gather(g["x"], g["topk_ids"], g["topk_weights"], 4)
    for k, want in (("packed_x", px), ("packed_w", pw), ("token_ids", tok), ("offsets", off)):
        assert_equal(g[k], want, f"moe_gather {k}")
    m, _ = _case(cases, "moe_matmul_bf16")
    want = oracle.moe_matmul(m["packed_x"], m["offsets"], m["weight"])
    assert_close(m["packed_out"], want, torch.bfloat16, "moe_matmul")
    s, _ = _case(cases, "moe_scatter_sum_bf16")
    want = oracle.moe_scatter_sum(s["packed_out"], s["packed_w"], s["token_ids"], 8)
    assert_close(s["out"], want, torch.bfloat16, "moe_scatter_sum")


def test_reduce_sum(cases, oracle):
    t, _ = _case(cases, "reduce_sum_f32")
    assert_close(t["out"], oracle.sum(t["x"]), torch.float32, "reduce sum")


def test_linear(cases, oracle):
    t, _ = _case(cases, "linear_f32")
    assert_close(t["out"], oracle.linear(t["x"], t["w"], t["b"]), torch.float32, "linear")


def test_matmul(cases, oracle):
    t, _ = _case(cases, "matmul_bf16")
    assert_close(t["out"], oracle.matmul(t["lhs"], t["rhs"], transpose_rhs=True), torch.bfloat16, "matmul")


def test_gather(cases, oracle):
    t, _ = _case(cases, "gather_bf16")
    assert_equal(t["out"], oracle.embedding(t["ids"], t["table"]), "gather")


def test_layer_norm(cases, oracle):
    t, _ = _case(cases, "layer_norm_f32")
    assert_close(t["out"], oracle.layer_norm(t["x"], t["w"], t["b"], 1e-5), torch.float32, "layer_norm")


def test_rope_position_ids(cases, oracle):
    t, _ = _case(cases, "rope_ids_f32")
    want = oracle.rope(t["x"], 500000.0, rotary_dim=32, split_half=False, position_ids=t["ids"])
    assert_close(t["out"], want, torch.float32, "rope with ids")


def test_layout_transpose(cases):
    t, _ = _case(cases, "layout_transpose_f32")
    assert_equal(t["out"], np.ascontiguousarray(t["x"].T), "transpose")


def test_softmax_paged(cases, oracle):
    t, _ = _case(cases, "softmax_paged_bf16")
    assert_close(t["out"], oracle.softmax(t["x"]), torch.bfloat16, "paged softmax")


def test_dense_attention(cases, oracle):
    t, _ = _case(cases, "attention_dense_bf16")
    want = oracle.attention(t["q"], t["k"], t["v"], position_offsets=t["pos"])
    assert_close(t["out"], want, torch.bfloat16, "dense attention")
