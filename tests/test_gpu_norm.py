"""GPU parity: RMSNorm, LayerNorm and residual-add + RMSNorm against the
oracle (restated src/core/TensorCalc.cpp:1953-2077), through the C ABI."""
import numpy as np
import pytest
import torch

from tests.helpers import assert_close, assert_equal, from_f32, normal, rng, to_oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from sandyrt_amd import ops
    return ops


SHAPES = [(4, 64), (37, 2048), (3, 5, 256), (8, 2560), (2, 4096), (5, 768), (3, 100), (2, 6000), (1, 8)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("with_weight", [True, False])
def test_rms_norm(ops, oracle, dtype, shape, with_weight):
    r = rng(hash((shape, with_weight)) % 2**32)
    x = from_f32(normal(r, shape), dtype)
    w = from_f32(normal(r, shape[-1:]), dtype) if with_weight else None
    got = ops.rms_norm(x, w, 1e-5)
    want = oracle.rms_norm(to_oracle(x), to_oracle(w) if w is not None else None, 1e-5)
    assert_close(got, want, dtype, f"rms_norm {shape}")


def test_rms_norm_bf16_bit_exact_tinyllama_rows(ops, oracle):
    """bf16 squares are exact in double, so the device row sum equals the CPU's
    sequential double sum and the output matches bit for bit."""
    r = rng(11)
    x = from_f32(normal(r, (64, 2048)), torch.bfloat16)
    w = from_f32(normal(r, (2048,)), torch.bfloat16)
    got = ops.rms_norm(x, w, 1e-5)
    assert_equal(got, oracle.rms_norm(to_oracle(x), to_oracle(w), 1e-5), "rms_norm bf16")


def test_rms_norm_known_answer(ops):
    # test/engine/CudaDeviceTest.cpp:3573-3643
    x = torch.tensor([[1, 2, 3, 4], [2, 0, -2, 4]], dtype=torch.float32, device="cuda")
    w = torch.tensor([1, 0.5, 2, -1], dtype=torch.float32, device="cuda")
    y = ops.rms_norm(x, w, 1e-6).cpu().numpy()
    i0 = 1 / np.sqrt(30 / 4 + 1e-6)
    i1 = 1 / np.sqrt(24 / 4 + 1e-6)
    np.testing.assert_allclose(y, [[i0, i0, 6 * i0, -4 * i0], [2 * i1, 0, -4 * i1, -4 * i1]], atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(4, 768), (7, 64), (3, 1000), (2, 8192)])
def test_layer_norm(ops, oracle, dtype, shape):
    r = rng(sum(shape))
    x = from_f32(normal(r, shape) + 1.5, dtype)
    w = from_f32(normal(r, shape[-1:]), dtype)
    b = from_f32(normal(r, shape[-1:]), dtype)
    got = ops.layer_norm(x, w, b, 1e-5)
    want = oracle.layer_norm(to_oracle(x), to_oracle(w), to_oracle(b), 1e-5)
    assert_close(got, want, dtype, f"layer_norm {shape}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(64, 2048), (5, 2560), (3, 300)])
def test_add_rms_norm_matches_unfused_chain(ops, oracle, dtype, shape):
    """The fused pair equals the reference's separate add then rms_norm; the
    sum output is bit-exact (one float add, one rounding)."""
    r = rng(7 + shape[0])
    x = from_f32(normal(r, shape), dtype)
    h = from_f32(normal(r, shape), dtype)
    w = from_f32(normal(r, shape[-1:]), dtype)
    s, y = ops.add_rms_norm(x, h, w, 1e-5)
    want_s = oracle.binary("add", to_oracle(x), to_oracle(h))
    want_y = oracle.rms_norm(want_s, to_oracle(w), 1e-5)
    assert_equal(s, want_s, "residual sum")
    assert_close(y, want_y, dtype, "rms_norm(sum)")


def test_add_rms_norm_in_place(ops, oracle):
    r = rng(3)
    x = from_f32(normal(r, (16, 2048)), torch.bfloat16)
    h = from_f32(normal(r, (16, 2048)), torch.bfloat16)
    w = from_f32(normal(r, (2048,)), torch.bfloat16)
    want_s = oracle.binary("add", to_oracle(x), to_oracle(h))
    ops.add_rms_norm(x, h, w, 1e-5, sum_out=x)
    assert_equal(x, want_s, "in-place residual sum")


def test_norm_rejects_bad_shapes(ops):
    from sandyrt_amd._lib import SandyError
    x = torch.zeros(4, 8, device="cuda")
    with pytest.raises(SandyError, match="rms_norm weight dimension mismatch"):
        ops.rms_norm(x, torch.zeros(7, device="cuda"), 1e-5)
    with pytest.raises(SandyError, match="operands must have same dtype"):
        ops.rms_norm(x, torch.zeros(8, device="cuda", dtype=torch.bfloat16), 1e-5)


# Launches of more than 1024 rows take the four-rows-per-workgroup form (the
# weights read after the reduction); 1024 and 1025 rows pin the switch.
LARGE = [(4096, 2048), (1500, 2560), (1030, 300), (1024, 512), (1025, 512)]


@pytest.mark.parametrize("shape", LARGE)
@pytest.mark.parametrize("with_weight", [True, False])
def test_rms_norm_many_rows(ops, oracle, shape, with_weight):
    r = rng(hash(("many", shape, with_weight)) % 2**32)
    x = from_f32(normal(r, shape), torch.bfloat16)
    w = from_f32(normal(r, shape[-1:]), torch.bfloat16) if with_weight else None
    got = ops.rms_norm(x, w, 1e-5)
    want = oracle.rms_norm(to_oracle(x), to_oracle(w) if w is not None else None, 1e-5)
    # bf16 squares are exact in double: the row sums, and so the outputs, are the CPU's bit for bit
    assert_equal(got, want, f"rms_norm {shape}")


@pytest.mark.parametrize("shape", LARGE)
def test_add_rms_norm_many_rows(ops, oracle, shape):
    r = rng(hash(("add", shape)) % 2**32)
    x = from_f32(normal(r, shape), torch.bfloat16)
    h = from_f32(normal(r, shape), torch.bfloat16)
    w = from_f32(normal(r, shape[-1:]), torch.bfloat16)
    s, y = ops.add_rms_norm(x, h, w, 1e-5)
    want_s = oracle.binary("add", to_oracle(x), to_oracle(h))
    assert_equal(s, want_s, f"residual sum {shape}")
    assert_close(y, oracle.rms_norm(want_s, to_oracle(w), 1e-5), torch.bfloat16, f"rms_norm(sum) {shape}")


def test_add_rms_norm_many_rows_f32(ops, oracle):
    r = rng(99)
    x = from_f32(normal(r, (2048, 1000)), torch.float32)
    h = from_f32(normal(r, (2048, 1000)), torch.float32)
    w = from_f32(normal(r, (1000,)), torch.float32)
    s, y = ops.add_rms_norm(x, h, w, 1e-5)
    want_s = oracle.binary("add", to_oracle(x), to_oracle(h))
    assert_equal(s, want_s, "residual sum f32")
    assert_close(y, oracle.rms_norm(want_s, to_oracle(w), 1e-5), torch.float32, "rms_norm(sum) f32")
