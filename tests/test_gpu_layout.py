"""LayoutTransformKernelOp through the C ABI (sandy_hip_layout_transform):
the logical elements of a strided view, in row-major order, into the output
-- the reference's copy (src/device/cuda/CudaLayoutTransformKernels.cu:25-78)
for the views the engine cannot alias (src/engine/Engine.cpp:606-754).  A
layout transform is a permutation of elements, so the expected output is the
view's elements read in row-major order (torch's .contiguous() of the same
view), bit for bit, for every dtype."""
import pytest
import torch

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float32, torch.uint8, torch.int64, torch.int32]


@pytest.fixture(scope="module")
def ops():
    from sandyrt_amd import ops
    return ops


def rand(shape, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    if dtype.is_floating_point:
        return torch.randn(shape, generator=g, device="cuda").to(dtype)
    return torch.randint(0, 250, shape, generator=g, device="cuda").to(dtype)


def same_bits(a, b):
    assert a.shape == b.shape and a.dtype == b.dtype
    assert torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(4096, 2048), (100, 70), (64, 64), (3, 1000)])
def test_transposed_view_to_contiguous(ops, dtype, shape):
    x = rand(shape, dtype, 1).t()  # the inner pair transposed: tile path (or per element when small)
    same_bits(ops.layout_transform(x), x.contiguous())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_head_permute_rows(ops, dtype):
    x = rand((2, 8, 96, 64), dtype, 2).permute(0, 2, 1, 3)  # [B, S, H, D] view of [B, H, S, D]: row copies
    same_bits(ops.layout_transform(x), x.contiguous())


@pytest.mark.parametrize("dtype", DTYPES)
def test_general_permutes(ops, dtype):
    x = rand((3, 4, 5, 6), dtype, 3)
    for perm in [(3, 1, 0, 2), (2, 0, 1, 3), (1, 0, 3, 2), (0, 3, 2, 1)]:
        v = x.permute(perm)
        same_bits(ops.layout_transform(v), v.contiguous())
    v = x[:, ::2, 1:, ::3]  # strided slices of every dim
    same_bits(ops.layout_transform(v), v.contiguous())


def test_contiguous_reshape_and_batched_transpose(ops):
    x = rand((8, 300, 70), torch.bfloat16, 4)
    same_bits(ops.layout_transform(x, torch.empty(8 * 300 * 70, dtype=torch.bfloat16, device="cuda"),
                                   kind=ops.RESHAPE), x.reshape(-1))
    v = x.transpose(1, 2)  # [8, 70, 300] view, batched inner transpose
    same_bits(ops.layout_transform(v), v.contiguous())
    # a reshape of a transposed view into another shape: linear order of the view
    out = torch.empty(70, 8, 300, dtype=torch.bfloat16, device="cuda")
    same_bits(ops.layout_transform(v, out, kind=ops.RESHAPE), v.contiguous().reshape(70, 8, 300))


def test_unaligned_and_strided_output(ops):
    base = rand((1 + 64 * 33,), torch.bfloat16, 5)
    x = base[1:].view(64, 33)  # 2 bytes off alignment, odd row length
    same_bits(ops.layout_transform(x), x.contiguous())
    y = rand((40, 24), torch.float32, 6)
    out_store = torch.zeros(24, 40, device="cuda")
    out = out_store.t()  # a strided output of y's shape
    ops.layout_transform(y, out, kind=ops.TRANSPOSE)
    same_bits(out, y)


def test_layout_errors(ops):
    from sandyrt_amd._lib import SandyError
    x = rand((4, 6), torch.float32, 7)
    with pytest.raises(SandyError, match="slice layout aliases must not launch"):
        ops.layout_transform(x, kind=ops.SLICE)
    with pytest.raises(SandyError, match="dtype mismatch"):
        ops.layout_transform(x, torch.empty(4, 6, dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(SandyError, match="element count mismatch"):
        ops.layout_transform(x, torch.empty(25, device="cuda"))
