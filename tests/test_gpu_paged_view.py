"""AttentionKernelOp over the reference's own paged K/V layout through the C
ABI (sandy_hip_attention_paged_view): a paged tensor [B, Hkv, T, D] whose
pages [B * Hkv, page_size, D] are separate allocations named by a device
page table (CudaPagedTensor.cpp:187-226, addressing CudaKernelUtils.cuh:
82-108), one page list for the whole batch, padded T and position_offsets
-- the batched decode the reference runs as rank-4 attention
(TensorCalc.cpp:1167-1314).  The oracle sees the dense tensors the pages
hold, as the reference CPU device materialises them (CpuDevice.cpp:611-676)."""
import numpy as np
import pytest
import torch

from tests.helpers import assert_close, from_f32, normal, rng, to_oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from sandyrt_amd import ops
    return ops


def make_view(ops, r, lead, T, D, P, dtype, spare=0):
    """Pages of [prod(lead), P, D], each its own allocation, in a page table;
    `spare` extra pages past the logical length.  Returns the view, the dense
    logical tensor (oracle encoding) and the page tensors (kept alive)."""
    rows = int(np.prod(lead))
    n = (T + P - 1) // P + spare
    pages = [from_f32(normal(r, (rows, P, D)), dtype) for _ in range(n)]
    table = torch.tensor([p.data_ptr() for p in pages], dtype=torch.int64, device="cuda")
    dense = torch.cat(pages, dim=1)[:, :T].reshape(*lead, T, D)
    return ops.PagedView(table, list(lead) + [T, D], P, dtype), to_oracle(dense), pages


def run(ops, oracle, seed, B, hq, hkv, D, P, T, tq, dtype, window=0, scale=-1.0, rank=4, spare=0):
    r = rng(seed)
    lead = [B, hkv] if rank == 4 else [hkv]
    kv, kd, keep_k = make_view(ops, r, lead, T, D, P, dtype, spare)
    vv, vd, keep_v = make_view(ops, r, lead, T, D, P, dtype, spare)
    qshape = [B, hq, tq, D] if rank == 4 else [hq, tq, D]
    q = from_f32(normal(r, qshape), dtype)
    nb = B if rank == 4 else 1
    pos = r.integers(0, T - tq + 1, nb).astype(np.int64)
    pos[0] = T - tq  # the longest query sees every key
    out = ops.attention_paged_view(q, kv, vv, torch.from_numpy(pos).cuda(), window=window, scale=scale)
    ops.check_device_errors()
    want = oracle.attention(to_oracle(q), kd, vd, pos, window, scale)
    assert_close(out, want, dtype, f"paged view attention B{B} hq{hq} hkv{hkv} D{D} T{T} tq{tq}")
    return out


def test_batched_decode_tinyllama_geometry(ops, oracle):
    """Config-3 heads over one shared page list, padded T (MFMA decode kernel)."""
    run(ops, oracle, 1, 8, 32, 4, 64, 16, 1000, 1, torch.bfloat16, scale=0.125)


def test_batched_decode_gemma_geometry_multi_split(ops, oracle):
    run(ops, oracle, 2, 4, 8, 2, 256, 16, 3000, 1, torch.bfloat16, scale=1.0, spare=3)


def test_unbatched_rank3_decode(ops, oracle):
    run(ops, oracle, 3, 1, 16, 2, 128, 32, 777, 1, torch.bfloat16, rank=3)


def test_decode_sliding_window(ops, oracle):
    run(ops, oracle, 4, 5, 8, 4, 64, 16, 900, 1, torch.bfloat16, window=100)


def test_f32_decode_general_kernel(ops, oracle):
    run(ops, oracle, 5, 3, 4, 2, 64, 8, 300, 1, torch.float32)


def test_prefill_over_pages_general_kernel(ops, oracle):
    run(ops, oracle, 6, 2, 8, 2, 64, 16, 200, 5, torch.bfloat16)


def test_paged_view_errors(ops):
    from sandyrt_amd._lib import SandyError
    r = rng(7)
    kv, _, keep = make_view(ops, r, [2, 2], 40, 64, 16, torch.bfloat16)
    short = ops.PagedView(kv.pages[:2], [2, 2, 40, 64], 16, torch.bfloat16)  # 40 rows need 3 pages
    q = torch.zeros(2, 4, 1, 64, dtype=torch.bfloat16, device="cuda")
    pos = torch.zeros(2, dtype=torch.int64, device="cuda")
    with pytest.raises(SandyError, match="page count does not cover"):
        ops.attention_paged_view(q, short, short, pos)
    with pytest.raises(SandyError, match="position_offsets length must match batch"):
        ops.attention_paged_view(q, kv, kv, torch.zeros(3, dtype=torch.int64, device="cuda"))
    odd = ops.PagedView(kv.pages, [2, 2, 40, 64], 12, torch.bfloat16)
    with pytest.raises(SandyError, match="power of two"):
        ops.attention_paged_view(q, odd, odd, pos)


@pytest.mark.parametrize("dtype,tq,D,unstaged", [(torch.float32, 1, 64, False), (torch.bfloat16, 5, 64, False),
                                                 (torch.bfloat16, 1, 64, False), (torch.bfloat16, 1, 96, False),
                                                 (torch.float32, 1, 64, True), (torch.bfloat16, 5, 64, True)])
def test_null_page_is_a_device_error(ops, monkeypatch, dtype, tq, D, unstaged):
    """A page-table entry of 0 inside the attended range is reported as a
    device error by every kernel that reads the view (f32 decode and prefill
    through the general kernels, bf16 decode through the MFMA kernel, a head
    dim the MFMA kernel does not take), and nothing is read from address 0."""
    from sandyrt_amd._lib import SandyError
    r = rng(11)
    kv, _, keep_k = make_view(ops, r, [2, 2], 40, D, 16, dtype)
    vv, _, keep_v = make_view(ops, r, [2, 2], 40, D, 16, dtype)
    holed = kv.pages.clone()
    holed[1] = 0  # keys 16..31 have no page
    kz = ops.PagedView(holed, [2, 2, 40, D], 16, dtype)
    vz = ops.PagedView(holed.clone(), [2, 2, 40, D], 16, dtype)
    q = from_f32(normal(r, (2, 4, tq, D)), dtype)
    pos = torch.tensor([39 - (tq - 1), 39 - (tq - 1)], dtype=torch.int64, device="cuda")
    for k_view, v_view in ((kz, vv), (kv, vz)):
        ops.attention_paged_view(q, k_view, v_view, pos)
        with pytest.raises(SandyError, match="block id outside the pool"):
            ops.check_device_errors()
    torch.cuda.synchronize()
