"""Paged inputs of the non-attention families through the C ABI: the
reference's element-wise, norm, RoPE, softmax, reduction and gather kernels
read a paged input in place (load_float / load_int over paged_storage_index,
src/device/cuda/CudaKernelUtils.cuh:82-157; tests
test/engine/CudaDeviceTest.cpp:685-855).  Here the input is gathered by
sandy_hip_paged_to_dense (or sandy_hip_paged_stage) and the dense kernel
runs.  The pages are separate allocations in a device page table in random
order; the oracle sees the dense tensor the pages hold, as the reference CPU
device materialises it (oracle paged_to_dense, CpuDevice.cpp:611-676), and
runs the op on it.  Results are compared bit for bit with the dense op on
the oracle's dense tensor, and to the north star's tolerance against the
oracle op."""
import ctypes as C

import numpy as np
import pytest
import torch

from tests.helpers import assert_close, assert_equal, from_f32, normal, rng, to_oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from sandyrt_amd import ops
    return ops


def make_paged(ops, oracle, r, dims, grow, P, dtype, values=None, shuffle=True, misalign=False, pages_short=0):
    """A paged tensor of logical shape dims growing along `grow` in pages of
    P rows: each page its own allocation of [prefix, P, inner] in a random
    allocation order.  Returns (PagedTensor, dense logical tensor in the
    oracle's encoding, keep-alive list).  misalign: page addresses 2 bytes
    past a 16-byte boundary.  pages_short: that many trailing pages left out
    of the table (their rows read as zero)."""
    prefix = int(np.prod(dims[:grow])) if grow else 1
    G = dims[grow]
    inner = int(np.prod(dims[grow + 1:])) if grow + 1 < len(dims) else 1
    n = (G + P - 1) // P
    if values is None:
        values = normal(r, (n, prefix, P, inner))
    pages = [from_f32(values[i], dtype) for i in range(n)]
    keep = list(pages)
    order = r.permutation(n) if shuffle else np.arange(n)
    addrs = []
    for i in range(n):
        p = pages[order[i]]
        if misalign:
            buf = torch.empty(p.numel() * p.element_size() + 64, dtype=torch.uint8, device="cuda")
            base = (buf.data_ptr() + 15) // 16 * 16 + 2
            off = base - buf.data_ptr()
            buf[off:off + p.numel() * p.element_size()].copy_(p.contiguous().view(torch.uint8).flatten())
            keep.append(buf)
            addrs.append(base)
        else:
            addrs.append(p.data_ptr())
    # logical page j is the j-th of `order`
    table_addrs = [0] * n
    for i in range(n):
        table_addrs[order[i]] = addrs[i]
    table = torch.tensor(table_addrs[:n - pages_short], dtype=torch.int64, device="cuda")
    pool = np.stack([to_oracle(p) for p in pages])  # [n, prefix, P, inner], logical order
    ids = np.arange(n, dtype=np.int32)
    dense = oracle.paged_to_dense(pool, ids, prefix, G, P, inner).reshape(dims)
    if pages_short:
        flat = dense.reshape(prefix, G, inner)
        flat[:, (n - pages_short) * P:, :] = 0
    keep.append(table)
    return ops.PagedTensor(table, dims, grow, P, dtype), dense, keep


def test_elementwise_reads_paged_tensor_known_answer(ops, oracle):
    """RunElementwiseReadsPagedTensorF32 (CudaDeviceTest.cpp:685-760): a
    [2, 3, 4] f32 tensor growing along dim 1 in pages of 2 rows holding 0..23
    row-major; x + 1 gives 1..24."""
    vals = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    pages = np.zeros((2, 2, 2, 4), np.float32)  # [page, prefix, P, inner]
    for g in range(3):
        pages[g // 2, :, g % 2] = vals[:, g]
    pt, dense, keep = make_paged(ops, oracle, rng(0), [2, 3, 4], 1, 2, torch.float32, values=pages)
    np.testing.assert_array_equal(dense, vals)
    nodes = [ops.ScalarNode(0, ops.LOAD, input_index=0), ops.ScalarNode(1, ops.CONST, constant=1.0),
             ops.ScalarNode(2, ops.ADD, operands=(0, 1))]
    out = ops.elementwise(nodes, 2, [pt])
    np.testing.assert_array_equal(to_oracle(out), vals + 1)


def test_elementwise_refreshed_meta_known_answer(ops, oracle):
    """RunElementwiseRefreshesPagedTensorMetaAtLaunch (CudaDeviceTest.cpp:
    762-855): appends of [2, 1, 4] (0..7) then [2, 2, 4] (8..23) to a [2, T,
    4] tensor in pages of 2 rows; a Load reads the expected interleaving."""
    first = np.arange(8, dtype=np.float32).reshape(2, 1, 4)
    second = np.arange(8, 24, dtype=np.float32).reshape(2, 2, 4)
    logical = np.concatenate([first, second], axis=1)  # the appended rows in grow order
    pages = np.zeros((2, 2, 2, 4), np.float32)
    for g in range(3):
        pages[g // 2, :, g % 2] = logical[:, g]
    pt, _, keep = make_paged(ops, oracle, rng(1), [2, 3, 4], 1, 2, torch.float32, values=pages)
    out = ops.elementwise([ops.ScalarNode(0, ops.LOAD, input_index=0)], 0, [pt])
    want = np.array([0, 1, 2, 3, 8, 9, 10, 11, 12, 13, 14, 15,
                     4, 5, 6, 7, 16, 17, 18, 19, 20, 21, 22, 23], np.float32).reshape(2, 3, 4)
    np.testing.assert_array_equal(to_oracle(out), want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_paged_silu_gate(ops, oracle, dtype):
    """A SiLU-gated element-wise group with one paged input ([1, 77, 512]
    growing along dim 1, pages of 16) and one dense input."""
    r = rng(2)
    g, gd, keep = make_paged(ops, oracle, r, [1, 77, 512], 1, 16, dtype)
    u = from_f32(normal(r, (1, 77, 512)), dtype)
    nodes, res = ops.silu_mul_nodes()
    out = ops.elementwise(nodes, res, [g, u])
    dense_out = ops.elementwise(nodes, res, [ops.paged_to_dense(g), u])
    assert_equal(out, to_oracle(dense_out), "paged vs dense element-wise")
    from oracle import oracle as O
    onodes = O.make_nodes([(a.id, a.op, a.input_index, a.constant, list(a.operands)) for a in nodes])
    want = oracle.elementwise_dag(onodes, res, [gd, to_oracle(u)], [0, 0], (1, 77, 512),
                                  np.uint16 if dtype == torch.bfloat16 else np.float32)
    assert_close(out, want, dtype, "paged silu gate")


@pytest.mark.parametrize("misalign", [False, True])
def test_paged_rms_norm(ops, oracle, misalign):
    """RMSNorm of a paged bf16 [2, 37, 2048] (grow dim 1, pages of 16, the
    last page partly used); misaligned page addresses take the bytewise read."""
    r = rng(3)
    x, xd, keep = make_paged(ops, oracle, r, [2, 37, 2048], 1, 16, torch.bfloat16, misalign=misalign)
    w = from_f32(normal(r, (2048,)), torch.bfloat16)
    out = ops.rms_norm(x, w, 1e-5)
    assert_equal(out, to_oracle(ops.rms_norm(ops.paged_to_dense(x), w, 1e-5)), "paged vs dense rms_norm")
    assert_close(out, oracle.rms_norm(xd, to_oracle(w), 1e-5), torch.bfloat16, "paged rms_norm")


def test_paged_layer_norm_softmax_sum(ops, oracle):
    r = rng(4)
    x, xd, keep = make_paged(ops, oracle, r, [3, 20, 768], 1, 8, torch.float32)
    w, b = from_f32(normal(r, (768,)), torch.float32), from_f32(normal(r, (768,)), torch.float32)
    assert_close(ops.layer_norm(x, w, b, 1e-5), oracle.layer_norm(xd, to_oracle(w), to_oracle(b), 1e-5),
                 torch.float32, "paged layer_norm")
    assert_close(ops.softmax(x, -1), oracle.softmax(xd, -1), torch.float32, "paged softmax")
    assert_close(ops.sum(x, -1, True), oracle.sum(xd, -1, True), torch.float32, "paged sum")


def test_paged_rope_and_position_ids(ops, oracle):
    """RoPE of a paged [1, 8, 40, 64] f32 q (grow dim 2, pages of 16) with
    paged int64 position ids ([40], grow dim 0, pages of 8)."""
    r = rng(5)
    q, qd, keep = make_paged(ops, oracle, r, [1, 8, 40, 64], 2, 16, torch.float32)
    pos_vals = r.integers(0, 4096, 40).astype(np.int64)
    pt = np.zeros((5, 1, 8, 1), np.int64)
    for g in range(40):
        pt[g // 8, 0, g % 8, 0] = pos_vals[g]
    pages = [torch.from_numpy(pt[i].copy()).cuda() for i in range(5)]
    table = torch.tensor([p.data_ptr() for p in pages], dtype=torch.int64, device="cuda")
    ids = ops.PagedTensor(table, [40], 0, 8, torch.int64)
    out = ops.rope(q, 1e4, split_half=True, position_ids=ids)
    want = oracle.rope(qd, 1e4, split_half=True, position_ids=pos_vals)
    assert_close(out, want, torch.float32, "paged rope")


def test_paged_embedding_table(ops, oracle):
    r = rng(6)
    table, td, keep = make_paged(ops, oracle, r, [100, 64], 0, 16, torch.bfloat16)
    ids = torch.from_numpy(r.integers(0, 100, 37).astype(np.int64)).cuda()
    out = ops.embedding(ids, table)
    assert_equal(out, td[ids.cpu().numpy()], "paged embedding table")


def test_missing_and_null_pages_read_zero(ops, oracle):
    """Rows on pages past the table's page count read as zero
    (load_float_at_storage returns 0 without a page)."""
    r = rng(7)
    x, xd, keep = make_paged(ops, oracle, r, [2, 40, 64], 1, 16, torch.float32, pages_short=1)
    out = ops.paged_to_dense(x)
    assert_equal(out, xd, "short page table")
    assert not xd[:, 32:].any() and xd[:, :32].any()
    x.pages[1] = 0  # a null page
    out = ops.paged_to_dense(x)
    want = xd.copy()
    want[:, 16:32] = 0
    assert_equal(out, want, "null page")


def test_paged_stage_slots(ops, oracle):
    """sandy_hip_paged_stage: the library's staging slot holds the dense copy."""
    from sandyrt_amd import _lib
    r = rng(8)
    x, xd, keep = make_paged(ops, oracle, r, [4, 33, 96], 1, 4, torch.bfloat16)
    dense = _lib.SandyTensor()
    _lib.call("sandy_hip_paged_stage", x.struct(), C.c_int32(3), C.byref(dense))
    assert dense.rank == 3 and list(dense.dims)[:3] == [4, 33, 96] and dense.strides[0] == 33 * 96
    out = torch.empty(4, 33, 96, dtype=torch.bfloat16, device="cuda")
    # read the staged copy back through a dense element-wise Load into `out`
    nodes = (_lib.SandyScalarNode * 1)()
    nodes[0].id, nodes[0].op, nodes[0].operand_count = 0, 0, 0
    bc = (C.c_int32 * 1)(0)
    _lib.call("sandy_hip_elementwise", nodes, C.c_int32(1), C.c_uint32(0), C.byref(dense), bc, C.c_int32(1),
              _lib.desc(out))
    assert_equal(out, xd, "staged slot")
    with pytest.raises(_lib.SandyError, match="slot out of range"):
        _lib.call("sandy_hip_paged_stage", x.struct(), C.c_int32(8), C.byref(dense))
