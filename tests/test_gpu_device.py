"""GPU tests of the device runtime (buffers, paged pools with device-side
append, graph capture of a decode step) against the reference's CPU device
semantics: CpuDevice::appendPaged / read(DevicePagedTensorView)
(src/device/cpu/CpuDevice.cpp:465-676) and its validation errors."""
import ctypes as C

import numpy as np
import pytest
import torch

from tests.helpers import assert_close, from_f32, normal, rng, to_oracle

pytestmark = pytest.mark.gpu


@pytest.fixture()
def dev():
    from sandyrt_amd.device import HipDevice
    d = HipDevice(0)
    yield d
    d.close()


def bf16_np(t):
    return to_oracle(t)


def test_buffers_roundtrip(dev):
    from sandyrt_amd._lib import SandyError
    a = np.arange(1000, dtype=np.float32)
    b = dev.load(a)
    assert np.frombuffer(dev.read(b, a.nbytes), np.float32).tolist() == a.tolist()
    assert np.frombuffer(dev.read(b, 40, offset=400), np.float32).tolist() == a[100:110].tolist()
    dev.dealloc(b)
    with pytest.raises(SandyError, match="hip device buffer not found"):
        dev.dealloc(b)


def test_paged_pool_validation(dev):
    from sandyrt_amd._lib import BF16, SandyError
    with pytest.raises(SandyError, match="page_size must be a power of two"):
        dev.create_paged_pool([1, 4, -1, 64], BF16, 2, 12)
    with pytest.raises(SandyError, match="grow_dim out of range"):
        dev.create_paged_pool([1, 4, -1, 64], BF16, 4, 16)
    with pytest.raises(SandyError, match="non-grow dimensions must be static and positive"):
        dev.create_paged_pool([1, 0, -1, 64], BF16, 2, 16)
    pool = dev.create_paged_pool([1, 2, -1, 8], BF16, 2, 16, max_pages=2, max_tensors=4, max_blocks=8)
    t = dev.alloc_paged(pool)
    dev.append_paged(t, torch.zeros(1, 2, 32, 8, dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(SandyError, match="paged pool capacity exceeded"):
        dev.append_paged(t, torch.zeros(1, 2, 1, 8, dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(SandyError, match="dtype mismatch"):
        dev.append_paged(t, torch.zeros(1, 2, 1, 8, dtype=torch.float32, device="cuda"))


def test_paged_append_and_read_match_cpu_semantics(dev):
    """Chunks of any length appended to several tensors read back as the
    concatenation along the grow dim (CpuDevice.cpp:465-554, 611-676)."""
    from sandyrt_amd._lib import BF16
    torch.cuda.synchronize()
    pool = dev.create_paged_pool([1, 4, -1, 64], BF16, 2, 16, initial_pages=4, max_tensors=8, max_blocks=64)
    r = rng(1)
    tensors = [dev.alloc_paged(pool) for _ in range(3)]
    want = {t: [] for t in tensors}
    for step, lens in enumerate([(37, 1, 16), (1, 15, 1), (1, 1, 17), (40, 3, 1)]):
        for t, n in zip(tensors, lens):
            chunk = from_f32(normal(r, (1, 4, n, 64)), torch.bfloat16)
            torch.cuda.synchronize()
            dev.append_paged(t, chunk)
            want[t].append(bf16_np(chunk))
    dev.synchronize()
    for t in tensors:
        dense = np.concatenate(want[t], axis=2)
        got = dev.read_paged(t, np.uint16)
        assert got.shape == dense.shape
        assert np.array_equal(got, dense)
        m = dev.paged_meta(t)
        assert m.grow_length == dense.shape[2] and m.page_count == (dense.shape[2] + 15) // 16
    # freed pages are reused by the next tensor
    dev.dealloc_paged(tensors[0])
    t4 = dev.alloc_paged(pool)
    chunk = from_f32(normal(r, (1, 4, 20, 64)), torch.bfloat16)
    torch.cuda.synchronize()
    dev.append_paged(t4, chunk)
    assert np.array_equal(dev.read_paged(t4, np.uint16), bf16_np(chunk))


def _decode_setup(dev, r, B, hq, hkv, D, ctx, P=16):
    from sandyrt_amd._lib import BF16
    kp = dev.create_paged_pool([1, hkv, -1, D], BF16, 2, P, max_tensors=B, max_blocks=256)
    vp = dev.create_paged_pool([1, hkv, -1, D], BF16, 2, P, max_tensors=B, max_blocks=256)
    ks = [dev.alloc_paged(kp) for _ in range(B)]
    vs = [dev.alloc_paged(vp) for _ in range(B)]
    dense_k, dense_v = [], []
    for b in range(B):
        k = from_f32(normal(r, (1, hkv, ctx[b], D)), torch.bfloat16)
        v = from_f32(normal(r, (1, hkv, ctx[b], D)), torch.bfloat16)
        torch.cuda.synchronize()
        dev.append_paged(ks[b], k)
        dev.append_paged(vs[b], v)
        dense_k.append(bf16_np(k))
        dense_v.append(bf16_np(v))
    return kp, vp, ks, vs, dense_k, dense_v


def _attend(dev, kp, vp, q, pos, out, B):
    from sandyrt_amd import _lib
    kc, table, _ = dev.paged_views(kp)
    vc, _, _ = dev.paged_views(vp)
    table.contents.dims[0] = B  # rows 0..B-1 are the tensors in allocation order
    _lib.call("sandy_hip_paged_attention", _lib.desc(q), kc, vc, table, _lib.desc(pos), 0, 0.125, _lib.desc(out),
              stream=dev.stream)


def test_decode_step_append_positions_attention(dev, oracle):
    """One decode step entirely on the device: append the new K/V row of every
    sequence at its device-side length, derive positions, attend."""
    r = rng(7)
    B, hq, hkv, D = 4, 32, 4, 64
    ctx = [1, 15, 16, 300]
    kp, vp, ks, vs, dk, dv = _decode_setup(dev, r, B, hq, hkv, D, ctx)
    newk = from_f32(normal(r, (B, hkv, 1, D)), torch.bfloat16)
    newv = from_f32(normal(r, (B, hkv, 1, D)), torch.bfloat16)
    q = from_f32(normal(r, (B, hq, 1, D)), torch.bfloat16)
    pos = torch.zeros(B, dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    torch.cuda.synchronize()
    dev.append_step(kp, ks, newk)
    dev.append_step(vp, vs, newv)
    dev.positions(kp, ks, pos)
    _attend(dev, kp, vp, q, pos, out, B)
    dev.synchronize()
    from sandyrt_amd import _lib
    _lib.take_device_errors(stream=dev.stream)
    assert pos.cpu().tolist() == [c for c in ctx]  # new length - 1
    T = max(ctx) + 1
    kd = np.zeros((B, hkv, T, D), np.uint16)
    vd = np.zeros_like(kd)
    for b in range(B):
        kd[b, :, :ctx[b] + 1] = np.concatenate([dk[b][0], bf16_np(newk[b:b + 1])[0]], axis=1)
        vd[b, :, :ctx[b] + 1] = np.concatenate([dv[b][0], bf16_np(newv[b:b + 1])[0]], axis=1)
        assert np.array_equal(dev.read_paged(ks[b], np.uint16)[0], kd[b, :, :ctx[b] + 1])
    want = oracle.attention(bf16_np(q), kd, vd, np.array(ctx, np.int64), 0, 0.125)
    assert_close(out, want, torch.bfloat16, "device decode step")


def test_graph_captured_decode_steps_match_eager(dev):
    """A captured decode step (two appends, positions, attention) replayed
    three times matches the same three steps run eagerly on a twin pool."""
    r = rng(9)
    B, hq, hkv, D = 3, 8, 2, 64
    ctx = [5, 40, 100]
    a = _decode_setup(dev, np.random.default_rng(1), B, hq, hkv, D, ctx)
    b = _decode_setup(dev, np.random.default_rng(1), B, hq, hkv, D, ctx)
    steps = 3
    rows_k = [from_f32(normal(r, (B, hkv, 1, D)), torch.bfloat16) for _ in range(steps)]
    rows_v = [from_f32(normal(r, (B, hkv, 1, D)), torch.bfloat16) for _ in range(steps)]
    q = from_f32(normal(r, (B, hq, 1, D)), torch.bfloat16)
    # graph inputs live in fixed buffers that are refilled between replays
    gk = torch.empty_like(rows_k[0])
    gv = torch.empty_like(rows_v[0])
    pos_a = torch.zeros(B, dtype=torch.int32, device="cuda")
    pos_b = torch.zeros(B, dtype=torch.int32, device="cuda")
    out_a = torch.empty_like(q)
    out_b = torch.empty_like(q)
    for t in a[2] + a[3]:  # reserve pages for the captured steps
        m = dev.paged_meta(t)
        dev.reserve_paged(t, (m.grow_length + steps + 15) // 16)
    # warm the attention workspace outside capture
    dev.positions(a[0], a[2], pos_a)
    _attend(dev, a[0], a[1], q, pos_a, out_a, B)
    torch.cuda.synchronize()
    dev.synchronize()
    dev.graph_begin()
    dev.append_step(a[0], a[2], gk)
    dev.append_step(a[1], a[3], gv)
    dev.positions(a[0], a[2], pos_a)
    _attend(dev, a[0], a[1], q, pos_a, out_a, B)
    graph = dev.graph_end()
    for s in range(steps):
        gk.copy_(rows_k[s])
        gv.copy_(rows_v[s])
        torch.cuda.synchronize()
        dev.graph_launch(graph)
        dev.synchronize()
        got = out_a.clone()
        dev.append_step(b[0], b[2], rows_k[s])
        dev.append_step(b[1], b[3], rows_v[s])
        dev.positions(b[0], b[2], pos_b)
        _attend(dev, b[0], b[1], q, pos_b, out_b, B)
        dev.synchronize()
        assert torch.equal(got, out_b), f"replay {s} differs from eager"
        assert torch.equal(pos_a, pos_b)
    dev.paged_sync(a[0])
    assert dev.paged_meta(a[2][2]).grow_length == ctx[2] + steps
    dev.graph_destroy(graph)


@pytest.mark.parametrize("split_half", [True, False])
def test_decode_qkv_matches_rope_and_step_append(split_half):
    """sandy_hip_device_decode_qkv == sandy_hip_rope (q and k, per-sequence
    positions) + sandy_hip_device_paged_append_step (k and v), bit for bit."""
    from sandyrt_amd import ops
    from sandyrt_amd._lib import BF16
    from sandyrt_amd.device import HipDevice
    B, hq, hkv, D, P = 3, 8, 2, 64, 16
    dev = HipDevice(0)
    try:
        pools, seqs = [], []
        for _ in range(4):  # fused K, fused V, reference K, reference V
            p = dev.create_paged_pool([1, hkv, -1, D], BF16, 2, P, max_tensors=B, max_blocks=8)
            ids = [dev.alloc_paged(p) for _ in range(B)]
            pools.append(p)
            seqs.append(ids)
        g = torch.Generator(device="cuda")
        g.manual_seed(3)
        for s, n in enumerate([15, 16, 40]):
            k0 = torch.randn(1, hkv, n, D, generator=g, device="cuda").to(torch.bfloat16)
            v0 = torch.randn(1, hkv, n, D, generator=g, device="cuda").to(torch.bfloat16)
            for i, t in ((0, k0), (1, v0), (2, k0), (3, v0)):
                dev.reserve_paged(seqs[i][s], 8)
                dev.append_paged(seqs[i][s], t)
        qkv = torch.randn(B, (hq + 2 * hkv) * D, generator=g, device="cuda").to(torch.bfloat16)
        pos = torch.tensor([15, 16, 40], dtype=torch.int64, device="cuda")
        q_out = torch.empty(B, hq, 1, D, dtype=torch.bfloat16, device="cuda")
        dev.decode_qkv(pools[0], seqs[0], pools[1], seqs[1], qkv, hq, pos, 1e4, q_out, split_half=split_half)
        # reference path: rope over [1, heads, B, D] views with position_ids[b], then the step appends
        q_ref = ops.rope(qkv[:, :hq * D].reshape(B, hq, D).permute(1, 0, 2).unsqueeze(0).contiguous(), 1e4,
                         split_half=split_half, position_ids=pos)
        k_ref = ops.rope(qkv[:, hq * D:(hq + hkv) * D].reshape(B, hkv, D).permute(1, 0, 2).unsqueeze(0).contiguous(),
                         1e4, split_half=split_half, position_ids=pos)
        k_rows = k_ref[0].permute(1, 0, 2).contiguous().view(B, hkv, 1, D)
        v_rows = qkv[:, (hq + hkv) * D:].contiguous().view(B, hkv, 1, D)
        dev.append_step(pools[2], seqs[2], k_rows)
        dev.append_step(pools[3], seqs[3], v_rows)
        dev.synchronize()
        ops.check_device_errors()
        assert torch.equal(q_out.view(B, hq, D), q_ref[0].permute(1, 0, 2))
        for s in range(B):
            for fused, ref in ((0, 2), (1, 3)):
                dev.paged_sync(pools[fused])
                dev.paged_sync(pools[ref])
                got = dev.read_paged(seqs[fused][s], np.uint16)
                assert got.shape[2] == [15, 16, 40][s] + 1
                assert np.array_equal(got, dev.read_paged(seqs[ref][s], np.uint16))
    finally:
        dev.close()


# (sequences, q heads, kv heads, head dim, k): TinyLlama's 32/4 x 64 at 1,
# 3 and 33 rows (16-column tiles at one row, 32-column tiles and three row
# tiles beyond), Gemma-like 8/2 x 256 with k 2560 (K split over two
# workgroups, last-arriving sum before the epilogue)
QKV_SHAPES = [(1, 32, 4, 64, 2048), (3, 32, 4, 64, 2048), (33, 8, 2, 64, 512), (4, 8, 2, 256, 2560)]


@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("split_half", [True, False])
@pytest.mark.parametrize("shape", QKV_SHAPES)
def test_matmul_qkv_matches_gemm_then_decode_qkv(shape, split_half, norm):
    _check_matmul_qkv(shape, split_half, norm, 16, torch.int64)


@pytest.mark.parametrize("page,pos_dtype", [(32, torch.int32), (8, torch.int64), (64, torch.int32)])
def test_matmul_qkv_page_sizes_and_int32_positions(page, pos_dtype):
    """Other page sizes (row within the page and block index from the page
    shift) and int32 positions, bit for bit against the two-launch path."""
    _check_matmul_qkv((5, 16, 4, 128, 1024), True, True, page, pos_dtype)


def _check_matmul_qkv(shape, split_half, norm, P, pos_dtype):
    """sandy_hip_device_matmul_qkv (q/k weight rows pair-ordered) == the q/k/v
    GEMM (sandy_hip_matmul_rms / sandy_hip_matmul) into a buffer followed by
    sandy_hip_device_decode_qkv: q rows, K/V pages and lengths bit for bit."""
    from sandyrt_amd import ops
    from sandyrt_amd._lib import BF16
    from sandyrt_amd.device import HipDevice
    B, hq, hkv, D, K = shape
    dev = HipDevice(0)
    try:
        pools, seqs = [], []
        for _ in range(4):  # fused K, fused V, reference K, reference V
            p = dev.create_paged_pool([1, hkv, -1, D], BF16, 2, P, max_tensors=B, max_blocks=128 // P + 1)
            pools.append(p)
            seqs.append([dev.alloc_paged(p) for _ in range(B)])
        g = torch.Generator(device="cuda")
        g.manual_seed(5)
        ctx = [(7 * s + 15) % 97 for s in range(B)]  # ragged, some on page boundaries
        ctx[0] = 16
        for s, n in enumerate(ctx):
            k0 = torch.randn(1, hkv, n, D, generator=g, device="cuda").to(torch.bfloat16)
            v0 = torch.randn(1, hkv, n, D, generator=g, device="cuda").to(torch.bfloat16)
            for i, t in ((0, k0), (1, v0), (2, k0), (3, v0)):
                dev.reserve_paged(seqs[i][s], 128 // P + 1)
                dev.append_paged(seqs[i][s], t)
        n = (hq + 2 * hkv) * D
        x = torch.randn(B, K, generator=g, device="cuda").to(torch.bfloat16)
        w = (torch.randn(n, K, generator=g, device="cuda") * K ** -0.5).to(torch.bfloat16)
        nw = (1 + 0.1 * torch.randn(K, generator=g, device="cuda")).to(torch.bfloat16)
        pos = torch.tensor(ctx, dtype=pos_dtype, device="cuda")
        q_got = torch.empty(B, hq, 1, D, dtype=torch.bfloat16, device="cuda")
        q_ref = torch.empty_like(q_got)
        stats = None
        if norm:  # exact float64 sums of squares per (row, 16-column group), as the residual epilogue leaves them
            v = x.double().cpu().numpy()
            stats = torch.from_numpy((v * v).reshape(B, K // 16, 16).sum(axis=2)).cuda()
            qkv = ops.matmul_rms(x, stats, nw, 1e-5, w)
        else:
            qkv = ops.matmul(x, w, transpose_rhs=True)
        wp = ops.pair_rope_weight(w, hq, hkv, D, split_half)
        dev.matmul_qkv(x, wp, pools[0], seqs[0], pools[1], seqs[1], hq, pos, 1e4, q_got, split_half=split_half,
                       stats=stats, norm_weight=nw if norm else None, eps=1e-5)
        dev.decode_qkv(pools[2], seqs[2], pools[3], seqs[3], qkv, hq, pos, 1e4, q_ref, split_half=split_half)
        dev.synchronize()
        ops.check_device_errors()
        assert torch.equal(q_got, q_ref)
        for s in range(B):
            for fused, ref in ((0, 2), (1, 3)):
                dev.paged_sync(pools[fused])
                dev.paged_sync(pools[ref])
                got = dev.read_paged(seqs[fused][s], np.uint16)
                assert got.shape[2] == ctx[s] + 1
                assert np.array_equal(got, dev.read_paged(seqs[ref][s], np.uint16)), (s, fused)
        # device lengths advanced: the next positions are ctx + 1
        nxt = torch.empty(B, dtype=torch.int64, device="cuda")
        dev.lengths(pools[0], seqs[0], nxt)
        dev.lengths(pools[1], seqs[1], pos)
        dev.synchronize()
        assert nxt.tolist() == [c + 1 for c in ctx] and pos.tolist() == nxt.tolist()
    finally:
        dev.close()


@pytest.mark.parametrize("split_half", [True, False])
def test_matmul_qkv_matches_oracle_chain(oracle, split_half):
    """sandy_hip_device_matmul_qkv at TinyLlama's width against the oracle's
    op chain (RMSNorm, q/k/v matmul, RoPE of q and k at each sequence's
    position): the q rows and the K/V rows appended at that position, bf16
    tolerance per op, the earlier history untouched."""
    from sandyrt_amd import ops
    from sandyrt_amd._lib import BF16
    from sandyrt_amd.device import HipDevice
    B, hq, hkv, D, K, P = 3, 32, 4, 64, 2048, 16
    dev = HipDevice(0)
    try:
        kp = dev.create_paged_pool([1, hkv, -1, D], BF16, 2, P, max_tensors=B, max_blocks=8)
        vp = dev.create_paged_pool([1, hkv, -1, D], BF16, 2, P, max_tensors=B, max_blocks=8)
        ks, vs = [dev.alloc_paged(kp) for _ in range(B)], [dev.alloc_paged(vp) for _ in range(B)]
        r = rng(91 + split_half)
        ctx = [16, 5, 47]
        hist = []
        for s, n in enumerate(ctx):
            k0 = from_f32(normal(r, (1, hkv, n, D)), torch.bfloat16)
            v0 = from_f32(normal(r, (1, hkv, n, D)), torch.bfloat16)
            for t, h in ((ks[s], k0), (vs[s], v0)):
                dev.reserve_paged(t, 8)
                dev.append_paged(t, h)
            hist.append((to_oracle(k0), to_oracle(v0)))
        x = from_f32(normal(r, (B, K)), torch.bfloat16)
        w = from_f32(normal(r, ((hq + 2 * hkv) * D, K), K ** -0.5), torch.bfloat16)
        nw = from_f32(1.0 + normal(r, (K,), 0.1), torch.bfloat16)
        v = x.double().cpu().numpy()
        stats = torch.from_numpy((v * v).reshape(B, K // 16, 16).sum(axis=2)).cuda()
        pos = torch.tensor(ctx, dtype=torch.int64, device="cuda")
        q_got = torch.empty(B, hq, 1, D, dtype=torch.bfloat16, device="cuda")
        dev.matmul_qkv(x, ops.pair_rope_weight(w, hq, hkv, D, split_half), kp, ks, vp, vs, hq, pos, 1e4, q_got,
                       split_half=split_half, stats=stats, norm_weight=nw, eps=1e-5)
        dev.synchronize()
        ops.check_device_errors()
        qkv = oracle.matmul(oracle.rms_norm(to_oracle(x), to_oracle(nw), 1e-5), to_oracle(w), transpose_rhs=True)
        positions = np.array(ctx, np.int64)

        def roped(lo, heads):  # [1, heads, B, D] with sequence b at position ctx[b]
            t = np.ascontiguousarray(qkv[:, lo:lo + heads * D].reshape(B, heads, D).transpose(1, 0, 2)[None])
            return oracle.rope(t, 1e4, split_half=split_half, position_ids=positions)[0].transpose(1, 0, 2)

        assert_close(q_got.view(B, hq, D), roped(0, hq), torch.bfloat16, "q")
        k_new = roped(hq * D, hkv)
        v_new = qkv[:, (hq + hkv) * D:].reshape(B, hkv, D)
        dev.paged_sync(kp)
        dev.paged_sync(vp)
        for s in range(B):
            gk = dev.read_paged(ks[s], np.uint16)
            gv = dev.read_paged(vs[s], np.uint16)
            assert gk.shape[2] == gv.shape[2] == ctx[s] + 1
            assert np.array_equal(gk[:, :, :ctx[s]], hist[s][0]) and np.array_equal(gv[:, :, :ctx[s]], hist[s][1])
            assert_close(gk[0, :, ctx[s]], k_new[s], torch.bfloat16, f"k row of sequence {s}")
            assert_close(gv[0, :, ctx[s]], v_new[s], torch.bfloat16, f"v row of sequence {s}")
    finally:
        dev.close()


def test_matmul_qkv_position_must_equal_length():
    """A position that is not the sequence's length is reported as a device
    position error (SANDY_DEVERR_POSITION) and leaves the length as it was."""
    from sandyrt_amd import ops
    from sandyrt_amd._lib import BF16, SandyError
    from sandyrt_amd.device import HipDevice
    dev = HipDevice(0)
    try:
        kp = dev.create_paged_pool([1, 2, -1, 64], BF16, 2, 16, max_tensors=1, max_blocks=4)
        vp = dev.create_paged_pool([1, 2, -1, 64], BF16, 2, 16, max_tensors=1, max_blocks=4)
        k, v = dev.alloc_paged(kp), dev.alloc_paged(vp)
        dev.reserve_paged(k, 4)
        dev.reserve_paged(v, 4)
        x = torch.ones(1, 64, dtype=torch.bfloat16, device="cuda")
        w = torch.zeros(12 * 64, 64, dtype=torch.bfloat16, device="cuda")
        q = torch.empty(1, 8, 1, 64, dtype=torch.bfloat16, device="cuda")
        pos = torch.tensor([3], dtype=torch.int64, device="cuda")
        dev.matmul_qkv(x, w, kp, [k], vp, [v], 8, pos, 1e4, q)
        with pytest.raises(SandyError, match="position"):
            ops.check_device_errors()
        nxt = torch.empty(1, dtype=torch.int64, device="cuda")
        dev.lengths(kp, [k], nxt)
        dev.synchronize()
        assert nxt.tolist() == [0]
        with pytest.raises(SandyError, match="weight must be"):
            dev.matmul_qkv(x, w[:700], kp, [k], vp, [v], 8, pos, 1e4, q)
        # one tensor named by two sequences: rejected before any length moves
        x2 = torch.ones(2, 64, dtype=torch.bfloat16, device="cuda")
        q2 = torch.empty(2, 8, 1, 64, dtype=torch.bfloat16, device="cuda")
        pos2 = torch.zeros(2, dtype=torch.int64, device="cuda")
        with pytest.raises(SandyError, match="tensors must be distinct"):
            dev.matmul_qkv(x2, w, kp, [k, k], vp, [v, v], 8, pos2, 1e4, q2)
        with pytest.raises(SandyError, match="tensors must be distinct"):
            dev.decode_qkv(kp, [k, k], vp, [v, v], torch.zeros(2, 12 * 64, dtype=torch.bfloat16, device="cuda"), 8,
                           pos2, 1e4, q2)
        assert dev.paged_meta(k).grow_length == 1  # only the one call above that launched
    finally:
        dev.close()


def test_matmul_qkv_stale_position_keeps_history():
    """A position behind the sequence's length (a stale one) is reported as a
    device position error and stores nothing: the committed K/V rows stay as
    they were.  A call that fails a check of the GEMM itself (bad row
    statistics) fails before any length moves."""
    from sandyrt_amd import ops
    from sandyrt_amd._lib import BF16, SandyError
    from sandyrt_amd.device import HipDevice
    dev = HipDevice(0)
    try:
        kp = dev.create_paged_pool([1, 2, -1, 64], BF16, 2, 16, max_tensors=1, max_blocks=4)
        vp = dev.create_paged_pool([1, 2, -1, 64], BF16, 2, 16, max_tensors=1, max_blocks=4)
        k, v = dev.alloc_paged(kp), dev.alloc_paged(vp)
        g = torch.Generator().manual_seed(7)
        w = torch.randn(12 * 64, 64, generator=g).to(torch.bfloat16).cuda()
        q = torch.empty(1, 8, 1, 64, dtype=torch.bfloat16, device="cuda")
        for p in range(2):
            x = torch.randn(1, 64, generator=g).to(torch.bfloat16).cuda()
            dev.matmul_qkv(x, w, kp, [k], vp, [v], 8, torch.tensor([p], device="cuda"), 1e4, q)
        ops.check_device_errors()
        dev.paged_sync(kp)
        dev.paged_sync(vp)
        k0, v0 = dev.read_paged(k, np.uint16).copy(), dev.read_paged(v, np.uint16).copy()
        assert k0.shape[2] == 2 and np.any(k0 != 0) and np.any(v0 != 0)
        x = torch.randn(1, 64, generator=g).to(torch.bfloat16).cuda()
        for stale in (0, 1):  # two behind the length, and one (pos = len - 1)
            dev.matmul_qkv(x, w, kp, [k], vp, [v], 8, torch.tensor([stale], device="cuda"), 1e4, q)
            with pytest.raises(SandyError, match="position"):
                ops.check_device_errors()
            dev.paged_sync(kp)
            dev.paged_sync(vp)
            np.testing.assert_array_equal(dev.read_paged(k, np.uint16), k0)
            np.testing.assert_array_equal(dev.read_paged(v, np.uint16), v0)
        nxt = torch.empty(1, dtype=torch.int64, device="cuda")
        dev.lengths(kp, [k], nxt)
        dev.synchronize()
        assert nxt.tolist() == [2]
        # bad row statistics (3 parts for a 64-wide row, which has 4)
        bad_stats = torch.zeros(1, 3, dtype=torch.float64, device="cuda")
        nw = torch.ones(64, dtype=torch.bfloat16, device="cuda")
        with pytest.raises(SandyError, match="row statistics"):
            dev.matmul_qkv(x, w, kp, [k], vp, [v], 8, torch.tensor([2], device="cuda"), 1e4, q, stats=bad_stats,
                           norm_weight=nw, eps=1e-5)
        with pytest.raises(SandyError, match="norm weight"):
            dev.matmul_qkv(x, w, kp, [k], vp, [v], 8, torch.tensor([2], device="cuda"), 1e4, q,
                           stats=torch.zeros(1, 4, dtype=torch.float64, device="cuda"), norm_weight=nw[:32], eps=1e-5)
        assert dev.paged_meta(k).grow_length == 2 and dev.paged_meta(v).grow_length == 2
        dev.lengths(kp, [k], nxt)
        dev.synchronize()
        assert nxt.tolist() == [2]
    finally:
        dev.close()


def test_decode_qkv_rejects_bad_shapes():
    from sandyrt_amd._lib import BF16, SandyError
    from sandyrt_amd.device import HipDevice
    dev = HipDevice(0)
    try:
        kp = dev.create_paged_pool([1, 2, -1, 64], BF16, 2, 16, max_tensors=2, max_blocks=4)
        vp = dev.create_paged_pool([1, 2, -1, 64], BF16, 2, 16, max_tensors=2, max_blocks=4)
        k, v = dev.alloc_paged(kp), dev.alloc_paged(vp)
        pos = torch.zeros(1, dtype=torch.int64, device="cuda")
        q_out = torch.empty(1, 8, 1, 64, dtype=torch.bfloat16, device="cuda")
        bad = torch.zeros(1, 100, dtype=torch.bfloat16, device="cuda")
        with pytest.raises(SandyError, match="decode qkv input must be"):
            dev.decode_qkv(kp, [k], vp, [v], bad, 8, pos, 1e4, q_out)
        good = torch.zeros(1, 12 * 64, dtype=torch.bfloat16, device="cuda")
        with pytest.raises(SandyError, match="attention heads must be divisible by kv_heads"):
            dev.decode_qkv(kp, [k], vp, [v], good, 7, pos, 1e4, q_out)
    finally:
        dev.close()


# (rows per sequence, row bytes): the pre-requested fast form (<= 16 rows of
# <= 1 KiB, 16-byte multiples) at its limits, and the loop forms past them
# (17 rows, 2 KiB rows, 6-byte rows).
STEP_SHAPES = [(12, 256), (16, 1024), (17, 128), (4, 2048), (3, 6)]


@pytest.mark.parametrize("prefix,row_bytes", STEP_SHAPES)
def test_append_step_row_shapes_bit_exact(dev, prefix, row_bytes):
    """Several decode steps of append_step, read back as the concatenation of
    the rows (CpuDevice.cpp:465-554, 611-676), bit for bit."""
    from sandyrt_amd._lib import BF16
    inner = row_bytes // 2
    count = 3
    torch.cuda.synchronize()
    pool = dev.create_paged_pool([1, prefix, -1, inner], BF16, 2, 16, max_tensors=count, max_blocks=8)
    ts = [dev.alloc_paged(pool) for _ in range(count)]
    r = rng(prefix * 1000 + row_bytes)
    want = [[] for _ in ts]
    for step in range(18):  # crosses a page boundary
        rows = from_f32(normal(r, (count, prefix, 1, inner)), torch.bfloat16)
        torch.cuda.synchronize()
        dev.append_step(pool, ts, rows)
        for i in range(count):
            want[i].append(bf16_np(rows[i:i + 1]))
    dev.synchronize()
    for i, t in enumerate(ts):
        assert np.array_equal(dev.read_paged(t, np.uint16), np.concatenate(want[i], axis=2))


def test_append_step_misaligned_rows_view(dev):
    """A rows view whose storage offset leaves it 2 bytes off 16-byte
    alignment takes the element-wise copy and still appends exactly."""
    from sandyrt_amd._lib import BF16
    prefix, inner, count = 4, 64, 2
    torch.cuda.synchronize()
    pool = dev.create_paged_pool([1, prefix, -1, inner], BF16, 2, 16, max_tensors=count, max_blocks=4)
    ts = [dev.alloc_paged(pool) for _ in range(count)]
    r = rng(5)
    base = from_f32(normal(r, (count * prefix * inner + 1,)), torch.bfloat16)
    rows = base[1:].view(count, prefix, 1, inner)
    assert rows.data_ptr() % 16 == 2
    torch.cuda.synchronize()
    dev.append_step(pool, ts, rows)
    dev.synchronize()
    for i, t in enumerate(ts):
        assert np.array_equal(dev.read_paged(t, np.uint16), bf16_np(rows[i:i + 1].contiguous()))


def test_append_step_rejects_repeated_tensor(dev):
    from sandyrt_amd._lib import BF16, SandyError
    pool = dev.create_paged_pool([1, 2, -1, 64], BF16, 2, 16, max_tensors=2, max_blocks=4)
    t = dev.alloc_paged(pool)
    rows = torch.zeros(2, 2, 1, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(SandyError, match="tensors must be distinct"):
        dev.append_step(pool, [t, t], rows)


def test_append_step_kv_equals_two_step_appends(dev):
    """K and V step appends in one launch: the pages read back as the rows
    appended, for both caches (a K and a V pool, three sequences, a page
    boundary crossed), lengths advanced on the host and the device."""
    from sandyrt_amd._lib import BF16
    count, hkv, D = 3, 2, 64
    torch.cuda.synchronize()
    kp = dev.create_paged_pool([1, hkv, -1, D], BF16, 2, 16, max_tensors=count, max_blocks=4)
    vp = dev.create_paged_pool([1, hkv, -1, D], BF16, 2, 16, max_tensors=count, max_blocks=4)
    ks, vs = [dev.alloc_paged(kp) for _ in range(count)], [dev.alloc_paged(vp) for _ in range(count)]
    r = rng(77)
    want_k, want_v = [[] for _ in ks], [[] for _ in vs]
    for step in range(20):
        kr = from_f32(normal(r, (count, hkv, 1, D)), torch.bfloat16)
        vr = from_f32(normal(r, (count, hkv, 1, D)), torch.bfloat16)
        torch.cuda.synchronize()
        dev.append_step_kv(kp, ks, vp, vs, kr, vr)
        for i in range(count):
            want_k[i].append(bf16_np(kr[i:i + 1]))
            want_v[i].append(bf16_np(vr[i:i + 1]))
    dev.synchronize()
    for i in range(count):
        assert dev.paged_meta(ks[i]).grow_length == 20 and dev.paged_meta(vs[i]).grow_length == 20
        assert np.array_equal(dev.read_paged(ks[i], np.uint16), np.concatenate(want_k[i], axis=2))
        assert np.array_equal(dev.read_paged(vs[i], np.uint16), np.concatenate(want_v[i], axis=2))
    lengths = torch.empty(count, dtype=torch.int64, device="cuda")
    dev.lengths(vp, vs, lengths)
    dev.synchronize()
    assert lengths.tolist() == [20] * count


def test_append_step_kv_rejects_before_moving_bookkeeping(dev):
    from sandyrt_amd._lib import BF16, SandyError
    kp = dev.create_paged_pool([1, 2, -1, 64], BF16, 2, 16, max_tensors=2, max_blocks=2)
    vp = dev.create_paged_pool([1, 2, -1, 64], BF16, 2, 16, max_tensors=2, max_blocks=2)
    ks, vs = [dev.alloc_paged(kp) for _ in range(2)], [dev.alloc_paged(vp) for _ in range(2)]
    good = torch.zeros(2, 2, 1, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(SandyError, match="rows shape mismatch"):
        dev.append_step_kv(kp, ks, vp, vs, good, torch.zeros(2, 2, 1, 32, dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(SandyError, match="tensors must be distinct"):
        dev.append_step_kv(kp, [ks[0], ks[0]], vp, vs, good, good)
    with pytest.raises(SandyError, match="paged tensor not found"):
        dev.append_step_kv(kp, ks, vp, [vs[0], ks[1]], good, good)  # a K tensor given as V
    for t in ks + vs:
        assert dev.paged_meta(t).grow_length == 0  # nothing moved
    with pytest.raises(SandyError, match="count out of range"):
        many = torch.zeros(65, 2, 1, 64, dtype=torch.bfloat16, device="cuda")
        dev.append_step_kv(kp, list(range(65)), vp, list(range(65)), many, many)
