"""GPU parity of decode attention over a paged KV cache (the MFMA hot path and
the general kernel) and of dense attention, against the oracle's restatement
of src/core/TensorCalc.cpp:1167-1314 on the dense K/V that the reference CPU
device materialises from pages (src/device/cpu/CpuDevice.cpp:611-676)."""
import os

import numpy as np
import pytest
import torch

from tests.helpers import assert_close, from_f32, normal, rng, to_oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from sandyrt_amd import ops
    return ops


def make_paged(r, B, hq, hkv, D, P, ctx, pool_pages, dtype, scale_q=1.0):
    """Random pools, per-sequence block tables drawn from a permutation of the pool."""
    max_blocks = max(1, int(max((c + P - 1) // P for c in ctx)))
    perm = r.permutation(pool_pages)
    need = sum((c + P - 1) // P for c in ctx)
    assert need <= pool_pages
    table = np.zeros((B, max_blocks), np.int32)
    off = 0
    for b, c in enumerate(ctx):
        n = (c + P - 1) // P
        table[b, :n] = perm[off:off + n]
        table[b, n:] = perm[(off + n) % pool_pages]  # padding entries point at real pages
        off += n
    kpool = from_f32(normal(r, (pool_pages, hkv, P, D)), dtype)
    vpool = from_f32(normal(r, (pool_pages, hkv, P, D)), dtype)
    q = from_f32(normal(r, (B, hq, 1, D), scale_q), dtype)
    pos = np.array([c - 1 for c in ctx], np.int64)
    return q, kpool, vpool, table, pos


def oracle_paged(oracle, q, kpool, vpool, table, pos, window, scale):
    B, hq, _, D = q.shape
    _, hkv, P, _ = kpool.shape
    tk = int(max(pos) + 1)
    kn, vn = to_oracle(kpool), to_oracle(vpool)
    kd = np.zeros((B, hkv, tk, D), kn.dtype)
    vd = np.zeros((B, hkv, tk, D), vn.dtype)
    for b in range(B):
        c = int(pos[b]) + 1
        kd[b, :, :c] = oracle.paged_to_dense(kn, table[b], hkv, c, P, D)
        vd[b, :, :c] = oracle.paged_to_dense(vn, table[b], hkv, c, P, D)
    return oracle.attention(to_oracle(q), kd, vd, pos, window, scale)


def run_case(ops, oracle, seed, B, hq, hkv, D, P, ctx, dtype, window=0, scale=-1.0, pool_pages=None, subset=None):
    r = rng(seed)
    pool_pages = pool_pages or sum((c + P - 1) // P for c in ctx) + 7
    q, kpool, vpool, table, pos = make_paged(r, B, hq, hkv, D, P, ctx, pool_pages, dtype)
    out = ops.paged_attention(q, ops.PagedCache(kpool), ops.PagedCache(vpool), torch.from_numpy(table).cuda(),
                              torch.from_numpy(pos).cuda(), window=window, scale=scale)
    ops.check_device_errors()
    if subset is not None:
        sel = np.array(subset)
        want = oracle_paged(oracle, q[sel], kpool, vpool, table[sel], pos[sel], window, scale)
        assert_close(out[sel], want, dtype, f"paged attention subset {subset}")
    else:
        want = oracle_paged(oracle, q, kpool, vpool, table, pos, window, scale)
        assert_close(out, want, dtype, "paged attention")
    return out


EDGE_CTX = [1, 2, 15, 16, 17, 63, 64, 65, 300, 513]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_paged_decode_tinyllama_heads(ops, oracle, dtype):
    """32 q / 4 kv heads, D 64, block 16 (config 3 geometry), ragged contexts."""
    run_case(ops, oracle, 2, len(EDGE_CTX), 32, 4, 64, 16, EDGE_CTX, dtype, scale=0.125)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_paged_decode_gemma_heads(ops, oracle, dtype):
    """8 q / 2 kv heads, D 256, scale 1.0 (config 4 geometry)."""
    run_case(ops, oracle, 3, 4, 8, 2, 256, 16, [1, 40, 1024, 1500], dtype, scale=1.0 / 16)


@pytest.mark.parametrize("group,D", [(1, 128), (16, 64), (2, 128), (5, 64), (3, 256)])
def test_paged_decode_group_shapes(ops, oracle, group, D):
    run_case(ops, oracle, 4 + group, 3, 2 * group, 2, D, 32, [70, 200, 33], torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("window", [1, 7, 64, 500])
def test_paged_decode_sliding_window(ops, oracle, window, dtype):
    run_case(ops, oracle, 10 + window, 4, 16, 2, 64, 16, [5, 100, 700, 1200], dtype, window=window)


def test_paged_decode_small_pages_use_general_kernel(ops, oracle):
    run_case(ops, oracle, 20, 3, 4, 2, 64, 2, [1, 9, 30], torch.bfloat16)
    run_case(ops, oracle, 21, 3, 4, 2, 32, 4, [3, 17, 30], torch.float32)


def test_paged_decode_config3_full_size(ops, oracle):
    """BASELINE config 3 at full size: 32 sequences, ctx U[512, 4096], a random
    permutation of a 32768-block pool; the oracle checks 4 of the sequences."""
    r = rng(2)
    ctx = [int(c) for c in r.integers(512, 4097, 32)]
    run_case(ops, oracle, 2, 32, 32, 4, 64, 16, ctx, torch.bfloat16, scale=0.125, pool_pages=32768,
             subset=[0, 7, 19, int(np.argmax(ctx))])


def test_paged_decode_repeat_and_split_invariance(ops, oracle, monkeypatch):
    """Repeated launches reuse the merge counters; different split sizes
    agree within tolerance."""
    r = rng(33)
    ctx = [4000, 2500, 900]
    q, kpool, vpool, table, pos = make_paged(r, 3, 32, 4, 64, 16, ctx, 1000, torch.bfloat16)
    args = (q, ops.PagedCache(kpool), ops.PagedCache(vpool), torch.from_numpy(table).cuda(), torch.from_numpy(pos).cuda())
    o1 = ops.paged_attention(*args)
    o2 = ops.paged_attention(*args)
    assert torch.equal(o1, o2)
    outs = []
    for split in ("256", "1024", "4096"):
        monkeypatch.setenv("SANDY_PAGED_SPLIT", split)
        outs.append(ops.paged_attention(*args))
    monkeypatch.delenv("SANDY_PAGED_SPLIT")
    want = oracle_paged(oracle, q, kpool, vpool, table, pos, 0, -1.0)
    for o in outs:
        assert_close(o, want, torch.bfloat16, "split size")


def test_paged_decode_bad_block_sets_device_error(ops):
    from sandyrt_amd._lib import SandyError
    kpool = torch.zeros(4, 1, 16, 64, dtype=torch.bfloat16, device="cuda")
    q = torch.zeros(1, 2, 1, 64, dtype=torch.bfloat16, device="cuda")
    table = torch.tensor([[0, 9]], dtype=torch.int32, device="cuda")
    ops.paged_attention(q, ops.PagedCache(kpool), ops.PagedCache(kpool.clone()), table,
                        torch.tensor([20], device="cuda"))
    with pytest.raises(SandyError, match="block id outside the pool"):
        ops.check_device_errors()


# ------------------------------------------------------------------ dense attention
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", [
    dict(B=2, hq=8, hkv=2, tq=1, tk=40, D=64, window=0, pos=[39, 17]),
    dict(B=1, hq=4, hkv=4, tq=3, tk=5, D=16, window=0, pos=None),
    dict(B=2, hq=4, hkv=1, tq=2, tk=30, D=32, window=5, pos=[20, 3]),
    dict(B=1, hq=2, hkv=1, tq=1, tk=4, D=16, window=3, pos=[20]),
    dict(B=1, hq=2, hkv=2, tq=4, tk=9, D=512, window=0, pos=[5]),
])
def test_dense_attention(ops, oracle, dtype, case):
    r = rng(case["tk"] + case["D"])
    q = from_f32(normal(r, (case["B"], case["hq"], case["tq"], case["D"]), 0.35), dtype)
    k = from_f32(normal(r, (case["B"], case["hkv"], case["tk"], case["D"]), 0.35), dtype)
    v = from_f32(normal(r, (case["B"], case["hkv"], case["tk"], case["D"])), dtype)
    pos = torch.tensor(case["pos"], device="cuda") if case["pos"] is not None else None
    got = ops.attention(q, k, v, pos, case["window"], -1.0)
    want = oracle.attention(to_oracle(q), to_oracle(k), to_oracle(v), pos.cpu().numpy() if pos is not None else None,
                            case["window"], -1.0)
    assert_close(got, want, dtype, f"attention {case}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_general_attention_staged_equals_unstaged(ops, monkeypatch, dtype):
    """Up to 2048 keys the general attention runs its staged form (row
    offsets, scores and probabilities in LDS, batched K/V loads);
    SANDY_ATTN_UNSTAGED forces the per-use form.  Same operation order:
    the outputs must agree bit for bit (dense and paged, windows, head
    dimensions that are not a multiple of the 64-value K batch)."""
    r = rng(77)
    for B, hq, hkv, tq, tk, D, window, pos in [(2, 8, 2, 1, 300, 64, 0, [299, 17]), (1, 4, 1, 3, 90, 100, 20, [80]),
                                              (1, 2, 2, 1, 2048, 64, 0, [2047]), (2, 2, 1, 2, 33, 512, 0, None)]:
        q = from_f32(normal(r, (B, hq, tq, D), 0.35), dtype)
        k = from_f32(normal(r, (B, hkv, tk, D), 0.35), dtype)
        v = from_f32(normal(r, (B, hkv, tk, D)), dtype)
        p_ = torch.tensor(pos, device="cuda") if pos is not None else None
        got = ops.attention(q, k, v, p_, window, -1.0)
        monkeypatch.setenv("SANDY_ATTN_UNSTAGED", "1")
        want = ops.attention(q, k, v, p_, window, -1.0)
        monkeypatch.delenv("SANDY_ATTN_UNSTAGED")
        assert torch.equal(got, want), (B, hq, hkv, tq, tk, D)
    # paged pools with small pages (the general kernel's paged form)
    q, kpool, vpool, table, pos = make_paged(r, 3, 4, 2, 64, 2, [1, 9, 30], 30, dtype)
    args = (q, ops.PagedCache(kpool), ops.PagedCache(vpool), torch.from_numpy(table).cuda(), torch.from_numpy(pos).cuda())
    got = ops.paged_attention(*args, window=5)
    monkeypatch.setenv("SANDY_ATTN_UNSTAGED", "1")
    want = ops.paged_attention(*args, window=5)
    monkeypatch.delenv("SANDY_ATTN_UNSTAGED")
    if dtype == torch.float32:  # fp32 decode steps take the decode kernel (its P.V sums in four key ranges)
        assert_close(got, to_oracle(want), dtype, "paged fp32 decode kernel vs general kernel")
    else:
        assert torch.equal(got, want), "paged"


def test_general_attention_long_keys_unstaged(ops, oracle):
    """More than 2048 keys take the per-use form (scores in the workspace)."""
    r = rng(78)
    q = from_f32(normal(r, (1, 2, 1, 64), 0.35), torch.float32)
    k = from_f32(normal(r, (1, 1, 2500, 64), 0.35), torch.float32)
    v = from_f32(normal(r, (1, 1, 2500, 64)), torch.float32)
    pos = torch.tensor([2400], device="cuda")
    got = ops.attention(q, k, v, pos, 0, -1.0)
    want = oracle.attention(to_oracle(q), to_oracle(k), to_oracle(v), pos.cpu().numpy(), 0, -1.0)
    assert_close(got, want, torch.float32, "attention 2500 keys")


def test_dense_attention_seeded_fuzz(ops, oracle):
    """The reference's own fuzz recipe (CudaDeviceTest.cpp:3082-3170): seed
    0x5a17d00d, uniform inputs, random windows, offsets and GQA groups."""
    r = np.random.default_rng(0x5A17D00D)
    for it in range(60):
        D = int(r.choice([64, 64, 128, 256]))
        B = 2 if r.random() < 0.25 else 1
        hkv = 2 if r.random() < 0.2 else 1
        hq = hkv * int(r.choice([1, 1, 2, 4]))
        tq = 1 if r.random() < 0.35 else int(2 + r.integers(0, 5))
        tk = int(1 + r.integers(0, 384)) if tq == 1 else int(1 + r.integers(0, 12))
        window = int(1 + r.integers(0, tk + tq + 4)) if r.random() < 0.7 else 0
        scale = float((0.5 + r.random() * 1.5) / np.sqrt(D))
        pos = r.integers(0, tk + tq + 5, B).astype(np.int64)
        qf = r.uniform(-0.35, 0.35, (B, hq, tq, D)).astype(np.float32)
        kf = r.uniform(-0.35, 0.35, (B, hkv, tk, D)).astype(np.float32)
        vf = r.uniform(-0.75, 0.75, (B, hkv, tk, D)).astype(np.float32)
        got = ops.attention(from_f32(qf, torch.float32), from_f32(kf, torch.float32), from_f32(vf, torch.float32),
                            torch.from_numpy(pos).cuda(), window, scale)
        want = oracle.attention(qf, kf, vf, pos, window, scale)
        np.testing.assert_allclose(got.cpu().numpy(), want, atol=5e-4, err_msg=f"iteration {it}")


@pytest.mark.parametrize("fused", ["0", "1"])
@pytest.mark.parametrize("split", ["128", "256", "512", "2048"])
def test_paged_decode_split_sizes(ops, oracle, monkeypatch, split, fused):
    """Every split size (one split per sequence written as final output,
    several merged by the merge kernel or by the last workgroup of each
    sequence and kv head) matches the oracle; repeated launches agree bit
    for bit."""
    monkeypatch.setenv("SANDY_PAGED_SPLIT", split)
    monkeypatch.setenv("SANDY_PAGED_FUSED_MERGE", fused)
    out1 = run_case(ops, oracle, 40, 5, 32, 4, 64, 16, [1, 300, 1500, 2049, 700], torch.bfloat16)
    out2 = run_case(ops, oracle, 40, 5, 32, 4, 64, 16, [1, 300, 1500, 2049, 700], torch.bfloat16)
    assert torch.equal(out1, out2)


@pytest.mark.parametrize("fused", ["0", "1"])
@pytest.mark.parametrize("split", ["128", "2048"])
@pytest.mark.parametrize("pos_dtype", [torch.int32, torch.int64])
def test_paged_decode_negative_position(ops, oracle, monkeypatch, pos_dtype, split, fused):
    """A negative position raises the reference's error when the device
    errors are read; the other sequences are still attended correctly and the
    bad row comes out zero (it owns no work unit)."""
    from sandyrt_amd._lib import SandyError
    monkeypatch.setenv("SANDY_PAGED_SPLIT", split)
    monkeypatch.setenv("SANDY_PAGED_FUSED_MERGE", fused)
    r = rng(91)
    ctx = [100, 50, 700, 1]
    q, kpool, vpool, table, pos = make_paged(r, 4, 8, 2, 64, 16, ctx, 80, torch.bfloat16)
    bad = pos.copy()
    bad[1] = -3
    out = ops.paged_attention(q, ops.PagedCache(kpool), ops.PagedCache(vpool), torch.from_numpy(table).cuda(),
                              torch.from_numpy(bad).to(pos_dtype).cuda(), window=0, scale=-1.0)
    with pytest.raises(SandyError, match="attention position_offsets must be non-negative"):
        ops.check_device_errors()
    sel = np.array([0, 2, 3])
    want = oracle_paged(oracle, q[sel], kpool, vpool, table[sel], pos[sel], 0, -1.0)
    assert_close(out[sel], want, torch.bfloat16, "rows with valid positions")
    assert torch.count_nonzero(out[1]).item() == 0


@pytest.mark.parametrize("B", [65, 150, 256, 300])
def test_paged_decode_many_sequences(ops, oracle, B):
    """Batches past one 64-lane scan chunk of the work-unit numbering,
    ragged short contexts."""
    r = rng(500 + B)
    ctx = [int(c) for c in r.integers(1, 90, B)]
    run_case(ops, oracle, 600 + B, B, 8, 2, 64, 16, ctx, torch.bfloat16)




@pytest.mark.parametrize("D,P", [(64, 16), (128, 64)])
def test_paged_decode_longest_first_unit_order(ops, oracle, D, P):
    """A grid past two rounds of resident workgroups (256 sequences of
    300..3000 keys: three 1024-key splits each at most, whole splits numbered
    before the shorter last splits), pages of 16 and 64 keys; against the
    oracle on a subset that holds the shortest, the longest and split-boundary
    lengths, and the whole batch against itself run twice (the merge adds
    the splits in split order whichever workgroup arrives last)."""
    r = rng(700 + D)
    ctx = [int(c) for c in r.integers(300, 3001, 256)]
    ctx[0], ctx[1], ctx[2], ctx[3] = 300, 3000, 1024, 2049
    sub = [0, 1, 2, 3, int(np.argmin(ctx)), int(np.argmax(ctx)), 100, 255]
    out1 = run_case(ops, oracle, 800 + D, 256, 16, 4, D, P, ctx, torch.bfloat16, subset=sub)
    out2 = run_case(ops, oracle, 800 + D, 256, 16, 4, D, P, ctx, torch.bfloat16, subset=sub)
    assert torch.equal(out1, out2)
