"""GPU parity of the MoE path against the oracle (src/core/TensorCalc.cpp
topk 1447-1518, moe_gather 1565-1667, moe_matmul 1669-1743, moe_scatter_sum
1745-1811) and of the router chain of src/models/gemma4a4b26b/common.sandy.go:
11-28.  Index outputs are compared exactly; the combine is bit-exact."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import assert_close, assert_equal, from_f32, from_oracle, normal, rng, to_oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from sandyrt_amd import ops
    return ops


# ------------------------------------------------------------------ top-k
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape,k", [((512, 128), 8), ((7, 64), 64), ((3, 1000), 17), ((4, 3000), 5), ((1, 1), 1),
                                     ((1, 50257), 1), ((2, 262144), 1), ((3, 4097), 16), ((2, 5000), 17),
                                     ((1, 1025), 1), ((5, 9000), 3)])
def test_topk_bit_exact(ops, oracle, dtype, shape, k):
    """Row kernels (axis <= 1024), the two-phase long-row kernels (chunk
    candidates then a merge; k <= 16) and the column fallback (k = 17)."""
    r = rng(shape[-1] + k)
    xf = np.round(normal(r, shape) * 3) / 3  # frequent ties: index order decides
    x = from_f32(xf, dtype)
    v, i = ops.topk(x, k)
    wv, wi = oracle.topk(to_oracle(x), k)
    assert_equal(i, wi, "topk indices")
    assert_equal(v, wv, "topk values")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_greedy_argmax_ties_take_lowest_id(ops, dtype):
    """Greedy selection over a vocabulary (Sampler.cpp:69-79: stable sort by
    logit, so equal maxima resolve to the lowest token id), with the maximum
    repeated across chunk boundaries."""
    r = rng(3)
    x = from_f32(normal(r, (3, 262144)), dtype)
    x[0, 70000] = 30.0
    x[0, 4095] = 30.0
    x[0, 200000] = 30.0
    x[1, 262143] = 31.0
    x[2, 8191] = 29.0
    x[2, 8192] = 29.0
    v, i = ops.topk(x, 1)
    assert i[:, 0].cpu().tolist() == [4095, 262143, 8191]
    assert v[:, 0].float().cpu().tolist() == [30.0, 31.0, 29.0]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_greedy_argmax_signed_zero_and_negative_rows(ops, oracle, dtype):
    """The one-pass argmax orders values through an integer key: -0 and +0
    must stay equal (index decides, the stored value keeps its sign bit),
    all-negative and -inf rows must resolve like the CPU."""
    x = torch.full((4, 20000), -5.0, dtype=dtype, device="cuda")
    x[0, :] = -1.0
    x[0, 7] = -0.0
    x[0, 9000] = 0.0          # equal to -0: lowest index (7) wins, value -0
    x[1, :] = float("-inf")   # every element equal: index 0
    x[2, 19999] = -4.0
    x[3, 123] = 0.0
    x[3, 50] = -0.0
    for _ in range(2):  # the second call runs on the slots the first reset
        v, i = ops.topk(x, 1)
        wv, wi = oracle.topk(to_oracle(x), 1)
        assert_equal(i, wi, "argmax indices")
        assert_equal(v, wv, "argmax values")
        assert torch.signbit(v.float()).cpu().tolist() == [[True], [True], [True], [True]]
        assert i[:, 0].cpu().tolist() == [7, 0, 19999, 50]


@pytest.mark.parametrize("shape", [(160, 262144), (64, 262144), (9, 100003)])
@pytest.mark.parametrize("index_dtype", [torch.int64, torch.int32])
def test_greedy_argmax_many_rows_repeated(ops, oracle, shape, index_dtype):
    """All three chunk widths of the one-pass argmax (the row count sets it),
    two calls in a row, int32 and int64 indices."""
    r = rng(shape[0])
    x = from_f32(np.round(normal(r, shape) * 4) / 4, torch.bfloat16)
    wv, wi = oracle.topk(to_oracle(x), 1, index_dtype=np.int64 if index_dtype == torch.int64 else np.int32)
    for _ in range(2):
        v, i = ops.topk(x, 1, index_dtype=index_dtype)
        assert_equal(i, wi, "argmax indices")
        assert_equal(v, wv, "argmax values")


def test_topk_middle_axis_and_i32(ops, oracle):
    r = rng(3)
    x = from_f32(np.round(normal(r, (3, 40, 5)) * 2) / 2, torch.float32)
    v, i = ops.topk(x, 6, axis=1, index_dtype=torch.int32)
    wv, wi = oracle.topk(to_oracle(x), 6, axis=1, index_dtype=np.int32)
    assert_equal(i, wi, "topk axis 1 indices")
    assert_equal(v, wv, "topk axis 1 values")


# ------------------------------------------------------------------ router chain (config 5)
def test_router_chain_config5(ops, oracle):
    """softmax -> top-8 -> sum -> div -> per-expert scale, logits [512, 128]
    N(0,1) seed 4 (fp32, as the router matmul produces)."""
    r = rng(4)
    logits = from_f32(normal(r, (512, 128)), torch.float32)
    scale_t = from_f32(np.abs(normal(r, (128,))) + 0.5, torch.float32)
    probs = ops.softmax(logits, -1)
    tw, tid = ops.topk(probs, 8)
    denom = ops.sum(tw, -1, True)
    div_nodes = [ops.ScalarNode(0, ops.LOAD, 0), ops.ScalarNode(1, ops.LOAD, 1), ops.ScalarNode(2, ops.DIV, operands=(0, 1))]
    tw = ops.elementwise(div_nodes, 2, [tw, denom.expand(512, 8).contiguous()])
    es = ops.embedding(tid, scale_t)
    mul_nodes = [ops.ScalarNode(0, ops.LOAD, 0), ops.ScalarNode(1, ops.LOAD, 1), ops.ScalarNode(2, ops.MUL, operands=(0, 1))]
    tw = ops.elementwise(mul_nodes, 2, [tw, es])

    p_ = oracle.softmax(to_oracle(logits), -1)
    wv, wi = oracle.topk(p_, 8)
    d_ = oracle.sum(wv, -1, True)
    wv = oracle.binary("div", wv, d_)
    es_ = oracle.embedding(wi, to_oracle(scale_t))
    wv = oracle.binary("mul", wv, es_)
    assert_equal(tid, wi, "router expert ids")
    assert_close(tw, wv, torch.float32, "router weights")


# ------------------------------------------------------------------ moe_gather
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("T,H,E,K", [(512, 2816, 128, 8), (37, 64, 16, 4), (5, 24, 300, 2), (1, 8, 4, 1),
                                     (700, 16, 64, 8), (130, 16, 8, 3), (1024, 16, 64, 8), (1100, 16, 64, 8),
                                     (3, 20, 1, 1)])
@pytest.mark.parametrize("idx", [np.int64, np.int32])
@pytest.mark.parametrize("ranking", ["dispatch", "general"])
def test_moe_gather_bit_exact(ops, oracle, monkeypatch, dtype, T, H, E, K, idx, ranking):
    """The token-major dispatch (the default up to 8192 routes with 16-byte
    rows), the expert-major dispatch (rows of other widths: H = 20 in bf16)
    and the single-workgroup ballot ranking plus row copy (the path past 8192
    routes, forced here by SANDY_MOE_ROUTE_GENERAL) give the reference's
    packing bit for bit; 1100 x 8 routes always take the general path."""
    if ranking == "general":
        monkeypatch.setenv("SANDY_MOE_ROUTE_GENERAL", "1")
    r = rng(T * 7 + E)
    ids = np.stack([r.permutation(E)[:K] for _ in range(T)]).astype(idx)
    w = np.abs(normal(r, (T, K)))
    x = from_f32(normal(r, (T, H)), dtype)
    wt = from_f32(w, dtype)
    tid = torch.from_numpy(ids).cuda()
    tdt = torch.int64 if idx == np.int64 else torch.int32
    px, pw, tok, off = ops.moe_gather(x, tid, wt, E, index_dtype=tdt)
    ops.check_device_errors()
    wpx, wpw, wtok, woff = oracle.moe_gather(to_oracle(x), ids, to_oracle(wt), E, index_dtype=idx)
    assert_equal(off, woff, "expert_offsets")
    assert_equal(tok, wtok, "token_ids")
    assert_equal(pw, wpw, "packed_weights")
    assert_equal(px, wpx, "packed_x")


def test_moe_gather_batched_and_skewed(ops, oracle):
    """Rank-3 inputs, and routes concentrated on few experts (long same-expert
    runs inside a wave exercise the ballot ranking)."""
    r = rng(12)
    B, T, H, E, K = 3, 300, 40, 8, 2
    ids = r.integers(0, 3, (B, T, K)).astype(np.int64)  # experts 0..2 only, repeats allowed
    x = from_f32(normal(r, (B, T, H)), torch.bfloat16)
    w = from_f32(np.abs(normal(r, (B, T, K))), torch.bfloat16)
    got = ops.moe_gather(x, torch.from_numpy(ids).cuda(), w, E)
    want = oracle.moe_gather(to_oracle(x), ids, to_oracle(w), E)
    for g, wnt, name in zip(got, want, ["packed_x", "packed_weights", "token_ids", "offsets"]):
        assert_equal(g, wnt, name)


def test_moe_gather_bad_expert_sets_device_error(ops):
    from sandyrt_amd._lib import SandyError
    x = torch.zeros(2, 8, device="cuda")
    ops.moe_gather(x, torch.tensor([[0], [9]], device="cuda"), torch.ones(2, 1, device="cuda"), 4)
    with pytest.raises(SandyError, match="moe_gather topk expert id out of range"):
        ops.check_device_errors()


@pytest.mark.parametrize("bad,tdt", [(-1, torch.int32), (-1, torch.int64), (1 << 33, torch.int64)])
def test_moe_gather_bad_expert_top8(ops, oracle, bad, tdt):
    """Top-8 routes (the dispatch compiled for 8 routes per token) with one
    invalid id: a negative one, or an int64 id whose high word is set.  The
    flag is raised and every valid route is still packed as the reference
    packs it (the invalid route is skipped)."""
    from sandyrt_amd._lib import SandyError
    r = rng(33)
    T, H, E, K = 40, 64, 16, 8
    ids = np.stack([r.permutation(E)[:K] for _ in range(T)]).astype(np.int64)
    ids[17, 3] = bad
    x = from_f32(normal(r, (T, H)), torch.bfloat16)
    w = from_f32(np.abs(normal(r, (T, K))), torch.bfloat16)
    px, pw, tok, off = ops.moe_gather(x, torch.from_numpy(ids).to(tdt).cuda(), w, E)
    with pytest.raises(SandyError, match="moe_gather topk expert id out of range"):
        ops.check_device_errors()
    valid = (ids >= 0) & (ids < E)
    keep = np.where(valid, ids, 0)
    # the reference's packing of the valid routes: expert-major, then token, then slot
    order = sorted((int(keep[t, k]), t, k) for t in range(T) for k in range(K) if valid[t, k])
    xs, ws = to_oracle(x), to_oracle(w)
    n = len(order)
    assert_equal(px[:n], np.stack([xs[t] for _, t, _ in order]), "packed_x")
    assert_equal(pw[:n], np.array([ws[t, k] for _, t, k in order]), "packed_weights")
    assert_equal(tok[:n], np.array([t for _, t, _ in order]), "token_ids")
    counts = np.bincount([e for e, _, _ in order], minlength=E)
    assert_equal(off, np.concatenate([[0], np.cumsum(counts)]), "expert_offsets")


# ------------------------------------------------------------------ moe_matmul
def oracle_matmul_experts(oracle, x, off, w, experts, transpose_rhs=True):
    """Oracle on selected experts only (each expert's rows are independent)."""
    out = {}
    for e in experts:
        lo, hi = int(off[e]), int(off[e + 1])
        if hi == lo:
            continue
        sub_off = np.array([0, hi - lo], np.int64)
        out[e] = oracle.moe_matmul(np.ascontiguousarray(x[lo:hi]), sub_off, np.ascontiguousarray(w[e:e + 1]), transpose_rhs)
    return out


def _moe_matmul_ragged(ops, oracle, dtype, transpose_rhs):
    """Ragged experts (empty, 1 row, more rows than one pass), K with an odd
    number of 32-wide steps, M not a multiple of a wave's columns."""
    r = rng(21)
    E, K, M = 6, 96, 40
    counts = np.array([0, 5, 17, 1, 40, 70])
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    x = from_f32(normal(r, (int(off[-1]), K)), dtype)
    w = from_f32(normal(r, (E, M, K) if transpose_rhs else (E, K, M), 0.2), dtype)
    got = ops.moe_matmul(x, torch.from_numpy(off).cuda(), w, transpose_rhs)
    want = oracle.moe_matmul(to_oracle(x), off, to_oracle(w), transpose_rhs)
    assert_close(got, want, dtype, "moe_matmul")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("transpose_rhs", [True, False])
def test_moe_matmul_small(ops, oracle, dtype, transpose_rhs):
    _moe_matmul_ragged(ops, oracle, dtype, transpose_rhs)


@pytest.mark.parametrize("tile", ["0", "1", "2", "3", "4", "5"])
def test_moe_matmul_tile_shapes(ops, oracle, monkeypatch, tile):
    """Every tile shape of the bf16 grouped-GEMM kernel on the ragged case."""
    monkeypatch.setenv("SANDY_MOE_GEMM", tile)
    _moe_matmul_ragged(ops, oracle, torch.bfloat16, True)


@pytest.mark.parametrize("shape", ["gate", "down"])
def test_moe_matmul_config5(ops, oracle, shape):
    """Config 5 grouped GEMM at full size (4096 routed rows, 128 experts);
    the oracle checks 4 experts, torch fp32 per-expert GEMMs check them all."""
    r = rng(4)
    E = 128
    K, M = (2816, 704) if shape == "gate" else (704, 2816)
    ids = np.stack([r.permutation(E)[:8] for _ in range(512)])
    counts = np.bincount(ids.reshape(-1), minlength=E)
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    g = torch.Generator(device="cuda").manual_seed(4)
    x = torch.randn(4096, K, generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn(E, M, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    got = ops.moe_matmul(x, torch.from_numpy(off).cuda(), w, True)
    xo, wo = to_oracle(x), None
    for e in [0, 1, int(np.argmax(counts)), E - 1]:
        lo, hi = int(off[e]), int(off[e + 1])
        want = oracle.moe_matmul(np.ascontiguousarray(xo[lo:hi]), np.array([0, hi - lo], np.int64),
                                 to_oracle(w[e:e + 1]), True)
        assert_close(got[lo:hi], want, torch.bfloat16, f"expert {e}")
    xf, wf = x.float(), w.float()
    for e in range(E):
        lo, hi = int(off[e]), int(off[e + 1])
        ref = (xf[lo:hi] @ wf[e].t()).to(torch.bfloat16)
        assert_close(got[lo:hi], to_oracle(ref), torch.bfloat16, f"expert {e} vs torch fp32")


def test_moe_matmul_bad_offsets_sets_device_error(ops):
    from sandyrt_amd._lib import SandyError
    x = torch.zeros(4, 32, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(2, 16, 32, dtype=torch.bfloat16, device="cuda")
    ops.moe_matmul(x, torch.tensor([0, 3, 9], device="cuda"), w, True)
    with pytest.raises(SandyError, match="moe_matmul invalid expert offsets"):
        ops.check_device_errors()


# ------------------------------------------------------------------ moe_scatter_sum
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("T,H,K", [(512, 2816, 8), (9, 24, 3), (4, 100, 2), (1100, 16, 8), (3, 16, 90), (2, 16, 150),
                                   (1, 8, 300), (5, 1024, 3), (6, 1040, 4)])
def test_moe_scatter_sum_bit_exact(ops, oracle, dtype, T, H, K):
    """Token row lists built by LDS appends and put back in row order (up to
    128 rows per token, 8800 rows in all at 1100 x 8), and tokens with more
    rows than a list holds (about 150 and 300 rows), which are collected in
    row order by ballots instead; rows of exactly two 512-column groups and
    of two groups plus a ragged 16-column one."""
    r = rng(T + H)
    tok = np.sort(r.integers(0, T, T * K)).astype(np.int64)
    r.shuffle(tok)
    p = from_f32(normal(r, (T * K, H)), dtype)
    w = from_f32(np.abs(normal(r, (T * K,))), dtype)
    got = ops.moe_scatter_sum(p, w, torch.from_numpy(tok).cuda(), T)
    ops.check_device_errors()
    assert_equal(got, oracle.moe_scatter_sum(to_oracle(p), to_oracle(w), tok, T), "moe_scatter_sum")


def test_moe_scatter_sum_batched(ops, oracle):
    r = rng(5)
    B, N, T, H = 2, 30, 7, 64
    tok = r.integers(0, T, (B, N)).astype(np.int32)
    p = from_f32(normal(r, (B, N, H)), torch.bfloat16)
    w = from_f32(normal(r, (B, N)), torch.bfloat16)
    got = ops.moe_scatter_sum(p, w, torch.from_numpy(tok).cuda(), T)
    assert_equal(got, oracle.moe_scatter_sum(to_oracle(p), to_oracle(w), tok, T), "batched combine")


def test_moe_scatter_sum_bad_token_sets_device_error(ops):
    from sandyrt_amd._lib import SandyError
    p = torch.zeros(3, 8, device="cuda")
    ops.moe_scatter_sum(p, torch.ones(3, device="cuda"), torch.tensor([0, 1, 5], device="cuda"), 2)
    with pytest.raises(SandyError, match="moe_scatter_sum token id out of range"):
        ops.check_device_errors()


# ------------------------------------------------------------------ the whole block
def test_moe_block_permute_unpermute_identity(ops, oracle):
    """gather -> scatter_sum with unit weights returns K * x (fp32: exact)."""
    r = rng(77)
    T, H, E, K = 64, 128, 16, 4
    ids = np.stack([r.permutation(E)[:K] for _ in range(T)])
    x = from_f32(np.round(normal(r, (T, H)) * 8) / 8, torch.float32)
    px, pw, tok, off = ops.moe_gather(x, torch.from_numpy(ids).cuda(), torch.ones(T, K, device="cuda"), E)
    y = ops.moe_scatter_sum(px, pw, tok, T)
    assert torch.equal(y, x * K)
