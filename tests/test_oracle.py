"""Pins the CPU oracle (oracle/sandy_oracle.c) before anything is checked
against it:

* golden vectors written by the reference's own CPU math (tests/golden),
  compared bit for bit;
* the closed-form known answers of the reference's own unit tests
  (test/engine/EngineTest.cpp, test/engine/CudaDeviceTest.cpp);
* mathematics: brute-force fp64 attention, sort-based top-k, counting-sort
  permute invariants, softmax rows summing to one, RoPE preserving pair norms;
* where the reference build exists in this container, seeded fuzz against it.
"""
import glob
import math
import os

import numpy as np
import pytest

from oracle import oracle as O
from tests.golden.make_golden import load as load_golden

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


def bits_equal(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    assert a.shape == b.shape and a.dtype == b.dtype
    if a.dtype == np.float32:
        # NaN-aware, sign-aware exact comparison
        return np.array_equal(a.view(np.uint32), b.view(np.uint32))
    return np.array_equal(a, b)


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[:-4] for p in GOLDEN])
def test_oracle_matches_reference_golden(oracle, path):
    fn, kw, outs = load_golden(path)
    got = getattr(oracle, fn)(**kw)
    got = got if isinstance(got, tuple) else (got,)
    assert len(got) == len(outs)
    for g, e in zip(got, outs):
        assert bits_equal(g, e), f"{fn}: oracle differs from the reference CPU math"


def test_golden_set_is_present():
    assert len(GOLDEN) >= 30


# ---------------------------------------------------------------- bf16 (EngineTest.cpp:819-878)
def test_bf16_rne():
    assert O.f32_to_bf16(np.array([1.0], np.float32))[0] == 0x3F80
    third = O.bf16_to_f32(O.f32_to_bf16(np.array([1 / 3], np.float32)))[0]
    assert abs(third - 1 / 3) < 0.002
    # ties to even: 1 + 2^-8 lies halfway between two bf16 values
    halfway = np.array([np.float32(1.0 + 2.0 ** -8), np.float32(1.0 + 3 * 2.0 ** -8)], np.float32)
    assert list(O.f32_to_bf16(halfway)) == [0x3F80, 0x3F82]


def test_bf16_elementwise_known_answers(oracle):
    out = oracle.binary("add", O.f32_to_bf16(np.array([1, 2, 3], np.float32)),
                        O.f32_to_bf16(np.array([10, 20, 30], np.float32)))
    assert list(O.bf16_to_f32(out)) == [11.0, 22.0, 33.0]


# ---------------------------------------------------------------- softmax (EngineTest.cpp:1289-1352)
def test_softmax_known_answers(oracle):
    x = np.array([[1, 1], [1, 2], [-np.inf, -np.inf]], np.float32)
    y = oracle.softmax(x)
    inv = 1.0 / (1.0 + math.exp(1.0))
    np.testing.assert_allclose(y[0], [0.5, 0.5], atol=1e-6)
    np.testing.assert_allclose(y[1], [inv, 1 - inv], atol=1e-6)
    assert list(y[2]) == [0.0, 0.0]
    x = np.array([[[1, 10], [1, 20], [1, 30]]], np.float32)
    y = oracle.softmax(x, axis=1)
    e0, e1 = math.exp(-20), math.exp(-10)
    s = e0 + e1 + 1
    np.testing.assert_allclose(y[0, :, 0], [1 / 3] * 3, atol=1e-6)
    np.testing.assert_allclose(y[0, :, 1], [e0 / s, e1 / s, 1 / s], atol=1e-6)


def test_softmax_rows_sum_to_one(oracle):
    x = np.random.default_rng(0).standard_normal((16, 128)).astype(np.float32) * 5
    np.testing.assert_allclose(oracle.softmax(x).sum(-1), 1.0, atol=1e-5)


# ---------------------------------------------------------------- RoPE (EngineTest.cpp:1430-1537)
def test_rope_known_answers(oracle):
    v = np.zeros((2, 2, 3, 4), np.float32).reshape(-1, 4)
    v[0] = [1, 2, 3, 4]
    v[1] = [1, 0, 0, 1]
    v[2] = [0, 1, 1, 0]
    v[7] = [2, 0, 0, 2]
    y = oracle.rope(v.reshape(2, 2, 3, 4), 10000.0).reshape(-1)
    c, s = math.cos, math.sin
    np.testing.assert_array_equal(y[0:4], [1, 2, 3, 4])
    np.testing.assert_allclose(y[4:8], [c(1), s(1), -s(0.01), c(0.01)], atol=1e-6)
    np.testing.assert_allclose(y[8:12], [-s(2), c(2), c(0.02), s(0.02)], atol=1e-6)
    np.testing.assert_allclose(y[28:32], [2 * c(1), 2 * s(1), -2 * s(0.01), 2 * c(0.01)], atol=1e-6)
    # partial rotary dim copies the tail
    y = oracle.rope(np.array([[[1, 2, 3, 4], [1, 0, 5, 6]]], np.float32), 10000.0, rotary_dim=2).reshape(-1)
    np.testing.assert_allclose(y, [1, 2, 3, 4, c(1), s(1), 5, 6], atol=1e-6)
    # runtime position ids (numel 1 = offset)
    y = oracle.rope(np.array([[[1, 0, 0, 1]]], np.float32), 10000.0,
                    position_ids=np.array([3], np.int64)).reshape(-1)
    np.testing.assert_allclose(y, [c(3), s(3), -s(0.03), c(0.03)], atol=1e-6)


def test_rope_split_half_closed_form(oracle):
    # CudaDeviceTest.cpp:3403-3460 -- split-half pairs (i, i + d/2)
    x = np.zeros((1, 2, 4), np.float32)
    x[0, 1] = [1, 0, 0, 1]
    y = oracle.rope(x, 10000.0, split_half=True).reshape(-1)
    # pair 0: (1, 0) at angle 1; pair 1: (0, 1) at angle 1/100
    np.testing.assert_allclose(y[4:], [math.cos(1), -math.sin(0.01), math.sin(1), math.cos(0.01)], atol=1e-6)


def test_rope_preserves_pair_norms(oracle):
    x = np.random.default_rng(1).standard_normal((3, 64, 64)).astype(np.float32)
    y = oracle.rope(x, 10000.0, split_half=True)
    nx = x[..., :32] ** 2 + x[..., 32:] ** 2
    ny = y[..., :32] ** 2 + y[..., 32:] ** 2
    np.testing.assert_allclose(ny, nx, rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------- norms (EngineTest.cpp:1538-1643)
def test_rms_norm_known_answers(oracle):
    eps = 1e-6
    x = np.array([[1, 2, 2], [0, 3, 4]], np.float32)
    w = np.array([1, 10, -1], np.float32)
    y = oracle.rms_norm(x, w, eps)
    r0 = 1 / math.sqrt(3 + eps)
    r1 = 1 / math.sqrt(25 / 3 + eps)
    np.testing.assert_allclose(y, [[r0, 20 * r0, -2 * r0], [0, 30 * r1, -4 * r1]], atol=1e-5)
    y = oracle.rms_norm(x, None, eps)
    np.testing.assert_allclose(y, [[r0, 2 * r0, 2 * r0], [0, 3 * r1, 4 * r1]], atol=1e-5)
    # CudaDeviceTest.cpp:3573-3643
    x = np.array([[1, 2, 3, 4], [2, 0, -2, 4]], np.float32)
    w = np.array([1, 0.5, 2, -1], np.float32)
    i0 = 1 / math.sqrt(30 / 4 + 1e-6)
    i1 = 1 / math.sqrt(24 / 4 + 1e-6)
    np.testing.assert_allclose(oracle.rms_norm(x, w, 1e-6),
                               [[i0, i0, 6 * i0, -4 * i0], [2 * i1, 0, -4 * i1, -4 * i1]], atol=1e-5)


def test_layer_norm_known_answers(oracle):
    x = np.array([[1, 2], [3, 5], [10, 14], [-2, 2]], np.float32)
    w = np.array([2, -1], np.float32)
    b = np.array([0.5, 10], np.float32)
    y = oracle.layer_norm(x, w, b, 1e-5)
    for r in range(4):
        a, c = x[r]
        m = (a + c) / 2
        var = ((a - m) ** 2 + (c - m) ** 2) / 2
        inv = 1 / math.sqrt(var + 1e-5)
        np.testing.assert_allclose(y[r], [(a - m) * inv * 2 + 0.5, (c - m) * inv * -1 + 10], atol=1e-5)


# ---------------------------------------------------------------- attention vs brute force fp64
def naive_attention(q, k, v, pos, window, scale):
    b, h, tq, d = q.shape
    hkv, tk = k.shape[1], k.shape[2]
    if scale <= 0:
        scale = 1 / math.sqrt(d)
    out = np.zeros(q.shape, np.float64)
    for bi in range(b):
        for hi in range(h):
            kh = hi // (h // hkv)
            for qi in range(tq):
                qp = (pos[bi] if pos is not None else 0) + qi
                lo = max(0, qp + 1 - window) if window > 0 else 0
                keys = [j for j in range(tk) if lo <= j <= qp]
                if not keys:
                    continue
                s = np.array([q[bi, hi, qi].astype(np.float64) @ k[bi, kh, j] * scale for j in keys])
                p = np.exp(s - s.max())
                p /= p.sum()
                out[bi, hi, qi] = p @ v[bi, kh, keys].astype(np.float64)
    return out


@pytest.mark.parametrize("seed", range(6))
def test_attention_matches_fp64_brute_force(oracle, seed):
    rng = np.random.default_rng(0x5A17D00D + seed)
    b, hkv, g = 2, 2, [1, 2, 4][seed % 3]
    d, tk, tq = [16, 32, 64][seed % 3], int(rng.integers(1, 50)), 1 if seed % 2 == 0 else 3
    q = rng.uniform(-0.35, 0.35, (b, hkv * g, tq, d)).astype(np.float32)
    k = rng.uniform(-0.35, 0.35, (b, hkv, tk, d)).astype(np.float32)
    v = rng.uniform(-0.75, 0.75, (b, hkv, tk, d)).astype(np.float32)
    pos = rng.integers(0, tk + tq + 4, b).astype(np.int64)
    window = int(rng.integers(0, tk + 4)) if seed >= 3 else 0
    got = oracle.attention(q, k, v, pos, window, 0.1)
    np.testing.assert_allclose(got, naive_attention(q, k, v, pos, window, 0.1), atol=2e-6)


# ---------------------------------------------------------------- top-k = sort comparator
def test_topk_equals_sort_comparator(oracle):
    rng = np.random.default_rng(7)
    x = (np.round(rng.standard_normal((20, 128)) * 3) / 3).astype(np.float32)  # ties
    vals, idx = oracle.topk(x, 8)
    for r in range(20):
        order = sorted(range(128), key=lambda i: (-x[r, i], i))[:8]
        assert list(idx[r]) == order
        np.testing.assert_array_equal(vals[r], x[r, order])


# ---------------------------------------------------------------- MoE chain invariants
def test_moe_permute_is_stable_counting_sort(oracle):
    rng = np.random.default_rng(3)
    T, H, E, K = 40, 8, 16, 4
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int64)
    w = rng.random((T, K)).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    px, pw, tok, off = oracle.moe_gather(x, ids, w, E)
    # offsets: exclusive prefix sum of expert counts, off[E] = T*K
    counts = np.bincount(ids.reshape(-1), minlength=E)
    np.testing.assert_array_equal(off, np.concatenate([[0], np.cumsum(counts)]))
    # rows: stable order (expert, token, slot)
    routes = sorted(((ids[t, s], t, s) for t in range(T) for s in range(K)))
    for row, (e, t, s) in enumerate(routes):
        assert tok[row] == t and pw[row] == w[t, s]
        np.testing.assert_array_equal(px[row], x[t])
    # unpermute(permute(x)) with weights 1 is K * x
    y = oracle.moe_scatter_sum(px, np.ones_like(pw), tok, T)
    np.testing.assert_allclose(y, K * x, rtol=1e-6)


def test_moe_matmul_matches_segmented_gemm(oracle):
    rng = np.random.default_rng(4)
    E, K, M = 5, 24, 12
    off = np.array([0, 2, 2, 7, 9, 15], np.int64)
    x = rng.standard_normal((15, K)).astype(np.float32)
    w = rng.standard_normal((E, M, K)).astype(np.float32)
    y = oracle.moe_matmul(x, off, w, transpose_rhs=True)
    for e in range(E):
        np.testing.assert_allclose(y[off[e]:off[e + 1]], x[off[e]:off[e + 1]] @ w[e].T, rtol=1e-5, atol=1e-5)


# matmul known answers: the reference's own device tests
# (test/engine/CudaDeviceTest.cpp:1145-1198, 1331-1384, 1386-1471)
MATMUL_LHS = np.arange(1, 7, dtype=np.float32).reshape(2, 3)
GROUPED_LHS = np.array([1, 0, 0, 0, 1, 0, 0, 0, 1, 1, 1, 0, 1, 2, 0, 0, 1, 1, 2, 0, 1, 1, 0, 1],
                       np.float32).reshape(1, 4, 2, 3)
GROUPED_RHS = np.array([10, 100, 20, 200, 30, 300, 1, 10, 2, 20, 3, 30], np.float32).reshape(1, 2, 3, 2)
GROUPED_OUT = [10, 100, 20, 200, 30, 300, 30, 300, 5, 50, 5, 50, 5, 50, 4, 40]


def test_matmul_known_answers(oracle):
    rhs = np.arange(7, 13, dtype=np.float32)
    assert oracle.matmul(MATMUL_LHS, rhs.reshape(3, 2)).ravel().tolist() == [58, 64, 139, 154]
    assert oracle.matmul(MATMUL_LHS, rhs.reshape(2, 3), transpose_rhs=True).ravel().tolist() == [50, 68, 122, 167]
    # lhs heads 0-1 use rhs head 0, heads 2-3 rhs head 1 (grouped batch broadcast)
    assert oracle.matmul(GROUPED_LHS, GROUPED_RHS).ravel().tolist() == GROUPED_OUT


@pytest.mark.parametrize("tl,tr", [(False, False), (True, False), (False, True), (True, True)])
def test_matmul_matches_float64_with_broadcast(oracle, tl, tr):
    rng = np.random.default_rng(7)
    a = rng.standard_normal((3, 1, 4, 24, 10)).astype(np.float32)  # [.., k, m] when transposed
    b = rng.standard_normal((2, 1, 24, 6)).astype(np.float32)
    lhs = a if tl else np.swapaxes(a, -1, -2).copy()
    rhs = np.swapaxes(b, -1, -2).copy() if tr else b
    got = oracle.matmul(lhs, rhs, transpose_lhs=tl, transpose_rhs=tr)
    want = np.swapaxes(a, -1, -2).astype(np.float64) @ b.astype(np.float64)  # [3, 2, 4, 10, 6]
    assert got.shape == (3, 2, 4, 10, 6)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_linear_is_bias_plus_matmul(oracle):
    rng = np.random.default_rng(8)
    x = rng.standard_normal((5, 40)).astype(np.float32)
    w = rng.standard_normal((7, 40)).astype(np.float32)
    b = rng.standard_normal(7).astype(np.float32)
    np.testing.assert_allclose(oracle.linear(x, w, b), x.astype(np.float64) @ w.T.astype(np.float64) + b,
                               rtol=1e-5, atol=1e-5)


def test_elementwise_dag_silu_gate(oracle):
    """silu(g) * u as lowered by BuiltinLowering.cpp:142-158: (0.5 g)(1 + tanh(0.5 g))"""
    rng = np.random.default_rng(5)
    g = rng.standard_normal(257).astype(np.float32)
    u = rng.standard_normal(257).astype(np.float32)
    nodes = O.make_nodes([
        (0, O.LOAD, 0, 0, []), (1, O.CONST, 0, 0.5, []), (2, O.MUL, 0, 0, [1, 0]),
        (3, O.TANH, 0, 0, [2]), (4, O.CONST, 0, 1.0, []), (5, O.ADD, 0, 0, [4, 3]),
        (6, O.MUL, 0, 0, [2, 5]), (7, O.LOAD, 1, 0, []), (8, O.MUL, 0, 0, [6, 7]),
    ])
    y = oracle.elementwise_dag(nodes, 8, [g, u], [0, 0], (257,), np.float32)
    gd = g.astype(np.float64)
    np.testing.assert_allclose(y, gd / (1 + np.exp(-gd)) * u, rtol=1e-5, atol=1e-6)


def test_paged_to_dense_roundtrip(oracle):
    rng = np.random.default_rng(6)
    prefix, page, inner, grow = 3, 4, 5, 10
    dense = rng.standard_normal((prefix, grow, inner)).astype(np.float32)
    ids = np.array([7, 2, 5], np.int32)
    pool = np.zeros((8, prefix, page, inner), np.float32)
    for g in range(grow):
        pool[ids[g // page], :, g % page] = dense[:, g]
    np.testing.assert_array_equal(oracle.paged_to_dense(pool, ids, prefix, grow, page, inner), dense)


def test_oracle_errors_match_reference_wording(oracle):
    with pytest.raises(O.OracleError, match="moe_gather topk expert id out of range"):
        oracle.moe_gather(np.zeros((2, 4), np.float32), np.array([[0], [9]], np.int64),
                          np.ones((2, 1), np.float32), 4)
    with pytest.raises(O.OracleError, match="rope position_ids must be non-negative"):
        oracle.rope(np.zeros((1, 1, 4), np.float32), 1e4, position_ids=np.array([-1], np.int64))
    with pytest.raises(O.OracleError, match="attention heads must be divisible by kv_heads"):
        oracle.attention(np.zeros((1, 3, 1, 4), np.float32), np.zeros((1, 2, 2, 4), np.float32),
                         np.zeros((1, 2, 2, 4), np.float32))


# ---------------------------------------------------------------- fuzz against the reference build
@pytest.mark.parametrize("seed", range(4))
def test_oracle_fuzz_against_reference_build(oracle, ref, seed):
    rng = np.random.default_rng(100 + seed)
    bf = lambda a: O.f32_to_bf16(a.astype(np.float32))  # noqa: E731
    for dt in (np.float32, np.uint16):
        cv = (lambda a: a.astype(np.float32)) if dt == np.float32 else bf
        x = cv(rng.standard_normal((7, 200)))
        w = cv(rng.standard_normal(200))
        b = cv(rng.standard_normal(200))
        assert bits_equal(oracle.rms_norm(x, w, 1e-5), ref.rms_norm(x, w, 1e-5))
        assert bits_equal(oracle.layer_norm(x, w, b, 1e-5), ref.layer_norm(x, w, b, 1e-5))
        assert bits_equal(oracle.softmax(x), ref.softmax(x))
        r = cv(rng.standard_normal((2, 4, 33, 64)))
        assert bits_equal(oracle.rope(r, 1e4, split_half=True), ref.rope(r, 1e4, split_half=True))
        assert bits_equal(oracle.rope(r, 1e4, rotary_dim=48), ref.rope(r, 1e4, rotary_dim=48))
        q = cv(rng.standard_normal((3, 8, 1, 64)) * 0.5)
        k = cv(rng.standard_normal((3, 2, 70, 64)) * 0.5)
        v = cv(rng.standard_normal((3, 2, 70, 64)))
        pos = rng.integers(0, 75, 3).astype(np.int64)
        assert bits_equal(oracle.attention(q, k, v, pos, 0, -1.0), ref.attention(q, k, v, pos, 0, -1.0))
        assert bits_equal(oracle.attention(q, k, v, pos, 9, 0.2), ref.attention(q, k, v, pos, 9, 0.2))
        t = cv(np.round(rng.standard_normal((9, 128)) * 4) / 4)
        for a, e in zip(oracle.topk(t, 8), ref.topk(t, 8)):
            assert bits_equal(a, e)
        lm = cv(rng.standard_normal((2, 4, 5, 40)))
        rm = cv(rng.standard_normal((2, 1, 40, 7)))
        assert bits_equal(oracle.matmul(lm, rm), ref.matmul(lm, rm))
        assert bits_equal(oracle.matmul(lm, np.swapaxes(rm, -1, -2).copy(), transpose_rhs=True),
                          ref.matmul(lm, np.swapaxes(rm, -1, -2).copy(), transpose_rhs=True))


@pytest.mark.skipif(not os.path.exists(O.REF_PATH), reason="reference CPU build (oracle/_ref) not built here")
def test_gpt2_chain_matches_reference_build_bit_for_bit():
    """The GPT-2 op chain (oracle/gpt2.py) gives the same logits and greedy
    tokens on the reference's own src/core build as on the restatement."""
    from oracle.gpt2 import GPT2Oracle
    from sandyrt_amd.gpt2 import GPT2Config, prompt_ids, random_weights
    cfg = GPT2Config(layers=2, hidden=128, heads=2, ffn=512, vocab=700, positions=32)
    w = random_weights(cfg, seed=11)
    p = prompt_ids(cfg, 6, seed=11)
    a, b = GPT2Oracle(O.Oracle(), cfg, w), GPT2Oracle(O.Oracle(reference=True), cfg, w)
    ids = p
    for _ in range(3):
        la, lb = a.forward(ids), b.forward(ids)
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
        ids = [int(np.argmax(la))]
