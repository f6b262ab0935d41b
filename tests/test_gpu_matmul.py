"""GPU parity of dense matmul and linear against the oracle
(src/core/TensorCalc.cpp matmul 804-919, linear 722-773; validation of
launch_cuda_matmul, src/device/cuda/CudaMatMulKernels.cu:78-141).

f32 and every layout other than bf16 x [n, k] weights keep the reference's k
order per output: compared bit-exactly.  bf16 with transposed rhs runs on
MFMA with fp32 accumulation in another order: compared at the bf16
tolerance (2e-2)."""
import os

import numpy as np
import pytest
import torch

from tests.helpers import assert_close, assert_equal, from_f32, normal, rng, to_oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from sandyrt_amd import ops
    return ops


class env:
    """Temporarily set SANDY_* tuning variables (read on every call)."""

    def __init__(self, **kw):
        self.kw = {k: str(v) for k, v in kw.items()}

    def __enter__(self):
        self.old = {k: os.environ.get(k) for k in self.kw}
        os.environ.update(self.kw)

    def __exit__(self, *a):
        for k, v in self.old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def f32(a):
    return torch.tensor(a, dtype=torch.float32, device="cuda")


# ---------------------------------------------------------------- known answers
def test_matmul_reference_known_answers(ops):
    """The reference's device tests (test/engine/CudaDeviceTest.cpp:1145-1198,
    1200-1253, 1331-1384, 1386-1471)."""
    lhs = f32([[1, 2, 3], [4, 5, 6]])
    assert ops.matmul(lhs, f32([[7, 8], [9, 10], [11, 12]])).cpu().tolist() == [[58, 64], [139, 154]]
    assert ops.matmul(lhs, f32([[7, 8, 9], [10, 11, 12]]), transpose_rhs=True).cpu().tolist() == [[50, 68], [122, 167]]
    # a [1, 2] view at storage offset 4 of a [1, 3, 2] buffer
    base = f32([1, 2, 3, 4, 5, 6])
    view = base[4:6].view(1, 2)
    assert view.storage_offset() == 4
    assert ops.matmul(view, f32([[1, 0], [0, 1]])).cpu().tolist() == [[5, 6]]
    gl = f32([1, 0, 0, 0, 1, 0, 0, 0, 1, 1, 1, 0, 1, 2, 0, 0, 1, 1, 2, 0, 1, 1, 0, 1]).view(1, 4, 2, 3)
    gr = f32([10, 100, 20, 200, 30, 300, 1, 10, 2, 20, 3, 30]).view(1, 2, 3, 2)
    assert ops.matmul(gl, gr).cpu().flatten().tolist() == [10, 100, 20, 200, 30, 300, 30, 300, 5, 50, 5, 50, 5, 50, 4, 40]


def test_matmul_validation_errors(ops):
    from sandyrt_amd._lib import SandyError
    a = torch.zeros(2, 3, device="cuda")
    with pytest.raises(SandyError, match="contracting dimension mismatch"):
        ops.matmul(a, torch.zeros(4, 2, device="cuda"), out=torch.zeros(2, 2, device="cuda"))
    with pytest.raises(SandyError, match="operands must have same dtype"):
        ops.matmul(a, torch.zeros(3, 2, device="cuda", dtype=torch.bfloat16), out=torch.zeros(2, 2, device="cuda"))
    with pytest.raises(SandyError, match="output shape mismatch"):
        ops.matmul(a, torch.zeros(3, 2, device="cuda"), out=torch.zeros(2, 3, device="cuda"))
    with pytest.raises(SandyError, match="contiguous"):
        ops.matmul(torch.zeros(3, 2, device="cuda").t(), torch.zeros(3, 2, device="cuda"),
                   out=torch.zeros(2, 2, device="cuda"))
    with pytest.raises(SandyError, match="unsupported dtype"):
        ops.matmul(torch.zeros(2, 3, device="cuda", dtype=torch.int32), torch.zeros(3, 2, device="cuda", dtype=torch.int32),
                   out=torch.zeros(2, 2, device="cuda", dtype=torch.int32))
    with pytest.raises(SandyError, match="rank >= 2"):
        ops.matmul(torch.zeros(3, device="cuda"), torch.zeros(3, 2, device="cuda"), out=torch.zeros(2, device="cuda"))
    with pytest.raises(SandyError, match="linear bias shape mismatch"):
        ops.linear(a, torch.zeros(4, 3, device="cuda"), torch.zeros(5, device="cuda"))


# ---------------------------------------------------------------- exact-order paths
# bf16 with a transposed rhs and a plain lhs runs on MFMA: covered by the tolerance tests below
EXACT_LAYOUTS = [(dt, tl, tr) for dt in (torch.float32, torch.bfloat16)
                 for tl, tr in ((False, False), (True, False), (False, True), (True, True))
                 if not (dt == torch.bfloat16 and tr and not tl)]


@pytest.mark.parametrize("dtype,tl,tr", EXACT_LAYOUTS)
@pytest.mark.parametrize("lshape,rshape", [((70, 33), (33, 90)), ((2, 4, 17, 40), (2, 1, 40, 9)),
                                           ((3, 1, 5, 64), (2, 64, 130)), ((1, 8), (8, 1))])
def test_matmul_exact_order_bit_exact(ops, oracle, dtype, tl, tr, lshape, rshape):
    """f32 everywhere and bf16 outside the MFMA layout: same k order as the
    reference, so results are bit-identical (batch broadcast and grouped heads
    included)."""
    r = rng(sum(lshape) + sum(rshape) + 2 * tl + tr)
    lhs = normal(r, lshape)
    rhs = normal(r, rshape)
    if tl:
        lhs = np.swapaxes(lhs, -1, -2).copy()
    if tr:
        rhs = np.swapaxes(rhs, -1, -2).copy()
    L, R = from_f32(lhs, dtype), from_f32(rhs, dtype)
    got = ops.matmul(L, R, transpose_lhs=tl, transpose_rhs=tr)
    want = oracle.matmul(to_oracle(L), to_oracle(R), transpose_lhs=tl, transpose_rhs=tr)
    assert_equal(got, want, "matmul")


def test_matmul_bf16_simt_fallback_for_unaligned_k(ops, oracle):
    """bf16 with [n, k] weights but K not a multiple of 32 takes the exact-order
    kernel: bit-exact."""
    r = rng(5)
    L = from_f32(normal(r, (9, 40)), torch.bfloat16)
    R = from_f32(normal(r, (33, 40)), torch.bfloat16)
    assert_equal(ops.matmul(L, R, transpose_rhs=True), oracle.matmul(to_oracle(L), to_oracle(R), transpose_rhs=True),
                 "matmul bf16 K=40")


def test_matmul_empty(ops):
    out = ops.matmul(torch.zeros(0, 64, device="cuda", dtype=torch.bfloat16),
                     torch.zeros(32, 64, device="cuda", dtype=torch.bfloat16), transpose_rhs=True)
    assert out.shape == (0, 32)
    out = ops.matmul(torch.zeros(3, 0, device="cuda"), torch.zeros(0, 4, device="cuda"))
    assert out.cpu().tolist() == [[0.0] * 4] * 3


# ---------------------------------------------------------------- MFMA path
# (M, N, K): decode rows against projection-like weights, ragged N, odd k-steps
# (24, 8192, 2048): 17-32 rows of a wide projection, one 32-row tile with the non-temporal weight stream;
# (1, 4096, 2048): one row tile, non-temporal (the default policy at 32 rows: (32, 2048, 512) and the
# RMSNorm-prologue tests, which compare bit for bit with the plain GEMM)
MFMA_SHAPES = [(1, 256, 64), (7, 200, 96), (16, 512, 2048), (32, 2048, 512), (33, 300, 160), (64, 1000, 256),
               (3, 700, 2560), (40, 96, 5632), (100, 520, 224), (256, 640, 1024), (130, 300, 96), (24, 8192, 2048),
               (1, 4096, 2048)]


@pytest.mark.parametrize("m,n,k", MFMA_SHAPES)
def test_matmul_bf16_mfma_matches_oracle(ops, oracle, m, n, k):
    r = rng(m * 7 + n + k)
    L = from_f32(normal(r, (m, k)), torch.bfloat16)
    W = from_f32(normal(r, (n, k), 0.05), torch.bfloat16)
    got = ops.matmul(L, W, transpose_rhs=True)
    want = oracle.matmul(to_oracle(L), to_oracle(W), transpose_rhs=True)
    assert_close(got, want, torch.bfloat16, f"matmul {m}x{n}x{k}")


@pytest.mark.parametrize("variant", [0, 1, 3, 4, 5, 6])
@pytest.mark.parametrize("cps", [2, 5, 12])
def test_matmul_bf16_wave_kernel_tiles_and_splits(ops, oracle, variant, cps):
    """The decode kernel (four independent waves per workgroup splitting K)
    for every tile and a short, odd and long run per wave: 1248 = 19.5
    chunks of 64 gives split K, idle waves, partial runs and a half chunk."""
    r = rng(variant * 100 + cps)
    m, n, k = 45, 600, 1248
    L = from_f32(normal(r, (m, k)), torch.bfloat16)
    W = from_f32(normal(r, (n, k), 0.05), torch.bfloat16)
    want = oracle.matmul(to_oracle(L), to_oracle(W), transpose_rhs=True)
    with env(SANDY_GEMM_WAVES=1, SANDY_GEMM_TILE=variant, SANDY_GEMM_CPS=cps):
        got = ops.matmul(L, W, transpose_rhs=True)
        again = ops.matmul(L, W, transpose_rhs=True)
    assert_close(got, want, torch.bfloat16, f"waves variant {variant} cps {cps}")
    assert torch.equal(got, again), "split-K result is not deterministic"


def test_matmul_bf16_split_counters_rearm(ops, oracle):
    """Back-to-back split-K launches of different shapes: each launch leaves its
    arrival counters at zero for the next."""
    r = rng(11)
    cases = [(32, 2048, 2048), (8, 700, 512), (32, 2048, 2048), (1, 64, 4096)]
    outs = []
    for m, n, k in cases:
        L = from_f32(normal(r, (m, k)), torch.bfloat16)
        W = from_f32(normal(r, (n, k), 0.05), torch.bfloat16)
        outs.append((ops.matmul(L, W, transpose_rhs=True), L, W))
    for got, L, W in outs:
        assert_close(got, oracle.matmul(to_oracle(L), to_oracle(W), transpose_rhs=True), torch.bfloat16, "rearm")


def test_matmul_bf16_mfma_batched_grouped_heads(ops, oracle):
    """Batched [n, k] rhs with grouped-head broadcast on the MFMA kernel."""
    r = rng(12)
    L = from_f32(normal(r, (2, 8, 5, 64)), torch.bfloat16)
    R = from_f32(normal(r, (2, 2, 48, 64)), torch.bfloat16)
    got = ops.matmul(L, R, transpose_rhs=True)
    want = oracle.matmul(to_oracle(L), to_oracle(R), transpose_rhs=True)
    assert_close(got, want, torch.bfloat16, "grouped heads")


# ---------------------------------------------------------------- linear
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("xshape,out_f", [((5, 768), 2304), ((2, 3, 64), 96), ((1, 40), 7), ((16,), 8)])
def test_linear_matches_oracle(ops, oracle, dtype, xshape, out_f):
    r = rng(len(xshape) + out_f)
    in_f = xshape[-1]
    x = from_f32(normal(r, xshape), dtype)
    w = from_f32(normal(r, (out_f, in_f), 0.02), dtype)
    b = from_f32(normal(r, (out_f,)), dtype)
    got = ops.linear(x, w, b)
    want = oracle.linear(to_oracle(x), to_oracle(w), to_oracle(b))
    if dtype == torch.float32 or in_f % 32:
        assert_equal(got, want, "linear exact order")  # acc starts at bias, k in order
    else:
        assert_close(got, want, dtype, "linear")


@pytest.mark.parametrize("rows,in_f,out_f", [(1, 772, 3000), (2, 768, 50), (3, 4, 130), (8, 1000, 65), (4, 770, 33)])
def test_linear_f32_few_rows_bit_exact(ops, oracle, rows, in_f, out_f):
    """f32 linear of a few rows (the GPT-2 decode shapes): the exact-order
    GEMV (k tails past the 8-float chunks included) and, for k not a multiple
    of 4, the general kernel -- both bit-identical to the CPU."""
    r = rng(rows * 1000 + in_f + out_f)
    x = from_f32(normal(r, (rows, in_f)), torch.float32)
    w = from_f32(normal(r, (out_f, in_f), 0.02), torch.float32)
    b = from_f32(normal(r, (out_f,)), torch.float32)
    assert_equal(ops.linear(x, w, b), oracle.linear(to_oracle(x), to_oracle(w), to_oracle(b)), "linear")
    assert_equal(ops.matmul(x, w, transpose_rhs=True),
                 oracle.matmul(to_oracle(x), to_oracle(w), transpose_rhs=True), "matmul transposed rhs")


@pytest.mark.parametrize("act", ["silu", "gelu"])
@pytest.mark.parametrize("m,k,ffn", [(1, 2048, 5632), (5, 64, 80), (32, 2048, 5632), (64, 2560, 1024),
                                     (32, 5632, 96), (3, 128, 40)])
def test_matmul_glu_matches_matmul_then_group(ops, act, m, k, ffn):
    """The gated epilogue equals the GEMM (gate and up outputs rounded to
    bf16) followed by the element-wise group, bit for bit; K-split shapes
    (k 5632) and odd row counts included."""
    r = rng(m + k + ffn)
    x = from_f32(normal(r, (m, k)), torch.bfloat16)
    wg = from_f32(normal(r, (ffn, k), 0.05), torch.bfloat16)
    wu = from_f32(normal(r, (ffn, k), 0.05), torch.bfloat16)
    got = ops.matmul_glu(x, ops.interleave_glu_weight(wg, wu), act)
    gate = ops.matmul(x, wg, transpose_rhs=True)
    up = ops.matmul(x, wu, transpose_rhs=True)
    nodes, res = ops.silu_mul_nodes() if act == "silu" else ops.gelu_mul_nodes()
    want = ops.elementwise(nodes, res, [gate, up])
    assert torch.equal(got, want)


def test_matmul_glu_rejects_unsupported(ops):
    from sandyrt_amd._lib import SandyError
    x = torch.zeros(2, 40, dtype=torch.bfloat16, device="cuda")  # k not a multiple of 32
    w = torch.zeros(8, 40, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(SandyError, match="gated matmul needs bf16 operands"):
        ops.matmul_glu(x, w)
    with pytest.raises(SandyError, match="with gate and up rows interleaved"):
        ops.matmul_glu(torch.zeros(2, 64, dtype=torch.bfloat16, device="cuda"),
                       torch.zeros(7, 64, dtype=torch.bfloat16, device="cuda"))


# ---------------------------------------------------------------- fused decode GEMMs
def _row_sumsq_groups(t):
    """Exact float64 sums of squares per (row, 16-column group) of a bf16 matrix."""
    v = t.float().double().cpu().numpy()
    m, n = v.shape
    g = (n + 15) // 16
    pad = np.zeros((m, g * 16))
    pad[:, :n] = v * v
    return pad.reshape(m, g, 16).sum(axis=2)


@pytest.mark.parametrize("m,k,n", [(1, 2048, 2048), (5, 2048, 2048), (32, 2048, 2048), (32, 5632, 2048),
                                   (33, 256, 200), (64, 1024, 2560), (3, 96, 40)])
def test_matmul_residual_matches_matmul_then_add(ops, m, k, n):
    """Residual epilogue: bit-identical to the GEMM's stored output followed by
    the residual add (K-split shapes at k 5632, odd widths and row counts);
    the row statistics equal the exact float64 sums of squares of the sum."""
    r = rng(m * 7 + k + n)
    x = from_f32(normal(r, (m, k)), torch.bfloat16)
    w = from_f32(normal(r, (n, k), 0.05), torch.bfloat16)
    res = from_f32(normal(r, (m, n)), torch.bfloat16)
    stats = ops.row_stats_buffer(m, n)
    got = ops.matmul_residual(x, w, res, stats)
    prod = ops.matmul(x, w, transpose_rhs=True)
    nodes, rid = ops.residual_add_nodes()
    want = ops.elementwise(nodes, rid, [prod, res])
    assert torch.equal(got, want)
    np.testing.assert_array_equal(stats.cpu().numpy(), _row_sumsq_groups(want))
    # in place: out is the residual
    res2 = res.clone()
    ops.matmul_residual(x, w, res2, None, out=res2)
    assert torch.equal(res2, want)


@pytest.mark.parametrize("act", [None, "silu", "gelu"])
@pytest.mark.parametrize("m,k,n", [(1, 2048, 2560), (32, 2048, 2560), (32, 2048, 11264), (16, 2048, 32000),
                                   (32, 2048, 32000), (48, 2560, 512), (64, 512, 96), (7, 160, 64)])
def test_matmul_rms_matches_norm_then_matmul(ops, act, m, k, n):
    """RMSNorm prologue from row statistics: bit-identical to sandy_hip_norm
    followed by the plain or gated GEMM (tile shapes of every decode
    projection, the lm-head's 32000 columns, 33..64-row tiles)."""
    if act and n % 2:
        pytest.skip("gated weights have an even row count")
    r = rng(m * 11 + k + n + (0 if act is None else len(act)))
    x = from_f32(normal(r, (m, k)), torch.bfloat16)
    nw = from_f32(1.0 + normal(r, (k,), 0.1), torch.bfloat16)
    w = from_f32(normal(r, (n, k), 0.05), torch.bfloat16)
    stats = torch.from_numpy(_row_sumsq_groups(x)).cuda()
    got = ops.matmul_rms(x, stats, nw, 1e-5, w, act)
    h = ops.rms_norm(x, nw, 1e-5)
    want = ops.matmul(h, w, transpose_rhs=True) if act is None else ops.matmul_glu(h, w, act)
    assert torch.equal(got, want)


def test_fused_chain_matches_unfused_block(ops):
    """o projection + residual -> gate/up with the post-attention norm, as the
    decode step chains them, against add_rms_norm between plain GEMMs."""
    r = rng(77)
    m, d, f = 32, 2048, 5632
    ctx = from_f32(normal(r, (m, d)), torch.bfloat16)
    x = from_f32(normal(r, (m, d)), torch.bfloat16)
    wo = from_f32(normal(r, (d, d), 0.02), torch.bfloat16)
    wgu = ops.interleave_glu_weight(from_f32(normal(r, (f, d), 0.02), torch.bfloat16),
                                    from_f32(normal(r, (f, d), 0.02), torch.bfloat16))
    nw = from_f32(1.0 + normal(r, (d,), 0.02), torch.bfloat16)
    stats = ops.row_stats_buffer(m, d)
    s = ops.matmul_residual(ctx, wo, x, stats)
    act = ops.matmul_rms(s, stats, nw, 1e-5, wgu, "silu")
    o = ops.matmul(ctx, wo, transpose_rhs=True)
    s2, h = ops.add_rms_norm(o, x, nw, 1e-5)
    assert torch.equal(s, s2)
    assert torch.equal(act, ops.matmul_glu(h, wgu, "silu"))


@pytest.mark.parametrize("m", [1, 32])
def test_fused_decode_gemms_match_oracle_chain(ops, oracle, m):
    """The fused decode GEMMs at TinyLlama's widths against the oracle's op
    chain (not against the unfused HIP ops): o projection + residual, then
    RMSNorm -> gate/up -> SiLU-gate, then down projection (K split over
    workgroups) + residual, then RMSNorm -> q/k/v, each stage fed the GPU's
    previous output so the comparison is per op; bf16 tolerance."""
    from tests.test_gpu_groups import oracle_nodes
    r = rng(4100 + m)
    d, f, nq = 2048, 5632, 2560
    ctx = from_f32(normal(r, (m, d)), torch.bfloat16)
    x = from_f32(normal(r, (m, d)), torch.bfloat16)
    wo = from_f32(normal(r, (d, d), 0.02), torch.bfloat16)
    wg = from_f32(normal(r, (f, d), 0.02), torch.bfloat16)
    wu = from_f32(normal(r, (f, d), 0.02), torch.bfloat16)
    wd = from_f32(normal(r, (d, f), 0.02), torch.bfloat16)
    wqkv = from_f32(normal(r, (nq, d), 0.02), torch.bfloat16)
    nw1 = from_f32(1.0 + normal(r, (d,), 0.1), torch.bfloat16)
    nw2 = from_f32(1.0 + normal(r, (d,), 0.1), torch.bfloat16)
    st_b, st_a = ops.row_stats_buffer(m, d), ops.row_stats_buffer(m, d)
    silu, sres = ops.silu_mul_nodes()

    s = ops.matmul_residual(ctx, wo, x, st_b)
    want_s = oracle.binary("add", to_oracle(x), oracle.matmul(to_oracle(ctx), to_oracle(wo), transpose_rhs=True))
    assert_close(s, want_s, torch.bfloat16, "o projection + residual")
    np.testing.assert_array_equal(st_b.cpu().numpy(), _row_sumsq_groups(s))

    act = ops.matmul_rms(s, st_b, nw1, 1e-5, ops.interleave_glu_weight(wg, wu), "silu")
    h = oracle.rms_norm(to_oracle(s), to_oracle(nw1), 1e-5)
    g_, u_ = (oracle.matmul(h, to_oracle(w_), transpose_rhs=True) for w_ in (wg, wu))
    want_act = oracle.elementwise_dag(oracle_nodes(silu), sres, [g_, u_], [0, 0], (m, f), g_.dtype)
    assert_close(act, want_act, torch.bfloat16, "RMSNorm -> gate/up -> SiLU-gate")

    x2 = ops.matmul_residual(act, wd, s, st_a)
    want_x2 = oracle.binary("add", to_oracle(s), oracle.matmul(to_oracle(act), to_oracle(wd), transpose_rhs=True))
    assert_close(x2, want_x2, torch.bfloat16, "down projection + residual")
    np.testing.assert_array_equal(st_a.cpu().numpy(), _row_sumsq_groups(x2))

    qkv = ops.matmul_rms(x2, st_a, nw2, 1e-5, wqkv)
    want_qkv = oracle.matmul(oracle.rms_norm(to_oracle(x2), to_oracle(nw2), 1e-5), to_oracle(wqkv), transpose_rhs=True)
    assert_close(qkv, want_qkv, torch.bfloat16, "RMSNorm -> q/k/v")


def test_fused_gemms_reject_bad_stats(ops):
    from sandyrt_amd._lib import SandyError
    x = torch.zeros(4, 64, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(32, 64, dtype=torch.bfloat16, device="cuda")
    nw = torch.ones(64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(SandyError, match=r"row statistics must be \[m, ceil\(k / 16\)\]"):
        ops.matmul_rms(x, ops.row_stats_buffer(4, 32), nw, 1e-5, w)
    with pytest.raises(SandyError, match=r"row statistics must be \[m, ceil\(n / 16\)\]"):
        ops.matmul_residual(x, w, torch.zeros(4, 32, dtype=torch.bfloat16, device="cuda"), ops.row_stats_buffer(4, 64))
    with pytest.raises(SandyError, match="out must not alias lhs"):
        sq = torch.zeros(4, 64, dtype=torch.bfloat16, device="cuda")
        ops.matmul_residual(sq, torch.zeros(64, 64, dtype=torch.bfloat16, device="cuda"), sq, None, out=sq)


@pytest.mark.parametrize("m,k,n,ln,act,res", [
    (1, 768, 2304, True, None, False),     # GPT-2 ln_1 -> q/k/v
    (1, 768, 768, False, None, True),      # c_proj + residual
    (1, 768, 3072, True, "gelu", False),   # ln_2 -> c_fc -> GELU
    (1, 3072, 768, False, None, True),     # mlp c_proj + residual
    (1, 768, 50257, True, None, False),    # ln_f -> lm-head (no bias)
    (3, 512, 333, True, "gelu", True),     # looped k, several rows, ragged n
    (4, 100, 37, False, None, False),
])
def test_decode_linear_matches_oracle_chain(ops, oracle, m, k, n, ln, act, res):
    """sandy_hip_decode_linear against the reference's unfused fp32 op chain
    (layer_norm, linear, the GELU node chain, add) at the fp32 tolerance."""
    from tests.test_gpu_groups import oracle_nodes
    r = rng(m * 1000 + k + n)
    x = from_f32(normal(r, (m, k)), torch.float32)
    w = from_f32(normal(r, (n, k), 0.02), torch.float32)
    bias = None if n == 50257 else from_f32(normal(r, (n,), 0.02), torch.float32)
    lw = from_f32(1 + normal(r, (k,), 0.1), torch.float32) if ln else None
    lb = from_f32(normal(r, (k,), 0.1), torch.float32) if ln else None
    resid = from_f32(normal(r, (m, n)), torch.float32) if res else None
    got = ops.decode_linear(x, w, bias, lw, lb, 1e-5, act, resid)
    h = oracle.layer_norm(to_oracle(x), to_oracle(lw), to_oracle(lb), 1e-5) if ln else to_oracle(x)
    if bias is None:
        y = oracle.matmul(h, to_oracle(w), transpose_rhs=True)
    else:
        y = oracle.linear(h, to_oracle(w), to_oracle(bias))
    if act == "gelu":
        nodes, out_id = ops.gelu_nodes()
        y = oracle.elementwise_dag(oracle_nodes(nodes), out_id, [y], [0], y.shape, np.float32)
    if res:
        y = oracle.binary("add", to_oracle(resid), y)
    # the dot products sum in another k order than the reference's loop: an
    # output near zero (cancellation) carries the rounding of its large terms,
    # so the bound is 1e-5 of the larger of |want| and the outputs' rms
    assert_close(got, y, torch.float32, f"decode linear {m}x{k}x{n}", floor=1.0)
    again = ops.decode_linear(x, w, bias, lw, lb, 1e-5, act, resid)
    assert torch.equal(got, again), "not deterministic"


def test_decode_linear_rejects(ops):
    from sandyrt_amd._lib import SandyError
    x = torch.zeros(5, 64, device="cuda")
    w = torch.zeros(8, 64, device="cuda")
    with pytest.raises(SandyError, match="1 to 4 rows"):
        ops.decode_linear(x, w)
    with pytest.raises(SandyError, match="both LayerNorm weight and bias"):
        ops.decode_linear(x[:1], w, ln_weight=torch.ones(64, device="cuda"))
    with pytest.raises(SandyError, match="feature mismatch"):
        ops.decode_linear(x[:1], w[:, :32].contiguous())
    sq = torch.zeros(1, 64, device="cuda")
    with pytest.raises(SandyError, match="out must not alias x"):
        ops.decode_linear(sq, torch.zeros(64, 64, device="cuda"), out=sq)
