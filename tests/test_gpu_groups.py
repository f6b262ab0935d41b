"""GPU parity of the fused-group family against the oracle: element-wise
DAGs (hipRTC-generated), RoPE, softmax, sum and embedding gather."""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import assert_close, assert_equal, from_f32, normal, rng, to_oracle

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16]


@pytest.fixture(scope="module")
def ops():
    from sandyrt_amd import ops
    return ops


def oracle_nodes(nodes):
    return O.make_nodes([(n.id, n.op, n.input_index, n.constant, list(n.operands)) for n in nodes])


# ------------------------------------------------------------------ element-wise groups
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(4096, 2048), (64, 10240), (3, 7), (1000, 24)])
@pytest.mark.parametrize("group", ["silu_mul", "gelu_mul", "residual_add"])
def test_fused_group_matches_fused_oracle(ops, oracle, dtype, shape, group):
    r = rng(hash((shape, group)) % 2**32)
    nodes, result = getattr(ops, group + "_nodes")()
    a = from_f32(normal(r, shape), dtype)
    b = from_f32(normal(r, shape), dtype)
    got = ops.elementwise(nodes, result, [a, b])
    want = oracle.elementwise_dag(oracle_nodes(nodes), result, [to_oracle(a), to_oracle(b)], [0, 0], shape,
                                  to_oracle(a).dtype)
    assert_close(got, want, dtype, group)


@pytest.mark.parametrize("dtype", DTYPES)
def test_silu_gate_matches_unfused_reference_chain(ops, oracle, dtype):
    """The fused group against the reference's unfused op chain (each op
    rounds to the tensor dtype), which is what the reference CPU device runs."""
    r = rng(21)
    g = from_f32(normal(r, (64, 5632)), dtype)
    u = from_f32(normal(r, (64, 5632)), dtype)
    nodes, result = ops.silu_mul_nodes()
    got = ops.elementwise(nodes, result, [g, u])
    go, uo = to_oracle(g), to_oracle(u)
    half = np.array(0.5, np.float32) if dtype == torch.float32 else O.f32_to_bf16(np.array(0.5, np.float32))
    one = np.array(1.0, np.float32) if dtype == torch.float32 else O.f32_to_bf16(np.array(1.0, np.float32))
    hx = oracle.binary("mul", half, go)
    t = oracle.unary("tanh", hx)
    op = oracle.binary("add", one, t)
    s = oracle.binary("mul", hx, op)
    want = oracle.binary("mul", s, uo)
    # the unfused chain rounds to bf16 after each of its five ops: a different
    # computation, compared on the tensor scale
    assert_close(got, want, dtype, "silu*up vs unfused chain", floor=1.0)


@pytest.mark.parametrize("dtype", DTYPES)
def test_softcap_group(ops, oracle, dtype):
    r = rng(30)
    x = from_f32(normal(r, (64, 4096), 20.0), dtype)
    nodes, result = ops.softcap_nodes(30.0)
    got = ops.elementwise(nodes, result, [x])
    want = oracle.elementwise_dag(oracle_nodes(nodes), result, [to_oracle(x)], [0], x.shape, to_oracle(x).dtype)
    assert_close(got, want, dtype, "softcap")
    assert float(got.float().abs().max()) <= 30.0


def test_broadcast_scalar_and_strided_inputs(ops, oracle):
    r = rng(31)
    x = from_f32(normal(r, (16, 64)), torch.float32)
    w = from_f32(normal(r, (64,)), torch.float32)           # right-aligned broadcast row
    c = torch.tensor(0.7, dtype=torch.float32, device="cuda")  # scalar
    y = from_f32(normal(r, (64, 16)), torch.float32).t()    # strided (transposed view)
    nodes = [ops.ScalarNode(0, ops.LOAD, 0), ops.ScalarNode(1, ops.LOAD, 1), ops.ScalarNode(2, ops.MUL, operands=(0, 1)),
             ops.ScalarNode(3, ops.LOAD, 2), ops.ScalarNode(4, ops.ADD, operands=(2, 3)),
             ops.ScalarNode(5, ops.LOAD, 3), ops.ScalarNode(6, ops.SUB, operands=(4, 5)),
             ops.ScalarNode(7, ops.EXP, operands=(6,)), ops.ScalarNode(8, ops.RSQRT, operands=(7,)),
             ops.ScalarNode(9, ops.MAX, operands=(8, 0)), ops.ScalarNode(10, ops.NEG, operands=(9,))]
    got = ops.elementwise(nodes, 10, [x, w, c, y], broadcast=[False, True, True, False])
    want = oracle.elementwise_dag(oracle_nodes(nodes), 10,
                                  [to_oracle(x), to_oracle(w), to_oracle(c).reshape(1), to_oracle(y.contiguous())],
                                  [0, 1, 1, 0], (16, 64), np.float32)
    assert_close(got, want, torch.float32, "mixed access modes")


def test_elementwise_rejects_bad_dag(ops):
    from sandyrt_amd._lib import SandyError
    x = torch.zeros(8, device="cuda")
    bad = [ops.ScalarNode(0, ops.LOAD, 0), ops.ScalarNode(1, ops.ADD, operands=(0, 2))]
    with pytest.raises(SandyError, match="dependency order"):
        ops.elementwise(bad, 1, [x])
    with pytest.raises(SandyError, match="invalid input"):
        ops.elementwise([ops.ScalarNode(0, ops.LOAD, 3)], 0, [x])


# ------------------------------------------------------------------ RoPE
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", [
    dict(shape=(1, 32, 4096, 64), split=True, rot=-1),      # C2 q
    dict(shape=(1, 4, 4096, 64), split=True, rot=-1),       # C2 k
    dict(shape=(2, 8, 33, 256), split=True, rot=-1),        # Gemma head dim
    dict(shape=(1, 2, 9, 512), split=True, rot=128),        # partial rotary
    dict(shape=(3, 5, 64), split=False, rot=32),            # interleaved partial
    dict(shape=(2, 7, 10), split=False, rot=-1),            # odd widths -> generic path
    dict(shape=(2, 3, 12), split=True, rot=8),
    dict(shape=(2, 4, 7, 96), split=True, rot=-1),         # 3 pieces per half: half-row kernel
    dict(shape=(2, 2, 9, 80), split=True, rot=48),         # 5 pieces, partial rotary
    dict(shape=(1, 3, 5, 16), split=True, rot=-1),         # one piece per half: 2-lane rows
    dict(shape=(2, 4, 9, 128), split=True, rot=-1),        # 16-lane rows (DPP row mirror exchange)
    dict(shape=(2, 3, 5, 128), split=True, rot=64),        # the same, partial rotary
    dict(shape=(3, 6, 7, 64), split=True, rot=48),         # 8-lane rows (DPP half-row mirror), partial
    dict(shape=(2, 5, 3, 32), split=True, rot=-1),         # 4-lane rows (lane exchange by ds_bpermute)
])
def test_rope(ops, oracle, dtype, case):
    r = rng(hash(tuple(case["shape"])) % 2**32)
    x = from_f32(normal(r, case["shape"]), dtype)
    got = ops.rope(x, 10000.0, rotary_dim=case["rot"], split_half=case["split"])
    want = oracle.rope(to_oracle(x), 10000.0, rotary_dim=case["rot"], split_half=case["split"])
    assert_close(got, want, dtype, f"rope {case}")


@pytest.mark.parametrize("kind", ["offset", "seq", "vectors"])
@pytest.mark.parametrize("dtype", DTYPES)
def test_rope_position_ids(ops, oracle, kind, dtype):
    r = rng(5)
    x = from_f32(normal(r, (2, 4, 6, 64)), dtype)
    n = {"offset": 1, "seq": 6, "vectors": 48}[kind]
    ids = torch.from_numpy(r.integers(0, 4000, n).astype(np.int64)).cuda()
    got = ops.rope(x, 1e4, split_half=True, position_ids=ids)
    want = oracle.rope(to_oracle(x), 1e4, split_half=True, position_ids=ids.cpu().numpy())
    assert_close(got, want, dtype, f"rope ids {kind}")


def test_rope_angles_bit_exact_at_long_positions(ops, oracle):
    """Angles pos / theta^(2i/d) are identical to the CPU (host powf, correctly
    rounded division); remaining error is cos/sin ulp only."""
    x = torch.zeros(1, 1, 8192, 64, device="cuda")
    x[..., :32] = 1.0  # output[p] = cos(angle_p), output[32 + p] = sin(angle_p), every pair
    got = ops.rope(x, 10000.0, split_half=True)
    want = oracle.rope(to_oracle(x), 10000.0, split_half=True)
    np.testing.assert_allclose(got.cpu().numpy(), want, atol=2e-7)


def test_rope_negative_position_sets_device_error(ops):
    from sandyrt_amd._lib import SandyError
    x = torch.zeros(1, 1, 4, device="cuda")
    ops.rope(x, 1e4, position_ids=torch.tensor([-1], device="cuda"))
    with pytest.raises(SandyError, match="rope position_ids must be non-negative"):
        ops.check_device_errors()
    ops.check_device_errors()  # cleared


# ------------------------------------------------------------------ softmax / sum / gather
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape,axis", [((512, 128), -1), ((3, 2048), -1), ((5, 3000), -1), ((2, 7, 3), 1),
                                        ((4, 1), -1), ((6, 50257), -1)])
def test_softmax(ops, oracle, dtype, shape, axis):
    r = rng(sum(shape))
    xf = normal(r, shape, 3.0)
    if shape == (3, 2048):
        xf[1, :] = -np.inf
    x = from_f32(xf, dtype)
    got = ops.softmax(x, axis)
    want = oracle.softmax(to_oracle(x), axis)
    assert_close(got, want, dtype, f"softmax {shape}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_sum_is_bit_exact(ops, oracle, dtype):
    r = rng(8)
    x = from_f32(np.abs(normal(r, (512, 8))), dtype)
    assert_equal(ops.sum(x, -1, True), oracle.sum(to_oracle(x), -1, True), "sum keepdims")
    y = from_f32(normal(r, (4, 6, 5)), dtype)
    assert_equal(ops.sum(y, 1, False), oracle.sum(to_oracle(y), 1, False), "sum middle axis")


@pytest.mark.parametrize("dtype", DTYPES)
def test_embedding_gather(ops, oracle, dtype):
    r = rng(9)
    w = from_f32(normal(r, (128, 2816)), dtype)
    ids = torch.from_numpy(r.integers(0, 128, (512, 8)).astype(np.int32)).cuda()
    assert_equal(ops.embedding(ids, w), oracle.embedding(ids.cpu().numpy(), to_oracle(w)), "embedding")
    w1 = from_f32(normal(r, (128,)), dtype)  # rank-1 table (per-expert scale)
    assert_equal(ops.embedding(ids, w1), oracle.embedding(ids.cpu().numpy(), to_oracle(w1)), "embedding rank 1")


def test_embedding_bad_id_sets_device_error(ops):
    from sandyrt_amd._lib import SandyError
    w = torch.zeros(4, 8, device="cuda")
    ops.embedding(torch.tensor([0, 4], device="cuda"), w)
    with pytest.raises(SandyError, match="embedding id out of range"):
        ops.check_device_errors()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("ids_kind", [None, "offset", "seq"])
def test_rope_pair_matches_two_single_calls(ops, dtype, split, ids_kind):
    """rope_pair(q, k) == rope(q), rope(k) bit for bit: one launch over both
    tensors' heads (per-vector ids: one launch per tensor)."""
    r = rng(17)
    q = from_f32(normal(r, (2, 8, 6, 64)), dtype)
    k = from_f32(normal(r, (2, 2, 6, 64)), dtype)
    ids = {None: None, "offset": torch.tensor([40], device="cuda"),
           "seq": torch.tensor([3, 9, 1, 4000, 7, 0], device="cuda")}[ids_kind]
    qo, ko = ops.rope_pair(q, k, 1e4, split_half=split, position_ids=ids)
    assert torch.equal(qo, ops.rope(q, 1e4, split_half=split, position_ids=ids))
    assert torch.equal(ko, ops.rope(k, 1e4, split_half=split, position_ids=ids))


def test_rope_pair_config2_shapes_and_fallback(ops, oracle):
    """BASELINE config 2's q [1,32,4096,64] and k [1,4,4096,64] in one launch
    against the oracle; unaligned views take the general kernel per tensor,
    and so do per-vector position ids (they differ between q and k)."""
    r = rng(18)
    q = from_f32(normal(r, (1, 32, 4096, 64)), torch.bfloat16)
    k = from_f32(normal(r, (1, 4, 4096, 64)), torch.bfloat16)
    qo, ko = ops.rope_pair(q, k, 1e4, split_half=True)
    assert_close(qo, oracle.rope(to_oracle(q), 1e4, split_half=True), torch.bfloat16, "q")
    assert_close(ko, oracle.rope(to_oracle(k), 1e4, split_half=True), torch.bfloat16, "k")
    qs, ks = q[:, :, 1:], k[:, :, 1:]  # strided views
    qo2, ko2 = ops.rope_pair(qs, ks, 1e4, split_half=True)
    assert torch.equal(qo2, ops.rope(qs, 1e4, split_half=True))
    assert torch.equal(ko2, ops.rope(ks, 1e4, split_half=True))
    # per-vector ids (q and k with equal vector counts): one launch per tensor
    qv, kv = q[:, :4, :5].contiguous(), k[:, :, :5].contiguous()
    ids = torch.arange(20, device="cuda") * 37
    qo3, ko3 = ops.rope_pair(qv, kv, 1e4, split_half=True, position_ids=ids)
    assert torch.equal(qo3, ops.rope(qv, 1e4, split_half=True, position_ids=ids))
    assert torch.equal(ko3, ops.rope(kv, 1e4, split_half=True, position_ids=ids))


def test_rope_pair_rejects_mismatched_tensors(ops):
    from sandyrt_amd._lib import SandyError
    q = torch.zeros(1, 4, 8, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(SandyError, match="must share sequence length and last dimension"):
        ops.rope_pair(q, torch.zeros(1, 2, 8, 32, dtype=torch.bfloat16, device="cuda"), 1e4)
    with pytest.raises(SandyError, match="must have one dtype"):
        ops.rope_pair(q, torch.zeros(1, 2, 8, 64, dtype=torch.float32, device="cuda"), 1e4)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("ids_kind", [None, "offset", "seq"])
@pytest.mark.parametrize("rotary", [-1, 32])
@pytest.mark.parametrize("hd", [64, 128])
def test_rope_from_cache_equals_direct(ops, dtype, ids_kind, rotary, hd):
    """A cos/sin cache built once, applied to q and k: bit-identical to the
    direct rope_pair (same angle, same sin/cos), full and partial rotary."""
    r = rng(19)
    q = from_f32(normal(r, (1, 12, 40, hd)), dtype)
    k = from_f32(normal(r, (1, 2, 40, hd)), dtype)
    ids = {None: None, "offset": torch.tensor([4000], device="cuda"),
           "seq": torch.from_numpy(r.integers(0, 100000, 40)).cuda()}[ids_kind]
    cache = ops.rope_cache(40, hd, 1e4, rotary_dim=rotary, split_half=True, position_ids=ids)
    qc, kc = ops.rope_pair_cached(q, k, cache)
    qd, kd = ops.rope_pair(q, k, 1e4, rotary_dim=rotary, split_half=True, position_ids=ids)
    assert torch.equal(qc, qd) and torch.equal(kc, kd)
    q1, none = ops.rope_pair_cached(q, None, cache)
    assert none is None and torch.equal(q1, qd)


def test_rope_from_cache_config2_against_oracle(ops, oracle):
    r = rng(20)
    q = from_f32(normal(r, (1, 32, 4096, 64)), torch.bfloat16)
    k = from_f32(normal(r, (1, 4, 4096, 64)), torch.bfloat16)
    cache = ops.rope_cache(4096, 64, 1e4, split_half=True)
    qo, ko = ops.rope_pair_cached(q, k, cache)
    assert_close(qo, oracle.rope(to_oracle(q), 1e4, split_half=True), torch.bfloat16, "q from cache")
    assert_close(ko, oracle.rope(to_oracle(k), 1e4, split_half=True), torch.bfloat16, "k from cache")
    # cache angles: (cos, sin) of pos / 10000^(2i/64), against the oracle's rotation of a unit pair
    x = torch.zeros(1, 1, 4096, 64, device="cuda")
    x[..., 0] = 1.0
    want = oracle.rope(to_oracle(x), 1e4, split_half=True)
    np.testing.assert_allclose(cache[:, 0, 0].cpu().numpy(), want[0, 0, :, 0], atol=2e-7)
    np.testing.assert_allclose(cache[:, 0, 1].cpu().numpy(), want[0, 0, :, 32], atol=2e-7)


def test_rope_cache_rejects(ops):
    from sandyrt_amd._lib import SandyError
    with pytest.raises(SandyError, match="rope cache must be"):
        ops.rope_cache(8, 64, 1e4, out=torch.empty(8, 31, 2, device="cuda"))
    cache = ops.rope_cache(8, 48, 1e4)
    q = torch.zeros(1, 2, 8, 48, dtype=torch.bfloat16, device="cuda")  # half 24: not a power-of-two multiple of 8
    with pytest.raises(SandyError, match="rope from a cache takes"):
        ops.rope_pair_cached(q, None, cache)


def test_rope_sin_cos_accuracy(ops):
    """The kernels' sin / cos of the RoPE angle against float64 sin / cos: with
    theta = 1 every pair's angle is the position itself, and rotating the
    pair (1, 0) returns (cos, sin) exactly (x cos - 0 sin, x sin + 0 cos), so
    the output is the sin / cos the kernel computed.  Positions up to 2^20;
    within 1 ulp (2^-23 absolute for values in [-1, 1])."""
    r = rng(12)
    pos = np.concatenate([np.arange(0, 4096), r.integers(0, 1 << 20, 4096)]).astype(np.int64)
    T, D = pos.size, 64
    x = torch.zeros(1, 1, T, D, dtype=torch.float32, device="cuda")
    x[..., : D // 2] = 1.0
    out = ops.rope(x, 1.0, split_half=True, position_ids=torch.from_numpy(pos).cuda()).cpu().numpy()[0, 0]
    ang = pos.astype(np.float32).astype(np.float64)
    c, s = np.cos(ang)[:, None], np.sin(ang)[:, None]
    err = max(np.abs(out[:, : D // 2] - c).max(), np.abs(out[:, D // 2:] - s).max())
    assert err <= 2.0 ** -23, err
