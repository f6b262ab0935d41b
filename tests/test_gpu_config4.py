"""BASELINE config 4 (Gemma-style layer, bf16, seed 3) at its real size:
paged decode over 64 sequences with contexts U[1024, 8192] (Hq 8, Hkv 2,
D 256, scale 1.0, block 16) and the layer's fused groups -- RMSNorm
[64, 2560], GeGLU [64, 10240], the tanh logit soft-cap 30 over [64, 262144]
and the greedy argmax of the capped logits.  The reference fuzzes HD 256
decode over long keys the same way (test/engine/CudaDeviceTest.cpp:
3082-3170); the oracle restates src/core/TensorCalc.cpp."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import assert_close, assert_equal, from_f32, normal, rng, to_oracle

pytestmark = pytest.mark.gpu

B, HQ, HKV, D, PAGE = 64, 8, 2, 256, 16


@pytest.fixture(scope="module")
def ops():
    from sandyrt_amd import ops
    return ops


@pytest.fixture(scope="module")
def decode_inputs():
    r = rng(3)
    ctx = [int(c) for c in r.integers(1024, 8193, B)]
    nblk = [(c + PAGE - 1) // PAGE for c in ctx]
    pool = sum(nblk) + 64
    perm = r.permutation(pool).astype(np.int32)
    table = np.zeros((B, max(nblk)), np.int32)
    off = 0
    for b, n in enumerate(nblk):
        table[b, :n] = perm[off:off + n]
        table[b, n:] = perm[off]  # padding points at a real page
        off += n
    g = torch.Generator(device="cuda").manual_seed(3)
    kpool = torch.randn(pool, HKV, PAGE, D, generator=g, device="cuda").to(torch.bfloat16)
    vpool = torch.randn(pool, HKV, PAGE, D, generator=g, device="cuda").to(torch.bfloat16)
    q = from_f32(normal(r, (B, HQ, 1, D), 0.0625), torch.bfloat16)
    pos = np.array([c - 1 for c in ctx], np.int64)
    return ctx, table, kpool, vpool, q, pos


def oracle_rows(oracle, sel, ctx, table, kpool, vpool, q, pos, scale):
    """The reference CPU device's path for the selected sequences: pages to
    dense K/V (CpuDevice.cpp:611-676), then attention_impl."""
    tk = max(ctx[b] for b in sel)
    kd = np.zeros((len(sel), HKV, tk, D), np.uint16)
    vd = np.zeros_like(kd)
    for i, b in enumerate(sel):
        ids = torch.from_numpy(table[b, :(ctx[b] + PAGE - 1) // PAGE].astype(np.int64)).cuda()
        kp, vp = to_oracle(kpool[ids]), to_oracle(vpool[ids])
        kd[i, :, :ctx[b]] = oracle.paged_to_dense(kp, np.arange(len(ids), dtype=np.int32), HKV, ctx[b], PAGE, D)
        vd[i, :, :ctx[b]] = oracle.paged_to_dense(vp, np.arange(len(ids), dtype=np.int32), HKV, ctx[b], PAGE, D)
    return oracle.attention(to_oracle(q)[sel], kd, vd, pos[sel], 0, scale)


@pytest.mark.parametrize("split", ["", "256"])
def test_config4_paged_decode_full_size(ops, oracle, decode_inputs, monkeypatch, split):
    """All 64 sequences run; the oracle checks five of them, the longest and
    the shortest included.  At 1024- (default) and 256-key splits every
    sequence takes the multi-split merge path (contexts > 1024)."""
    if split:
        monkeypatch.setenv("SANDY_PAGED_SPLIT", split)
    ctx, table, kpool, vpool, q, pos = decode_inputs
    out = ops.paged_attention(q, ops.PagedCache(kpool), ops.PagedCache(vpool), torch.from_numpy(table).cuda(),
                              torch.from_numpy(pos).cuda(), scale=1.0)
    ops.check_device_errors()
    sel = sorted({int(np.argmax(ctx)), int(np.argmin(ctx)), 0, 31, 63})
    assert max(ctx) > 4096
    want = oracle_rows(oracle, sel, ctx, table, kpool, vpool, q, pos, 1.0)
    assert_close(out[sel], want, torch.bfloat16, f"config-4 paged decode rows {sel}")


def test_config4_rms_norm(ops, oracle):
    r = rng(3)
    x = from_f32(normal(r, (B, 2560)), torch.bfloat16)
    w = from_f32(normal(r, (2560,)), torch.bfloat16)
    assert_equal(ops.rms_norm(x, w, 1e-6), oracle.rms_norm(to_oracle(x), to_oracle(w), 1e-6), "config-4 rms_norm")


def test_config4_geglu(ops, oracle):
    r = rng(3)
    g = from_f32(normal(r, (B, 10240)), torch.bfloat16)
    u = from_f32(normal(r, (B, 10240)), torch.bfloat16)
    nodes, result = ops.gelu_mul_nodes()
    onodes = O.make_nodes([(n.id, n.op, n.input_index, n.constant, list(n.operands)) for n in nodes])
    want = oracle.elementwise_dag(onodes, result, [to_oracle(g), to_oracle(u)], [0, 0], (B, 10240), np.uint16)
    assert_close(ops.elementwise(nodes, result, [g, u]), want, torch.bfloat16, "config-4 GeGLU")


def test_config4_softcap_then_greedy_argmax(ops, oracle):
    """tanh(x / 30) * 30 over the [64, 262144] logits, then the greedy token
    of each row (ties to the lowest id), bit-exact against the CPU chain."""
    r = rng(3)
    x = from_f32(normal(r, (B, 262144), 8.0), torch.bfloat16)
    nodes, result = ops.softcap_nodes(30.0)
    onodes = O.make_nodes([(n.id, n.op, n.input_index, n.constant, list(n.operands)) for n in nodes])
    capped = ops.elementwise(nodes, result, [x])
    want = oracle.elementwise_dag(onodes, result, [to_oracle(x)], [0], (B, 262144), np.uint16)
    assert_close(capped, want, torch.bfloat16, "config-4 softcap")
    # argmax of the device's capped logits against the oracle's argmax of the same tensor
    v, i = ops.topk(capped, 1)
    wv, wi = oracle.topk(to_oracle(capped), 1)
    assert_equal(i, wi, "config-4 greedy ids")
    assert_equal(v, wv, "config-4 greedy values")
