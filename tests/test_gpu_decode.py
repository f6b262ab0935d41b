"""GPU parity of the greedy decode step (the reference's TinyLlama eval_token
program, src/models/tinyllama/eval_token.sandy.go and common.sandy.go:1-62)
against the oracle running the same op chain on the CPU: embedding, per block
RMSNorm / q,k,v projections / RoPE / append / attention / o projection /
residual add / RMSNorm / SiLU-gated MLP / residual add, final RMSNorm, lm-head
and greedy argmax.  A reduced model (2 blocks, hidden 256) keeps the CPU chain
to a second; the GPU runs one eager step, then a captured HIP graph replayed.
The oracle is fed the GPU's chosen token each step (teacher forcing), so every
step's logits are compared at the bf16 tolerance; the greedy token is compared
exactly wherever the oracle's top two logits are clearly apart."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import assert_close, from_f32, normal, rng, to_oracle

pytestmark = pytest.mark.gpu


def oracle_nodes(nodes):
    return O.make_nodes([(n.id, n.op, n.input_index, n.constant, list(n.operands)) for n in nodes])


def oracle_step(oracle, cfg, w, kc, vc, token, pos):
    """One decode step of the reference program on the oracle; kc/vc are the
    per-layer dense caches [1, kv_heads, T, D] (uint16 bf16), extended in place."""
    from sandyrt_amd import ops
    hq, hk, D = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim, cfg.head_dim
    pid = np.array([pos], np.int64)
    x = oracle.embedding(np.array([[token]], np.int64), w["embed"]).reshape(1, cfg.hidden)
    silu, sres = ops.silu_mul_nodes()
    for layer in range(cfg.layers):
        h = oracle.rms_norm(x, w[f"{layer}.in_norm"], cfg.eps)
        qkv = oracle.matmul(h, w[f"{layer}.qkv"], transpose_rhs=True)
        q = qkv[:, :hq].reshape(1, cfg.heads, 1, D)
        k = qkv[:, hq:hq + hk].reshape(1, cfg.kv_heads, 1, D)
        v = qkv[:, hq + hk:].reshape(1, cfg.kv_heads, 1, D)
        q = oracle.rope(np.ascontiguousarray(q), cfg.theta, split_half=True, position_ids=pid)
        k = oracle.rope(np.ascontiguousarray(k), cfg.theta, split_half=True, position_ids=pid)
        kc[layer] = np.concatenate([kc[layer], k], axis=2)
        vc[layer] = np.concatenate([vc[layer], np.ascontiguousarray(v)], axis=2)
        ctx = oracle.attention(q, kc[layer], vc[layer], pid, 0, 1.0 / np.sqrt(D))
        o = oracle.matmul(ctx.reshape(1, hq), w[f"{layer}.o"], transpose_rhs=True)
        x = oracle.binary("add", x, o)
        h = oracle.rms_norm(x, w[f"{layer}.post_norm"], cfg.eps)
        gu = oracle.matmul(h, w[f"{layer}.gate_up"], transpose_rhs=True)
        gate, up = np.ascontiguousarray(gu[:, :cfg.ffn]), np.ascontiguousarray(gu[:, cfg.ffn:])
        act = oracle.elementwise_dag(oracle_nodes(silu), sres, [gate, up], [0, 0], gate.shape, gate.dtype)
        d = oracle.matmul(act, w[f"{layer}.down"], transpose_rhs=True)
        x = oracle.binary("add", x, d)
    h = oracle.rms_norm(x, w["norm"], cfg.eps)
    return oracle.matmul(h, w["lm_head"], transpose_rhs=True)


@pytest.mark.parametrize("width", ["reduced", "tinyllama"])
def test_decode_step_eager_and_graph_match_oracle(oracle, width):
    """The decode step's fused kernels (q/k/v GEMM with the RMSNorm prologue
    and the RoPE + append epilogue, o and down GEMMs with the residual
    epilogue, gate/up GEMM with the gated epilogue, lm-head with the final
    norm) against the oracle's unfused op chain: a reduced model (2 blocks,
    hidden 256), and one block at TinyLlama-1.1B's full width (hidden 2048,
    32 q / 4 kv heads, FFN 5632; the vocabulary cut to 1000)."""
    from sandyrt_amd.decode import DecodeConfig, TinyLlamaDecoder, random_weights
    from sandyrt_amd.device import HipDevice
    if width == "reduced":
        cfg = DecodeConfig(layers=2, hidden=256, heads=8, kv_heads=2, head_dim=64, ffn=512, vocab=1000, page_size=32,
                           max_context=128)
    else:
        cfg = DecodeConfig(layers=1, hidden=2048, heads=32, kv_heads=4, head_dim=64, ffn=5632, vocab=1000,
                           page_size=16, max_context=128)
    w = random_weights(cfg, seed=1)
    wn = {k: to_oracle(v) for k, v in w.items()}
    dev = HipDevice(0)
    try:
        dec = TinyLlamaDecoder(dev, cfg, w)
        r = rng(3)
        ctx0 = 37
        ks = [from_f32(normal(r, (1, cfg.kv_heads, ctx0, cfg.head_dim)), torch.bfloat16) for _ in range(cfg.layers)]
        vs = [from_f32(normal(r, (1, cfg.kv_heads, ctx0, cfg.head_dim)), torch.bfloat16) for _ in range(cfg.layers)]
        dec.prefill_cache(ks, vs)
        kc = [to_oracle(k) for k in ks]
        vc = [to_oracle(v) for v in vs]
        token = 5
        dec.set_token(token)
        for step in range(4):
            print(f"decode step {step} ({'eager' if step == 0 else 'graph replay'})", flush=True)
            if step == 0:
                dec.step()
            else:
                if dec.graph is None:
                    dec.capture()
                dec.replay()
            dev.synchronize()
            got_logits = to_oracle(dec.logits)
            got_token = int(dec.token.item())
            want = oracle_step(oracle, cfg, wn, kc, vc, token, ctx0 + step)
            assert_close(got_logits, want, torch.bfloat16, f"logits, step {step}", floor=1.0)  # whole-model chain
            wf = O.to_f32(want).ravel()
            top2 = np.sort(wf)[-2:]
            if top2[1] - top2[0] > 0.05 * float(np.sqrt(np.mean(wf ** 2))):
                assert got_token == int(np.argmax(wf)), f"greedy token, step {step}"
            assert dec.length() == ctx0 + step + 1
            token = got_token
        # the K cache on the device holds the oracle's roped keys for every step
        for layer in range(cfg.layers):
            dev.paged_sync(dec.k_pools[layer])
            got_k = dev.read_paged(dec.k_seq[layer][0], np.uint16)
            assert got_k.shape == kc[layer].shape
            assert_close(got_k, kc[layer], torch.bfloat16, f"K cache layer {layer}", floor=1.0)
        dec.close()
    finally:
        dev.close()


def test_decode_graph_replay_matches_eager_bit_for_bit():
    """Two decoders with the same weights and context: one steps eagerly, the
    other replays one captured step; tokens and logits agree exactly."""
    from sandyrt_amd.decode import DecodeConfig, TinyLlamaDecoder, random_weights
    from sandyrt_amd.device import HipDevice
    cfg = DecodeConfig(layers=3, hidden=512, heads=8, kv_heads=2, head_dim=64, ffn=1024, vocab=2000,
                       max_context=256)
    w = random_weights(cfg, seed=2)
    dev = HipDevice(0)
    try:
        a, b = TinyLlamaDecoder(dev, cfg, w), TinyLlamaDecoder(dev, cfg, w)
        r = rng(4)
        ks = [from_f32(normal(r, (1, cfg.kv_heads, 70, cfg.head_dim)), torch.bfloat16) for _ in range(cfg.layers)]
        vs = [from_f32(normal(r, (1, cfg.kv_heads, 70, cfg.head_dim)), torch.bfloat16) for _ in range(cfg.layers)]
        a.prefill_cache(ks, vs)
        b.prefill_cache(ks, vs)
        a.set_token(11)
        b.set_token(11)
        a.step()
        b.step()  # warm step (workspaces, generated kernels) before capture
        b.capture()
        for step in range(5):
            a.step()
            b.replay()
            dev.synchronize()
            assert torch.equal(a.logits, b.logits), f"step {step}"
            assert torch.equal(a.token, b.token)
        assert a.length() == b.length() == 70 + 6
        a.close()
        b.close()
    finally:
        dev.close()


def test_batched_decode_matches_oracle_per_sequence(oracle):
    """Three sequences with different context lengths decoded together (one
    eager step, then graph replays): each sequence's logits match the
    oracle chain run on that sequence alone, its greedy token matches where
    the top two logits are apart, and each cache grows by one row a step."""
    from sandyrt_amd.decode import DecodeConfig, TinyLlamaDecoder, random_weights
    from sandyrt_amd.device import HipDevice
    cfg = DecodeConfig(layers=2, hidden=256, heads=8, kv_heads=2, head_dim=64, ffn=512, vocab=1000, page_size=16,
                       max_context=160)
    w = random_weights(cfg, seed=5)
    wn = {k: to_oracle(v) for k, v in w.items()}
    ctx0 = [37, 5, 120]
    B = len(ctx0)
    dev = HipDevice(0)
    try:
        dec = TinyLlamaDecoder(dev, cfg, w, batch=B)
        r = rng(6)
        kc, vc = [], []
        for b, n in enumerate(ctx0):
            ks = [from_f32(normal(r, (1, cfg.kv_heads, n, cfg.head_dim)), torch.bfloat16) for _ in range(cfg.layers)]
            vs = [from_f32(normal(r, (1, cfg.kv_heads, n, cfg.head_dim)), torch.bfloat16) for _ in range(cfg.layers)]
            dec.prefill_cache(ks, vs, seq=b)
            kc.append([to_oracle(k) for k in ks])
            vc.append([to_oracle(v) for v in vs])
        tokens = [5, 17, 999]
        dec.set_token(tokens)
        for step in range(3):
            print(f"batched decode step {step} ({'eager' if step == 0 else 'graph replay'})", flush=True)
            if step == 0:
                dec.step()
            else:
                if dec.graph is None:
                    dec.capture()
                dec.replay()
            dev.synchronize()
            got_logits = to_oracle(dec.logits)
            got_tokens = dec.token.view(-1).cpu().tolist()
            for b in range(B):
                want = oracle_step(oracle, cfg, wn, kc[b], vc[b], tokens[b], ctx0[b] + step)
                assert_close(got_logits[b:b + 1], want, torch.bfloat16, f"logits, sequence {b}, step {step}",
                             floor=1.0)  # whole-model chain
                wf = O.to_f32(want).ravel()
                top2 = np.sort(wf)[-2:]
                if top2[1] - top2[0] > 0.05 * float(np.sqrt(np.mean(wf ** 2))):
                    assert got_tokens[b] == int(np.argmax(wf)), f"greedy token, sequence {b}, step {step}"
                assert dec.length(b) == ctx0[b] + step + 1
            tokens = got_tokens
        for b in range(B):
            dev.paged_sync(dec.k_pools[1])
            got_k = dev.read_paged(dec.k_seq[1][b], np.uint16)
            assert_close(got_k, kc[b][1], torch.bfloat16, f"K cache layer 1, sequence {b}", floor=1.0)
        dec.close()
    finally:
        dev.close()


def test_fused_qkv_step_matches_separate_ops_bit_for_bit():
    """The fused launches (RoPE q and k with both appends; the gate/up GEMM
    with the SiLU gate in its epilogue; the residual adds in the o / down GEMM
    epilogues and the RMSNorms in the q/k/v, gate/up and lm-head GEMM
    prologues) and the reference program's separate
    ops give identical logits, tokens and caches, step after step, for a
    batch with ragged contexts."""
    from sandyrt_amd.decode import DecodeConfig, TinyLlamaDecoder, random_weights
    from sandyrt_amd.device import HipDevice
    cfg = DecodeConfig(layers=2, hidden=512, heads=8, kv_heads=2, head_dim=64, ffn=1024, vocab=1500, page_size=16,
                       max_context=128)
    w = random_weights(cfg, seed=8)
    dev = HipDevice(0)
    try:
        a = TinyLlamaDecoder(dev, cfg, w, batch=4, fused_qkv=True, fused_glu=True)
        b = TinyLlamaDecoder(dev, cfg, w, batch=4, fused_qkv=False, fused_glu=False, fused_norm=False)
        r = rng(9)
        for s, n in enumerate([3, 16, 17, 90]):
            ks = [from_f32(normal(r, (1, cfg.kv_heads, n, cfg.head_dim)), torch.bfloat16) for _ in range(cfg.layers)]
            vs = [from_f32(normal(r, (1, cfg.kv_heads, n, cfg.head_dim)), torch.bfloat16) for _ in range(cfg.layers)]
            a.prefill_cache(ks, vs, seq=s)
            b.prefill_cache(ks, vs, seq=s)
        a.set_token([1, 2, 3, 4])
        b.set_token([1, 2, 3, 4])
        for step in range(4):
            a.step()
            b.step()
            dev.synchronize()
            assert torch.equal(a.logits, b.logits), f"step {step}"
            assert torch.equal(a.token, b.token), f"step {step}"
        for layer in range(cfg.layers):
            for s in range(4):
                for pa, pb, sa, sb in ((a.k_pools, b.k_pools, a.k_seq, b.k_seq), (a.v_pools, b.v_pools, a.v_seq, b.v_seq)):
                    dev.paged_sync(pa[layer])
                    dev.paged_sync(pb[layer])
                    assert np.array_equal(dev.read_paged(sa[layer][s], np.uint16), dev.read_paged(sb[layer][s], np.uint16))
        a.close()
        b.close()
    finally:
        dev.close()
